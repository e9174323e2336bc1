"""sas_fwd_noalloc_v1: the forward with its split partials in the library's
own 16 MiB device array instead of a caller workspace. Through the C ABI,
against sas_fwd_v1 (same plan, same kernels: bit for bit), on calls in a
row whose second input is smaller (the array keeps the previous call's
contents), and the host-side rejection of a plan beyond the array."""

from __future__ import annotations

import ctypes as C

import pytest
import torch

from dsv4_amd import _lib, cases

SCRATCH_BYTES = 16 << 20


def _args_for(name):
    from dsv4_amd.api import prepare_sparse_attn_sharedkv
    inp = cases.make_inputs(cases.CONFIGS[name], device="cuda")
    call = prepare_sparse_attn_sharedkv(inp.q, **inp.api_kwargs())
    return inp, call


def _noalloc(call):
    """sas_fwd_noalloc_v1 on the prepared call's inputs, into fresh outputs
    filled with NaN (every element must be written)."""
    a = _lib.SasFwdArgs.from_buffer_copy(call.args)
    out = torch.full_like(call.out, float("nan"))
    lse = torch.full_like(call.lse, float("nan"))
    a.out, a.lse = out.data_ptr(), lse.data_ptr()
    a.workspace, a.workspace_bytes, a.flags = None, 0, 0
    st = torch.cuda.current_stream().cuda_stream
    _lib.check(_lib.lib().sas_fwd_noalloc_v1(C.byref(a), C.c_void_p(st)), "sas_fwd_noalloc_v1")
    return out, lse


@pytest.mark.gpu
def test_noalloc_matches_workspace_entry_point_on_calls_in_a_row():
    runs = []
    for name in ("C2", "C1", "C2"):      # large partials, then a smaller call over stale contents
        print(f"[noalloc] {name}", flush=True)
        inp, call = _args_for(name)
        ns = C.c_int32(0)
        ws = C.c_size_t(0)
        _lib.check(_lib.lib().sas_fwd_plan(C.byref(call.args), C.byref(ns), C.byref(ws)), "plan")
        assert ns.value > 1 and 0 < ws.value <= SCRATCH_BYTES, (name, ns.value, ws.value)
        call.launch()
        out, lse = _noalloc(call)
        torch.cuda.synchronize()
        assert torch.equal(out, call.out), f"{name}: out differs from sas_fwd_v1"
        assert torch.equal(lse, call.lse), f"{name}: lse differs from sas_fwd_v1"
        runs.append((name, ns.value, ws.value))
    print(f"[noalloc] (config, splits, partial bytes): {runs}", flush=True)


def test_noalloc_rejects_plans_beyond_its_array():
    """Checked on the host before any device call: a plan whose partials
    exceed the array fails with SAS_ENOWS and says so; SAS_FWD_NO_COMBINE
    (partials left in the library's array) is refused."""
    L = _lib.lib()
    a = _lib.SasFwdArgs()
    fake = 1 << 20
    for f in ("q", "ori_kv", "ori_block_table", "cmp_kv", "cmp_block_table", "cmp_indices", "q_prefix",
              "act_q", "act_kv", "sinks", "out", "lse"):
        setattr(a, f, fake)
    a.T, a.B, a.H, a.D, a.DV = 4096, 1, 128, 576, 512
    a.ori_block_size, a.ori_bt_stride, a.ori_num_blocks = 64, 64, 64
    a.cmp_block_size, a.cmp_bt_stride, a.cmp_num_blocks = 64, 16, 16
    a.K, a.scenario, a.q_dtype, a.kv_dtype, a.cmp_ratio, a.win_left = 512, 3, 0, 0, 4, 127
    a.softmax_scale, a.num_splits = 0.04, 4
    ns = C.c_int32(0)
    ws = C.c_size_t(0)
    assert L.sas_fwd_plan(C.byref(a), C.byref(ns), C.byref(ws)) == _lib.SAS_OK
    assert ws.value > SCRATCH_BYTES
    assert L.sas_fwd_noalloc_v1(C.byref(a), None) == _lib.SAS_ENOWS
    msg = L.sas_last_error().decode()
    assert "scratch" in msg and str(SCRATCH_BYTES) in msg, msg
    a.num_splits, a.flags = 2, _lib.SAS_FWD_NO_COMBINE
    assert L.sas_fwd_noalloc_v1(C.byref(a), None) == _lib.SAS_EINVAL
    assert "NO_COMBINE" in L.sas_last_error().decode()
