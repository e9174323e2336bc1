"""C ABI of libsas.so: every function include/*.h declares is exported, and
argument validation fails with the documented status codes before any
device work (no GPU needed)."""

from __future__ import annotations

import ctypes as C
import os
import re

import pytest

from dsv4_amd import _lib

INCLUDE = os.path.join(os.path.dirname(__file__), "..", "include")
HEADER = os.path.join(INCLUDE, "sas.h")


def _declared():
    text = "\n".join(open(os.path.join(INCLUDE, f)).read() for f in sorted(os.listdir(INCLUDE)) if f.endswith(".h"))
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(sas_\w+)\s*\(", text, flags=re.M)))


def test_header_declares_the_exported_set():
    assert _declared() == sorted(_lib.EXPORTED)


def test_python_constants_match_the_header():
    text = open(HEADER).read()
    for name in ("SAS_FWD_NO_COMBINE", "SAS_META_SIZE", "SAS_BWD_WINDOW_TOKENS", "SAS_BWD_WINDOW_KEYS"):
        m = re.search(r"^#define\s+%s\s+(\d+)" % name, text, flags=re.M)
        assert m and int(m.group(1)) == getattr(_lib, name), name


@pytest.mark.parametrize("sym", _declared())
def test_symbol_exported(sym):
    assert hasattr(_lib.lib(), sym), f"libsas.so does not export {sym}"


def test_version():
    assert _lib.lib().sas_version().decode().startswith("libsas")


def _valid_args(**over):
    a = _lib.SasFwdArgs()
    a.T, a.B, a.H, a.D, a.DV = 4, 1, 64, 576, 512
    a.ori_block_size, a.ori_bt_stride, a.ori_num_blocks = 64, 8, 8
    a.cmp_block_size, a.cmp_bt_stride, a.cmp_num_blocks = 64, 2, 2
    a.K, a.scenario, a.q_dtype, a.kv_dtype = 64, _lib.SAS_SCFA, _lib.SAS_DT_BF16, _lib.SAS_DT_BF16
    a.cmp_ratio, a.win_left, a.softmax_scale = 4, 127, 0.0417
    for k, v in over.items():
        setattr(a, k, v)
    return a


def _plan(a):
    ns, ws = C.c_int32(-1), C.c_size_t(0)
    rc = _lib.lib().sas_fwd_plan(C.byref(a), C.byref(ns), C.byref(ws))
    return rc, ns.value, ws.value


def test_plan_valid():
    rc, ns, ws = _plan(_valid_args())
    assert rc == _lib.SAS_OK
    assert ns >= 1
    assert ws == (0 if ns == 1 else 4 * ns * 64 * (512 * 2 + 4 * 4))   # fp16 part_o + (m, l, e, e)


# The planner at the benchmark shapes, on the 256-CU, 8-XCD MI355X (the CU
# count it assumes when no device answers, as here): every XCD's share of
# workgroups, ceil(T / 8) tokens x head groups x splits, fits its 32 CUs.
@pytest.mark.parametrize("T,H,K,fp8,want", [
    (1, 16, 64, False, 4),       # C1: 192 slots, 16-head groups, 4 splits of 48 (exact schedule)
    (32, 64, 512, False, 4),     # C2: 32-head groups: 4 tokens x 2 groups x 4 splits per XCD
    (31, 128, 1024, False, 4),   # C4: 64-head groups: 4 tokens x 2 groups x 4 splits per XCD
    (8, 128, 1024, True, 6),     # C5: fp8 rows, 32-head groups, 6 splits (8 fit one round, 6 take
                                 # as many 32-row steps: the fewest such)
    (4096, 64, 512, False, 1),   # C3: prefill, one split
], ids=["C1", "C2", "C4", "C5", "C3"])
def test_plan_at_benchmark_shapes(T, H, K, fp8, want):
    kvd = _lib.SAS_DT_FP8_E4M3_ROW656 if fp8 else _lib.SAS_DT_BF16
    rc, ns, ws = _plan(_valid_args(T=T, H=H, K=K, kv_dtype=kvd))
    assert rc == _lib.SAS_OK and ns == want
    assert ws == (0 if ns == 1 else T * ns * H * (512 * 2 + 16))


def test_plan_explicit_splits_and_workspace():
    rc, ns, ws = _plan(_valid_args(num_splits=3))
    assert rc == _lib.SAS_OK and ns == 3
    assert ws == 4 * 3 * 64 * (512 * 2 + 16)


@pytest.mark.parametrize("field,value,needle", [
    ("D", 128, "D must be 512 or 576"),
    ("DV", 256, "DV must be 512"),
    ("H", 40, "multiple of 16"),
    ("scenario", 7, "scenario"),
    ("win_left", -1, "win_left"),
    ("head_waves", 3, "head_waves"),
    ("flags", 0x10, "flags"),
])
def test_plan_rejects(field, value, needle):
    rc, _, _ = _plan(_valid_args(**{field: value}))
    assert rc == _lib.SAS_EINVAL
    assert needle in _lib.lib().sas_last_error().decode()


def test_fwd_rejects_null_pointers_without_device_work():
    rc = _lib.lib().sas_fwd_v1(C.byref(_valid_args()), None)
    assert rc == _lib.SAS_EINVAL
    assert "null device pointer" in _lib.lib().sas_last_error().decode()


def test_fwd_empty_batch_is_a_no_op():
    assert _lib.lib().sas_fwd_v1(C.byref(_valid_args(T=0)), None) == _lib.SAS_OK
    assert _lib.lib().sas_last_error().decode() == ""


def test_fwd_missing_workspace():
    a = _valid_args(num_splits=2)
    fake = 1 << 40  # never dereferenced: validation fails first
    for f in ("q", "ori_kv", "ori_block_table", "cmp_kv", "cmp_block_table", "cmp_indices",
              "q_prefix", "act_q", "act_kv", "sinks", "out", "lse"):
        setattr(a, f, fake)
    assert _lib.lib().sas_fwd_v1(C.byref(a), None) == _lib.SAS_ENOWS
    assert "workspace" in _lib.lib().sas_last_error().decode()


def test_combine_rejects():
    ca = _lib.SasCombineArgs()
    assert _lib.lib().sas_combine_v1(C.byref(ca), None) == _lib.SAS_EINVAL
    fake = 1 << 40
    ca.part_o = ca.part_ml = ca.sinks = ca.out = ca.lse = fake
    ca.T, ca.S, ca.H, ca.DV, ca.out_dtype = 1, (1 << 16) + 1, 64, 512, _lib.SAS_DT_BF16
    assert _lib.lib().sas_combine_v1(C.byref(ca), None) == _lib.SAS_EINVAL
    assert "S must be" in _lib.lib().sas_last_error().decode()


def test_check_maps_status_to_exceptions():
    _lib.lib().sas_fwd_plan(C.byref(_valid_args(D=1)), None, None)
    with pytest.raises(ValueError, match="D must be"):
        _lib.check(_lib.SAS_EINVAL, "x")
    with pytest.raises(RuntimeError):
        _lib.check(_lib.SAS_ELAUNCH, "x")


def test_plan_long_rows_take_more_than_64_splits():
    """A token's key slots beyond 64 splits of 1280 (long CFA rows, wide
    windows) plan more splits; only beyond 2^16 splits is the call refused."""
    rc, ns, ws = _plan(_valid_args(scenario=_lib.SAS_CFA, K=200000))
    assert rc == _lib.SAS_OK and ns >= (200000 + 128 + 1279) // 1280
    rc, ns, _ = _plan(_valid_args(scenario=_lib.SAS_SWA, K=0, win_left=20000))
    assert rc == _lib.SAS_OK and ns >= 1
    rc, _, _ = _plan(_valid_args(scenario=_lib.SAS_CFA, K=(1 << 16) * 1280))
    assert rc == _lib.SAS_EINVAL


def test_bwd_rejects_both_window_modes_and_fwd_rejects_bwd_flags():
    """sas_bwd_v1 takes one of the two window-gradient modes, never both
    (refused before any device work); the forward refuses the backward's
    flags."""
    fake = 1 << 40  # never dereferenced: validation fails first
    a = _valid_args(flags=_lib.SAS_BWD_WINDOW_TOKENS | _lib.SAS_BWD_WINDOW_KEYS)
    for f in ("q", "ori_kv", "ori_block_table", "cmp_kv", "cmp_block_table", "cmp_indices",
              "q_prefix", "act_q", "act_kv", "sinks", "out", "lse"):
        setattr(a, f, fake)
    ba = _lib.SasBwdArgs(fwd=a, dout=fake, dq=fake, d_ori_kv=fake, d_cmp_kv=fake, d_sinks=fake)
    assert _lib.lib().sas_bwd_v1(C.byref(ba), None) == _lib.SAS_EINVAL
    assert "together" in _lib.lib().sas_last_error().decode()
    for fl in (_lib.SAS_BWD_WINDOW_TOKENS, _lib.SAS_BWD_WINDOW_KEYS):
        rc, _, _ = _plan(_valid_args(flags=fl))
        assert rc == _lib.SAS_EINVAL and "flags" in _lib.lib().sas_last_error().decode()
