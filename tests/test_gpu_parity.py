"""GPU parity: libsas (through its C ABI, via the drop-in API) against the
CPU oracle on identical seeded inputs.

Tolerances (BASELINE): output atol = rtol = 2e-2 in the query dtype; LSE
absolute 1e-3. The reference suite's own criterion (>= 99.5 % of elements
within bf16 rtol 2^-7 / atol 1e-4, worst normalised error < 10;
test_sparse_attn_sharedkv.py:394-481) is applied to its six scenarios, whose
U(-10,10) data gives LSE values in the hundreds; there the LSE bound is the
reference's (rtol 0.015, atol 0.005 for bf16).
"""

from __future__ import annotations

import ctypes as C
import functools
import math

import numpy as np
import pytest
import torch

from dsv4_amd import _lib, cases, paged
from dsv4_amd.api import prepare_sparse_attn_sharedkv, sparse_attn_sharedkv
from oracle import golden_ref as O

pytestmark = pytest.mark.gpu

OUT_TOL = 2e-2
LSE_ATOL = 1e-3
# elements beyond 2e-2 of golden: at most FAR_MUL x golden's own count
# against its fp64-score twin + FAR_ADD (the twin count itself moves with
# the host's fp32 summation order: 1 to 3 of 33.5 M on the reference's
# scfa_prefill@1024)
FAR_MUL, FAR_ADD = 2, 8


def _oracle(inp: cases.Inputs, tokens=None, exact=False, scores_fp64=False):
    c = inp.cfg
    return O.golden_paged(
        inp.q, ori_kv=inp.ori_kv, ori_block_table=inp.ori_bt, cu_seqlens_q=inp.cu_seqlens_q,
        seqused_kv=inp.seqused_kv, sinks=inp.sinks, softmax_scale=c.scale,
        cmp_kv=inp.cmp_kv if c.scenario >= 2 else None,
        cmp_block_table=inp.cmp_bt if c.scenario >= 2 else None,
        cmp_sparse_indices=inp.cmp_idx if c.scenario == 3 else None,
        cmp_ratio=c.cmp_ratio, ori_win_left=c.win_left, dv=512,
        dequant=paged.dequantize_kv_fp8 if c.fp8 else None, tokens=tokens, exact=exact,
        scores_fp64=scores_fp64)


def _run(inp: cases.Inputs, num_splits=0, **kw):
    d = inp.to("cuda")
    args = d.api_kwargs()
    args.update(kw)
    call = prepare_sparse_attn_sharedkv(d.q, num_splits=num_splits, **args)
    call.launch()
    torch.cuda.synchronize()
    return call.out.cpu(), call.lse.cpu(), call.num_splits


def _check_baseline(out, lse, ref_out, ref_lse, name, tokens=None):
    if tokens is not None:
        out, lse, ref_out, ref_lse = out[tokens], lse[tokens], ref_out[tokens], ref_lse[tokens]
    assert torch.isfinite(out.float()).all(), f"{name}: non-finite output"
    torch.testing.assert_close(out.float(), ref_out.float(), atol=OUT_TOL, rtol=OUT_TOL,
                               msg=lambda m: f"{name} out: {m}")
    torch.testing.assert_close(lse, ref_lse, atol=LSE_ATOL, rtol=0.0,
                               msg=lambda m: f"{name} lse: {m}")


def _reference_rule(real, expt, rtol, atol):
    """test_sparse_attn_sharedkv.py:394-437 (and :440-481 for LSE): percent of
    elements within (rtol, atol) and the worst normalised error among the rest."""
    real = real.float().numpy().ravel()
    expt = expt.float().numpy().ravel()
    ok = np.isclose(real, expt, rtol=rtol, atol=atol, equal_nan=True)
    n_err = int((~ok).sum())
    pct = (real.size - n_err) / real.size * 100.0
    floor = (1.0 / (1 << 14)) / 0.005
    b = np.maximum(np.maximum(np.abs(real), np.abs(expt)), floor) + 1e-9
    rel = np.abs(real - expt) / b
    worst = float(rel[~ok].max()) if n_err else 0.0
    return pct, worst, n_err


def _check_reference_rule(real, expt, rtol, atol, what):
    pct, worst, n_err = _reference_rule(real, expt, rtol, atol)
    assert pct >= 99.5, f"{what}: only {pct:.3f}% within tolerance ({n_err} failing)"
    assert worst < 10.0, f"{what}: worst normalised error {worst:.3f}"


@functools.lru_cache(maxsize=None)
def _inputs(name):
    print(f"[parity] building {name}", flush=True)
    if name in cases.CONFIGS:
        return cases.make_inputs(cases.CONFIGS[name], device="cuda")
    base, _, s1 = name.partition("@")
    return cases.make_inputs(cases.shrink(cases.CONFIGS[base], int(s1)), device="cuda")


# ---------------------------------------------------------------------------
# the five measured workloads, full size
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("name", ["C1", "C2", "C4", "C5"])
def test_decode_configs_full(name):
    inp = _inputs(name)
    out, lse, ns = _run(inp)
    print(f"[parity] {name}: T={inp.T} splits={ns}", flush=True)
    ref_out, ref_lse = _oracle(inp)
    _check_baseline(out, lse, ref_out, ref_lse, name)


def test_prefill_4k_full():
    """C3: 4096-token causal prefill, every token checked."""
    inp = _inputs("C3")
    out, lse, ns = _run(inp)
    ref_out, ref_lse = _oracle(inp)
    _check_baseline(out, lse, ref_out, ref_lse, "C3")


@pytest.mark.parametrize("splits", [1, 2, 3, 7, 20])
def test_split_count_does_not_change_result(splits):
    """Any KV split count gives the no-split result (LSE merge invariant)."""
    inp = _inputs("C2")
    out1, lse1, ns1 = _run(inp, num_splits=1)
    assert ns1 == 1
    outn, lsen, nsn = _run(inp, num_splits=splits)
    torch.testing.assert_close(outn.float(), out1.float(), atol=1e-2, rtol=1e-2)
    torch.testing.assert_close(lsen, lse1, atol=2e-5, rtol=0.0)


def test_split_kernel_then_combine_entry_point():
    """SAS_FWD_NO_COMBINE leaves the partials; sas_combine_v1 on them gives
    the fused call's result bit for bit."""
    d = _inputs("C2")
    call = prepare_sparse_attn_sharedkv(d.q, num_splits=4, **d.api_kwargs())
    assert call.num_splits == 4
    call.launch()
    torch.cuda.synchronize()
    out_f, lse_f = call.out.clone(), call.lse.clone()
    call.out.zero_()
    call.lse.zero_()
    call.launch_split()
    torch.cuda.synchronize()
    assert float(call.lse.abs().max()) == 0.0, "split-only launch must not write lse"
    call.launch_combine()
    torch.cuda.synchronize()
    assert torch.equal(call.out, out_f)
    assert torch.equal(call.lse, lse_f)


@pytest.mark.parametrize("hw", [1, 2, 4])
def test_head_grouping_does_not_change_result(hw):
    """Heads per workgroup (16 x head_waves) only changes the work split."""
    inp = _inputs("C2")
    ref_out, ref_lse = _oracle(inp)
    out, lse, _ = _run(inp, head_waves=hw)
    _check_baseline(out, lse, ref_out, ref_lse, f"C2 hw{hw}")


@pytest.mark.parametrize("hw,waves", [(2, 4), (2, 8), (4, 4), (4, 8)])
def test_wave_layout_does_not_change_result(hw, waves):
    """4 or 8 waves per workgroup (with 8, each 16-head pair of waves splits
    the QK^T channels and the O channels) only changes the work split."""
    inp = _inputs("C2")
    ref_out, ref_lse = _oracle(inp)
    out, lse, _ = _run(inp, head_waves=hw, waves=waves)
    _check_baseline(out, lse, ref_out, ref_lse, f"C2 hw{hw} waves{waves}")


@pytest.mark.parametrize("splits", [1, 2, 3, 5, 9])
def test_two_key_group_pipeline_ragged_rows(splits):
    """32-head, 8-wave workgroups (two key-groups of 16-row steps, the
    batched-decode loop) on 1 to a few hundred rows per workgroup: key-groups
    of unequal step counts, an empty second key-group, partial last steps,
    one-step and two-step key-groups."""
    inp = _small(B=4, H=64, q_lens=[1, 3, 2, 5], kv_lens=[1, 40, 700, 3000], K=200)
    out, lse, ns = _run(inp, num_splits=splits, head_waves=2, waves=8)
    ref_out, ref_lse = _oracle(inp)
    _check_baseline(out, lse, ref_out, ref_lse, f"hw2 waves8 splits {splits}->{ns}")


@pytest.mark.parametrize("hw,waves", [(1, 4), (2, 4), (4, 4), (2, 8), (4, 8)])
@pytest.mark.parametrize("splits", [1, 2, 3, 5, 9])
def test_fp8_rows_every_layout_few_and_many_keys(hw, waves, splits):
    """fp8 rows against golden on the fp32-dequantised cache (the stated
    comparison), through every workgroup layout: 16, 32 and 64 heads, 4
    waves, and 8 waves whose 16-head pairs split the QK^T channels along the
    128-channel scale groups (32-head groups: two key-groups of 16-row steps,
    all waves taking every step's S exchange; 64-head groups: one key-group
    of 32-row steps). Tokens of 1 to 40 keys (token 0 has one) show any
    rounding of the scaled K in the LSE, which averages out over long rows:
    rounding e4m3 x scale to bf16 before QK^T put 17 LSEs of this input
    beyond 1e-3 (worst 2.2e-3 on the one-key token)."""
    inp = _small(B=4, H=128, q_lens=[1, 3, 2, 5], kv_lens=[1, 40, 700, 3000], K=200, fp8=True)
    out, lse, ns = _run(inp, num_splits=splits, head_waves=hw, waves=waves)
    ref_out, ref_lse = _oracle(inp)
    _check_baseline(out, lse, ref_out, ref_lse, f"fp8 hw{hw} waves{waves} splits {splits}->{ns}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
@pytest.mark.parametrize("hw,waves", [(1, 4), (1, 8), (2, 4), (2, 8), (4, 4), (4, 8)])
@pytest.mark.parametrize("splits", [1, 3])
def test_few_keys_every_layout(dtype, hw, waves, splits):
    """Caches in the query dtype, tokens of 1 to 40 keys beside long rows,
    through every workgroup layout (16 heads with 4 waves: the exact or
    streaming schedule; with 8: the register-streamed decode kernel; 32 and
    64 heads with 4 and 8 waves): the LSE of a one-key token is that key's
    score merged with the sink, so any error in S shows undiluted."""
    inp = _small(B=4, H=128, q_lens=[1, 3, 2, 5], kv_lens=[1, 40, 700, 3000], K=200, dtype=dtype)
    out, lse, ns = _run(inp, num_splits=splits, head_waves=hw, waves=waves)
    ref_out, ref_lse = _oracle(inp)
    _check_baseline(out, lse, ref_out, ref_lse, f"{dtype} hw{hw} waves{waves} splits {splits}->{ns}")


# ---------------------------------------------------------------------------
# the reference suite's scenarios (same data as its _build_case)
# ---------------------------------------------------------------------------

REF_CASES = [("scfa_decode", None), ("swa_decode", None), ("cfa_decode", None),
             ("scfa_prefill", 1024), ("swa_prefill", 1024), ("cfa_prefill", 1024)]


# The reference rule (>= 99.5 % of elements within bf16 rtol 2^-7) measures
# agreement with golden's own rounding of p to the query dtype, which golden
# does relative to the running max after each 512-row tile
# (golden.py:156-196). Window-only calls run the exact-window schedule (p
# rounded against the window's final max, golden's one tile), so swa_decode
# reproduces golden's rounding; the compressed scenarios round against each
# KV split's own reference max and meet the rule with margin.


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
@pytest.mark.parametrize("name,s1", REF_CASES, ids=[f"{n}{'@' + str(s) if s else ''}" for n, s in REF_CASES])
def test_reference_scenarios(name, s1, dtype):
    inp = cases.ref_case(name, dtype=dtype, s1=s1)
    out, lse, ns = _run(inp)
    ref_out, ref_lse = _oracle(inp)
    ex_out, ex_lse = _oracle(inp, exact=True)
    # accuracy against the fp64 exact result: no worse than golden's
    e_ours = float((out.double() - ex_out).abs().mean())
    e_gold = float((ref_out.double() - ex_out).abs().mean())
    print(f"[parity] {name} {dtype}: splits={ns} mean|err| vs fp64: ours {e_ours:.4g} "
          f"golden {e_gold:.4g}", flush=True)
    assert e_ours <= 1.10 * e_gold + 1e-6, f"{name}: less accurate than golden"
    torch.testing.assert_close(lse.double(), ex_lse, atol=1e-5, rtol=2e-6)
    # The BASELINE tolerance on every element: LSE within 1e-3 of golden; the
    # output within atol = rtol = 2e-2 of golden's formula evaluated in fp64.
    # On this U(-10,10) data golden's own output moves by more than 2e-2 at
    # cancellation points when only its fp32 score summation order changes
    # (tests/test_oracle.py::test_golden_depends_on_score_summation_order_*),
    # so two correct implementations can differ by that much; golden itself
    # meets the bound against the fp64 result, and so must the kernel.
    torch.testing.assert_close(lse, ref_lse, atol=LSE_ATOL, rtol=0.0,
                               msg=lambda m: f"{name} lse vs golden: {m}")
    _check_baseline(out, lse, ex_out, ex_lse.float(), f"{name} {dtype} vs fp64")
    # Elements beyond 2e-2 of golden itself: bounded by golden's own count
    # against its twin that sums q k^T in fp64 (same fp32 walk otherwise),
    # so a regression toward golden's cancellation points fails here
    # instead of only being printed.
    far = int(((out.float() - ref_out.float()).abs() > OUT_TOL + OUT_TOL * ref_out.float().abs()).sum())
    twin_out, _ = _oracle(inp, scores_fp64=True)
    far_twin = int(((twin_out.float() - ref_out.float()).abs() > OUT_TOL + OUT_TOL * ref_out.float().abs()).sum())
    print(f"[parity] {name}: {far} of {out.numel()} elements beyond 2e-2 of golden (golden's fp64-score "
          f"twin: {far_twin})", flush=True)
    assert far <= FAR_MUL * far_twin + FAR_ADD, f"{name}: {far} elements beyond 2e-2 of golden (twin: {far_twin})"
    if dtype == torch.bfloat16:
        rules = [(out, ref_out, 0.0078125, 1e-4, "out"), (lse, ref_lse, 0.015, 0.005, "lse")]
    else:
        rules = [(out, ref_out, 0.005, 2.5e-5, "out"), (lse, ref_lse, 0.01, 0.001, "lse")]
    for real, expt, rt, at, what in rules:
        pct, worst, n_err = _reference_rule(real, expt, rt, at)
        print(f"[parity] {name} {what}: {pct:.3f}% within, worst {worst:.3f}", flush=True)
        _check_reference_rule(real, expt, rt, at, f"{name} {what}")


REF_8K = [(n, d) for n in ("scfa_prefill", "swa_prefill", "cfa_prefill")
          for d in (torch.bfloat16, torch.float16)]


@pytest.mark.parametrize("name,dtype", REF_8K, ids=[f"{n}-{'bf16' if d == torch.bfloat16 else 'fp16'}"
                                                    for n, d in REF_8K])
def test_reference_scenario_8k_prefill(name, dtype):
    """The reference suite's prefill scenarios at their full 8192 tokens
    (test_sparse_attn_sharedkv.py:105-109, 151-155, 197-201; bf16 and fp16
    as its e2e runs, :586-605), every token checked against the oracle:
    the reference's rule for the dtype and the LSE within 1e-3."""
    inp = cases.ref_case(name, dtype=dtype)
    out, lse, _ = _run(inp)
    ref_out, ref_lse = _oracle(inp)
    if dtype == torch.bfloat16:
        rules = [(out, ref_out, 0.0078125, 1e-4, "out"), (lse, ref_lse, 0.015, 0.005, "lse")]
    else:
        rules = [(out, ref_out, 0.005, 2.5e-5, "out"), (lse, ref_lse, 0.01, 0.001, "lse")]
    for real, expt, rt, at, what in rules:
        pct, worst, n_err = _reference_rule(real, expt, rt, at)
        print(f"[parity] {name} 8K {dtype} {what}: {pct:.3f}% within, worst {worst:.3f}", flush=True)
        _check_reference_rule(real, expt, rt, at, f"{name} {what}")
    torch.testing.assert_close(lse, ref_lse, atol=LSE_ATOL, rtol=0.0, msg=lambda m: f"{name} lse: {m}")


def test_api_return_type():
    """return_softmax_lse switches between a tensor and an (out, lse) pair with
    identical output (test_sparse_attn_sharedkv.py:608-715)."""
    inp = cases.ref_case("swa_decode").to("cuda")
    kw = inp.api_kwargs()
    one = sparse_attn_sharedkv(inp.q, return_softmax_lse=False, **kw)
    two = sparse_attn_sharedkv(inp.q, return_softmax_lse=True, **kw)
    torch.cuda.synchronize()
    assert isinstance(one, torch.Tensor)
    assert isinstance(two, tuple) and len(two) == 2
    out, lse = two
    assert one.shape == (1, 64, 512) and one.dtype == torch.bfloat16
    assert lse.shape == (1, 64) and lse.dtype == torch.float32
    torch.testing.assert_close(out.cpu(), one.cpu())


def test_api_host_and_device_offsets_agree():
    """cu_seqlens_q / seqused_kv given on the host (pinned non-blocking
    copies) or on the device (offsets derived there, no host sync) give the
    same bits; the C4 ragged batch exercises non-trivial q offsets."""
    inp = cases.make_inputs(cases.CONFIGS["C4"], device="cpu")
    d = inp.to("cuda")
    kw = d.api_kwargs()
    kw.update(cu_seqlens_q=inp.cu_seqlens_q.cuda(), seqused_kv=inp.seqused_kv.cuda())
    dev_out, dev_lse = sparse_attn_sharedkv(d.q, return_softmax_lse=True, **kw)
    kw.update(cu_seqlens_q=inp.cu_seqlens_q.cpu(), seqused_kv=inp.seqused_kv.cpu())
    host_out, host_lse = sparse_attn_sharedkv(d.q, return_softmax_lse=True, **kw)
    torch.cuda.synchronize()
    assert torch.equal(dev_out.cpu(), host_out.cpu()) and torch.equal(dev_lse.cpu(), host_lse.cpu())
    ref_out, ref_lse = _oracle(inp)
    torch.testing.assert_close(dev_out.cpu().float(), ref_out.float(), atol=OUT_TOL, rtol=OUT_TOL)
    torch.testing.assert_close(dev_lse.cpu(), ref_lse, atol=LSE_ATOL, rtol=0)


def test_prepared_call_on_another_stream_and_metadata():
    """A prepared call launched on a stream other than the one it was
    prepared on (its device-side offsets are ordered first) gives the
    one-shot result; metadata() is the scheduler's bit-exact output."""
    from dsv4_amd.api import prepare_sparse_attn_sharedkv
    from dsv4_amd.metadata import sparse_attn_sharedkv_metadata
    inp = cases.make_inputs(cases.CONFIGS["C2"], device="cpu")
    d = inp.to("cuda")
    kw = d.api_kwargs()
    kw.update(cu_seqlens_q=inp.cu_seqlens_q.cuda(), seqused_kv=inp.seqused_kv.cuda())
    ref = sparse_attn_sharedkv(d.q, **kw)
    call = prepare_sparse_attn_sharedkv(d.q, **kw)
    side = torch.cuda.Stream()
    call.launch(side)
    side.synchronize()
    torch.cuda.synchronize()
    assert torch.equal(call.out.cpu(), ref.cpu())
    meta = sparse_attn_sharedkv_metadata(
        num_heads_q=64, num_heads_kv=1, head_dim=576, cu_seqlens_q=inp.cu_seqlens_q,
        seqused_kv=inp.seqused_kv, batch_size=len(inp.q_lens), max_seqlen_q=1,
        max_seqlen_kv=int(inp.seqused_kv.max()), ori_mask_mode=4, ori_win_left=127, ori_win_right=0,
        layout_q="TND", layout_kv="PA_ND", has_ori_kv=True, has_cmp_kv=True, aic_core_num=24,
        cmp_ratio=4, cmp_mask_mode=3, cmp_topk=512)
    assert torch.equal(call.metadata().cpu(), meta.cpu())


# ---------------------------------------------------------------------------
# edge cases
# ---------------------------------------------------------------------------

def _small(B, H, q_lens, kv_lens, K, ratio=4, bs=64, D=576, scenario=3, fp8=False, seed=0,
           dtype=torch.bfloat16, win=127, idx_fn=None):
    g = torch.Generator().manual_seed(seed)
    T = sum(q_lens)
    q = torch.randn(T, H, D, generator=g).to(dtype)
    ori_bt, ori_nb = paged.random_block_table(kv_lens, bs, g, extra_blocks=3)
    ori = torch.randn(ori_nb, bs, 1, D, generator=g).to(dtype)
    cmp_lens = [k // ratio for k in kv_lens]
    cmp_bt, cmp_nb = paged.random_block_table(cmp_lens, bs, g, extra_blocks=2)
    cmp_ = torch.randn(cmp_nb, bs, 1, D, generator=g).to(dtype)
    idx = cases.topk_indices(q_lens, kv_lens, K, ratio, g) if K else None
    if idx_fn is not None:
        idx = idx_fn(idx)
    if fp8:
        ori, cmp_ = paged.quantize_kv_fp8(ori.float()), paged.quantize_kv_fp8(cmp_.float())
    cu = torch.tensor([0] + np.cumsum(q_lens).tolist(), dtype=torch.int32)
    cfg = cases.Config("edge", B=B, H=H, D=D, K=K, cmp_ratio=ratio, scenario=scenario,
                       block_size=bs, fp8=fp8, win_left=win)
    return cases.Inputs(cfg=cfg, q=q, ori_kv=ori, ori_bt=ori_bt,
                        cmp_kv=cmp_ if scenario >= 2 else None,
                        cmp_bt=cmp_bt if scenario >= 2 else None,
                        cmp_idx=idx if scenario == 3 else None, cu_seqlens_q=cu,
                        seqused_kv=torch.tensor(kv_lens, dtype=torch.int32),
                        sinks=torch.randn(H, generator=g), q_lens=q_lens, kv_lens=kv_lens)


EDGE = {
    # kv shorter than the window, a 1-token cache, kv shorter than the query
    "short_kv": dict(B=4, H=64, q_lens=[1, 3, 2, 5], kv_lens=[1, 3, 60, 3], K=32),
    # block-boundary windows and tails, block size 16
    "bs16": dict(B=3, H=32, q_lens=[1, 4, 2], kv_lens=[129, 4100, 16], K=48, bs=16),
    # every top-k slot unused (-1): window + sink only
    "all_unused": dict(B=2, H=16, q_lens=[1, 1], kv_lens=[900, 5000], K=64,
                       idx_fn=lambda i: torch.full_like(i, -1)),
    # future / out-of-range indices are masked (kernel.py:705-722)
    "future_idx": dict(B=2, H=16, q_lens=[2, 1], kv_lens=[300, 1000], K=16,
                       idx_fn=lambda i: torch.where(torch.arange(16) % 3 == 0,
                                                    torch.full_like(i, 10 ** 6), i)),
    "h48_d512": dict(B=2, H=48, q_lens=[3, 1], kv_lens=[2000, 700], K=100, D=512),
    "h128_win63": dict(B=2, H=128, q_lens=[4, 2], kv_lens=[1500, 3000], K=200, win=63),
    "cfa_r8": dict(B=2, H=64, q_lens=[2, 1], kv_lens=[1000, 333], K=0, scenario=2, ratio=8),
    "swa_only": dict(B=3, H=64, q_lens=[1, 2, 1], kv_lens=[50, 700, 128], K=0, scenario=1),
    "fp8_small": dict(B=2, H=64, q_lens=[1, 2], kv_lens=[3000, 900], K=128, fp8=True),
    "fp16": dict(B=2, H=64, q_lens=[1, 2], kv_lens=[3000, 900], K=128, dtype=torch.float16),
    # D = 512 through the channel-split 8-wave kernel: 32-head groups (decode)
    # and 64-head groups (600 query rows)
    "d512": dict(B=2, H=64, q_lens=[3, 2], kv_lens=[2500, 800], K=100, D=512),
    "d512_prefill": dict(B=1, H=64, q_lens=[600], kv_lens=[2400], K=128, D=512),
    # window of one row (win_left 0) and of 256 rows
    "win0": dict(B=2, H=32, q_lens=[3, 1], kv_lens=[500, 90], K=64, win=0),
    "win255_prefill": dict(B=1, H=64, q_lens=[300], kv_lens=[1200], K=96, win=255),
    # block size 128, an odd top-k width, H = 128 in fp16
    "bs128_k77": dict(B=3, H=64, q_lens=[1, 2, 1], kv_lens=[3000, 777, 129], K=77, bs=128),
    "h128_fp16": dict(B=2, H=128, q_lens=[2, 1], kv_lens=[2500, 1000], K=256, dtype=torch.float16),
    # window-only calls: the exact-window schedule with 16, 32 and 64 heads
    # per workgroup, fp8 rows, a 64-row window, a padded BSND-like short
    # cache; a 201-row window exceeds the ring and streams instead
    "swa_h16": dict(B=2, H=16, q_lens=[1, 3], kv_lens=[200, 60], K=0, scenario=1),
    "swa_h48_d512_fp16": dict(B=2, H=48, q_lens=[2, 1], kv_lens=[900, 130], K=0, scenario=1, D=512,
                              dtype=torch.float16),
    "swa_h32_win63": dict(B=2, H=32, q_lens=[4, 1], kv_lens=[700, 64], K=0, scenario=1, win=63),
    "swa_fp8": dict(B=2, H=64, q_lens=[1, 2], kv_lens=[3000, 90], K=0, scenario=1, fp8=True),
    # 90,240 dense compressed + window slots per token: beyond 64 splits of
    # 1280 slots (71 splits), as long CFA contexts need (api.py:257-268)
    "cfa_beyond_64_splits": dict(B=1, H=16, q_lens=[1], kv_lens=[90000], K=0, scenario=2, ratio=1),
    # a 9000-row sliding window (win_left = 8999)
    "swa_window_9000": dict(B=2, H=64, q_lens=[1, 2], kv_lens=[12000, 9500], K=0, scenario=1, win=8999),
    "swa_prefill_h128": dict(B=1, H=128, q_lens=[300], kv_lens=[300], K=0, scenario=1),
    "swa_win200": dict(B=2, H=64, q_lens=[2, 1], kv_lens=[1000, 150], K=0, scenario=1, win=200),
}


@pytest.mark.parametrize("name", list(EDGE))
def test_edge_cases(name):
    inp = _small(**EDGE[name])
    ref_inp = inp
    if name == "future_idx":
        # The kernel masks each entry on its own (kernel.py:705-722); golden's
        # list walk agrees on prefix-valid lists, so the reference input moves
        # the surviving entries (in order) to the front.
        from dataclasses import replace
        idx = inp.cmp_idx.clone()
        for t in range(idx.shape[0]):
            row = idx[t, 0]
            good = row[row < 10 ** 6].clone()
            row[:] = -1
            row[:good.numel()] = good
        ref_inp = replace(inp, cmp_idx=idx)
    out, lse, _ = _run(inp)
    ref_out, ref_lse = _oracle(ref_inp)
    _check_baseline(out, lse, ref_out, ref_lse, name)


def test_swa_exact_and_streaming_schedules_agree():
    """Window-only decode: the exact-window schedule (one split, p rounded
    against the window's final max) and the streaming schedule (forced by
    an explicit split count) both meet the tolerance; the exact one is at
    least as close to golden, whose rounding it reproduces."""
    inp = _small(B=3, H=64, q_lens=[1, 1, 2], kv_lens=[4000, 128, 777], K=0, scenario=1, seed=3)
    ref_out, ref_lse = _oracle(inp)
    ex_out, ex_lse, ns1 = _run(inp)
    st_out, st_lse, ns2 = _run(inp, num_splits=2)
    assert ns1 == 1 and ns2 == 2
    _check_baseline(ex_out, ex_lse, ref_out, ref_lse, "swa exact")
    _check_baseline(st_out, st_lse, ref_out, ref_lse, "swa streaming")
    e_ex = float((ex_out.float() - ref_out.float()).abs().mean())
    e_st = float((st_out.float() - ref_out.float()).abs().mean())
    print(f"[parity] swa mean |out - golden|: exact {e_ex:.4g}, streaming {e_st:.4g}", flush=True)
    assert e_ex <= e_st


@pytest.mark.parametrize("win", [127, 135, 143], ids=["at_key0", "at_key8", "at_key16"])
@pytest.mark.parametrize("K", [16, 300], ids=["jump_in_last_step", "jump_mid_stream"])
def test_prefill_score_jump_moves_the_reference(K, win):
    """64-head single-split prefill whose top-k rows score ~60 nats (~87 log2
    units) above the window rows: the head max jumps far past the reference
    the first steps set (with K = 16 in the last step, with K = 300 in a
    middle one), so O and l are rescaled by ~2^-87 in one step. Both
    wave layouts meet the tolerance against the fp64 oracle. The window
    (win + 1 rows ahead of the top-k rows) puts the first jumping key at
    position 0, 8 or 16 of its 32-row step: in the 8-wave kernel, whose wave
    pairs split a step's keys 0-15 / 16-31, the jump then lands in the first
    half, in both, or in the second half alone (the halves' references move
    apart and are joined)."""
    inp = _small(B=1, H=64, q_lens=[300], kv_lens=[1500], K=K, seed=11, win=win)
    inp.q[:, :, 0] = 40.0
    inp.ori_kv[..., 0] = 0.0
    inp.cmp_kv[..., 0] = 36.0
    ref_out, ref_lse = _oracle(inp)
    for waves in (0, 4):
        out, lse, ns = _run(inp, waves=waves)
        assert ns == 1
        _check_baseline(out, lse, ref_out, ref_lse, f"score jump K={K} waves={waves}")


@pytest.mark.parametrize("scenario,K", [(3, 64), (2, 0), (3, 400)], ids=["scfa_k64", "cfa", "scfa_k400"])
def test_h16_exact_and_register_streamed_kernels_agree(scenario, K):
    """16-head groups: the exact schedule (the default while a split's rows
    fit the 128-row ring, with or without splits) and the register-streamed
    decode kernel (selected by waves=8) both meet the tolerance against
    golden, with 1, 2 and the planned number of splits."""
    inp = _small(B=3, H=16, q_lens=[1, 2, 1], kv_lens=[3000, 700, 129], K=K, scenario=scenario, seed=11)
    ref_out, ref_lse = _oracle(inp)
    for ns in (0, 1, 2):
        for waves in (0, 8):
            out, lse, got_ns = _run(inp, num_splits=ns, waves=waves)
            _check_baseline(out, lse, ref_out, ref_lse, f"h16 splits={ns}->{got_ns} waves={waves}")


def _fuzz_case(i):
    """Seeded random configuration i: scenario, head count, window, block
    size, compressed ratio and top-k width, head dim, dtype, fp8 rows, batch
    of decode or short prefill rows, optional explicit split count."""
    r = np.random.default_rng(1000 + i)
    scenario = int(r.choice([1, 2, 3]))
    D = int(r.choice([512, 576]))
    dtype = torch.float16 if r.random() < 0.25 else torch.bfloat16
    fp8 = D == 576 and dtype == torch.bfloat16 and r.random() < 0.25
    B = int(r.integers(1, 5))
    prefill = r.random() < 0.2
    q_lens = [int(r.integers(8, 65)) if prefill else int(r.integers(1, 4)) for _ in range(B)]
    kv_lens = [int(r.integers(1, 3001)) for _ in range(B)]
    kw = dict(B=B, H=int(r.choice([16, 32, 48, 64, 128])), q_lens=q_lens, kv_lens=kv_lens,
              K=int(r.choice([16, 100, 300, 700])) if scenario == 3 else 0,
              ratio=int(r.choice([4, 8])), bs=int(r.choice([16, 64, 128])), D=D, scenario=scenario,
              fp8=fp8, dtype=dtype, win=int(r.choice([0, 31, 63, 127, 255])), seed=i)
    splits = int(r.choice([0, 0, 1, 2, 5]))
    return kw, splits


def _key_split_case(i):
    """Seeded configuration i for the 64-head 8-wave plan (wave pairs that
    split each 32-row step's keys): 64 or 128 heads, D 512 or 576, bf16 or
    fp16, row counts from a few keys (the second key half of the only step
    empty) to several steps with a ragged last one, 1 to 3 splits."""
    r = np.random.default_rng(5000 + i)
    scenario = int(r.choice([1, 2, 3]))
    B = int(r.integers(1, 4))
    kw = dict(B=B, H=int(r.choice([64, 128])), q_lens=[int(r.integers(1, 6)) for _ in range(B)],
              kv_lens=[int(r.choice([int(r.integers(1, 48)), int(r.integers(48, 3001))])) for _ in range(B)],
              K=int(r.choice([7, 16, 40, 300])) if scenario == 3 else 0, ratio=int(r.choice([4, 8])),
              bs=int(r.choice([16, 64])), D=int(r.choice([512, 576])), scenario=scenario,
              dtype=torch.float16 if r.random() < 0.5 else torch.bfloat16,
              win=int(r.choice([0, 5, 15, 16, 31, 127])), seed=i)
    return kw, int(r.choice([1, 2, 3]))


@pytest.mark.parametrize("i", range(16))
def test_key_split_pairs_against_oracle(i):
    """The 64-head 8-wave kernel (forced) on seeded small configurations:
    out within atol = rtol = 2e-2, LSE within 1e-3 of the oracle."""
    kw, splits = _key_split_case(i)
    print(f"[key-split {i}] {kw} splits={splits}", flush=True)
    inp = _small(**kw)
    out, lse, ns = _run(inp, num_splits=splits, head_waves=4, waves=8)
    ref_out, ref_lse = _oracle(inp)
    _check_baseline(out, lse, ref_out, ref_lse, f"key-split {i} (splits {ns})")


@pytest.mark.parametrize("i", range(64))
def test_random_configurations_against_oracle(i):
    """Random configurations (seeded) through the planner's own choices or an
    explicit split count: out within atol = rtol = 2e-2, LSE within 1e-3."""
    kw, splits = _fuzz_case(i)
    print(f"[fuzz {i}] {kw} splits={splits}", flush=True)
    inp = _small(**kw)
    out, lse, ns = _run(inp, num_splits=splits)
    ref_out, ref_lse = _oracle(inp)
    _check_baseline(out, lse, ref_out, ref_lse, f"fuzz {i} (splits {ns})")


def test_bsnd_layout_with_padding():
    """BSND q [B, S, N, D] with per-batch lengths from cu_seqlens_q: padded
    slots come back as zeros (golden.py:97), valid ones match TND."""
    inp = _small(B=2, H=64, q_lens=[3, 1], kv_lens=[800, 400], K=64)
    d = inp.to("cuda")
    q_b = torch.zeros(2, 3, 64, 576, dtype=torch.bfloat16, device="cuda")
    q_b[0, :3] = d.q[0:3]
    q_b[1, :1] = d.q[3:4]
    idx_b = torch.full((2, 3, 1, 64), -1, dtype=torch.int32, device="cuda")
    idx_b[0, :3] = d.cmp_idx[0:3]
    idx_b[1, :1] = d.cmp_idx[3:4]
    kw = d.api_kwargs()
    kw.update(layout_q="BSND", cmp_sparse_indices=idx_b)
    out, lse = sparse_attn_sharedkv(q_b, return_softmax_lse=True, **kw)
    torch.cuda.synchronize()
    assert out.shape == (2, 3, 64, 512) and lse.shape == (2, 3, 64)
    ref_out, ref_lse = _oracle(inp)
    torch.testing.assert_close(out[0, :3].cpu().float(), ref_out[0:3].float(), atol=OUT_TOL, rtol=OUT_TOL)
    torch.testing.assert_close(out[1, :1].cpu().float(), ref_out[3:4].float(), atol=OUT_TOL, rtol=OUT_TOL)
    torch.testing.assert_close(lse[1, :1].cpu(), ref_lse[3:4], atol=LSE_ATOL, rtol=0)
    assert torch.count_nonzero(out[1, 1:].cpu().float()) == 0
    assert torch.count_nonzero(lse[1, 1:].cpu()) == 0


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
def test_combine_entry_point_closed_form(out_dtype):
    """sas_combine_v1 against the closed-form LSE merge on random partials:
    values (fp16 under bf16 outputs, fp32 under fp16 outputs) with one
    power-of-two exponent per (token, split, head, 256-channel half),
    including exponents far outside fp16's range."""
    T, S, H, DV = 3, 5, 32, 512
    g = torch.Generator().manual_seed(1)
    vals = torch.randn(T, S, H, DV, generator=g)
    vals = vals.to(torch.float16) if out_dtype == torch.bfloat16 else vals
    lo = -20 if out_dtype == torch.bfloat16 else 0   # fp16 outputs: keep |out| below 65504
    ex = torch.randint(lo, 40, (T, S, H, 2), generator=g).float()
    ex[0, 1, 3, 0] = 120.0                      # O around 2^-120
    ex[2, 0, 5, 1] = -100.0                     # O around 2^100 (l large too)
    m2 = torch.randn(T, S, H, generator=g) * 3
    l = torch.rand(T, S, H, generator=g) * 10 + 0.1
    l[2, 0, 5] = 2.0 ** 100
    m2[1, 2] = -math.inf          # an empty split
    l[1, 2] = 0.0
    sinks = torch.randn(H, generator=g)
    ml = torch.stack([m2, l, ex[..., 0], ex[..., 1]], dim=-1).contiguous()
    out = torch.empty(T, H, DV, dtype=out_dtype, device="cuda")
    lse = torch.empty(T, H, dtype=torch.float32, device="cuda")
    dpo, dml, ds = vals.cuda(), ml.cuda(), sinks.cuda()
    a = _lib.SasCombineArgs(part_o=dpo.data_ptr(), part_ml=dml.data_ptr(), sinks=ds.data_ptr(),
                            out=out.data_ptr(), lse=lse.data_ptr(), T=T, S=S, H=H, DV=DV,
                            out_dtype=_lib.SAS_DT_BF16 if out_dtype == torch.bfloat16 else _lib.SAS_DT_FP16)
    st = torch.cuda.current_stream().cuda_stream
    _lib.check(_lib.lib().sas_combine_v1(C.byref(a), C.c_void_p(st)), "combine")
    torch.cuda.synchronize()
    ln2 = math.log(2.0)
    scale = torch.cat([ex[..., :1].expand(T, S, H, DV // 2), ex[..., 1:].expand(T, S, H, DV // 2)], dim=-1)
    po = vals.double() * torch.pow(2.0, -scale.double())   # the partial O the values encode
    m_nat = (m2 * ln2).double()                             # partial maxima, natural log
    sk = sinks.double().view(1, H)
    M = torch.maximum(sk, m_nat.amax(dim=1))
    w = torch.exp(m_nat - M.unsqueeze(1))                   # [T, S, H]
    L = torch.exp(sk - M) + (w * l.double()).sum(dim=1)
    ref = (w.unsqueeze(-1) * po).sum(dim=1) / L.unsqueeze(-1)
    tol = 1e-2 if out_dtype == torch.bfloat16 else 2e-3
    torch.testing.assert_close(out.cpu().float(), ref.to(out_dtype).float(), atol=tol, rtol=tol)
    torch.testing.assert_close(lse.cpu().double(), M + torch.log(L), atol=1e-5, rtol=1e-5)


def test_prepared_call_replays_in_a_hip_graph():
    """A prepared decode call (split kernel + combine, no memsets or host
    work inside) captured in a HIP graph: every replay, with eager work and
    synchronisations in between, equals the eager result."""
    from dsv4_amd.api import prepare_sparse_attn_sharedkv
    inp = cases.make_inputs(cases.CONFIGS["C2"], device="cpu")
    d = inp.to("cuda")
    kw = d.api_kwargs()
    call = prepare_sparse_attn_sharedkv(d.q, **kw)
    call.launch()
    torch.cuda.synchronize()
    ref_out, ref_lse = call.out.clone(), call.lse.clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        call.out.zero_()
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=side):
            call.launch(side)
    torch.cuda.synchronize()
    for i in range(4):
        call.out.fill_(float(i + 1))            # eager work between replays
        call.lse.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(call.out, ref_out) and torch.equal(call.lse, ref_lse), f"replay {i}"


def test_drop_in_call_captured_in_a_graph_keeps_its_workspace():
    """The drop-in call captured in a HIP graph owns its split workspace: an
    eager call with a larger workspace on the same stream afterwards (which
    replaces that stream's shared buffer) leaves the graph's replays equal to
    the eager result."""
    small = cases.make_inputs(cases.CONFIGS["C1"], device="cpu").to("cuda")
    big = cases.make_inputs(cases.CONFIGS["C2"], device="cpu").to("cuda")
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        ref_out, ref_lse = sparse_attn_sharedkv(small.q, return_softmax_lse=True, **small.api_kwargs())
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=side):
            g_out, g_lse = sparse_attn_sharedkv(small.q, return_softmax_lse=True, **small.api_kwargs())
        for i in range(3):
            # a larger call on the same stream grows (replaces) its shared workspace
            b_out = sparse_attn_sharedkv(big.q, **big.api_kwargs())
            g_out.fill_(float(i + 1))
            g_lse.zero_()
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(g_out, ref_out) and torch.equal(g_lse, ref_lse), f"replay {i}"
            del b_out


def test_api_repeated_calls_read_current_values():
    """The drop-in call caches its argument resolution per signature
    (shapes, dtypes, device addresses, scalars, stream): repeated calls must
    still read the current values of every input. Host sequence lengths
    changed in place, device q / indices rewritten in place, and a fresh q
    tensor each give the oracle's result for the values at that call."""
    inp = _small(B=3, H=64, q_lens=[1, 2, 1], kv_lens=[900, 700, 300], K=64, seed=5)
    d = inp.to("cuda")
    kw = d.api_kwargs()
    kw.update(cu_seqlens_q=inp.cu_seqlens_q.clone(), seqused_kv=inp.seqused_kv.clone())   # host
    from dataclasses import replace

    def check(cur, name):
        out, lse = sparse_attn_sharedkv(d.q, return_softmax_lse=True, **kw)
        torch.cuda.synchronize()
        ref_out, ref_lse = _oracle(cur)
        _check_baseline(out.cpu(), lse.cpu(), ref_out, ref_lse, name)

    check(inp, "first call")
    check(inp, "cached call")
    kw["seqused_kv"][:] = torch.tensor([850, 650, 290], dtype=torch.int32)   # host lengths, same tensor
    check(replace(inp, seqused_kv=kw["seqused_kv"].clone(), kv_lens=[850, 650, 290]), "host lengths changed")
    g = torch.Generator().manual_seed(9)
    newq = torch.randn(inp.q.shape, generator=g).to(inp.q.dtype)
    d.q.copy_(newq.cuda())                                                   # device q, same address
    cur = replace(inp, q=newq, seqused_kv=kw["seqused_kv"].clone(), kv_lens=[850, 650, 290])
    check(cur, "q rewritten in place")
    d = replace(d, q=newq.cuda().clone())                                    # a fresh q tensor
    check(cur, "fresh q tensor")


def _fp8_code_rows(T, seed=0):
    """T 656-byte fp8 rows whose latent bytes run through every non-NaN
    e4m3fn code (0x00-0x7e, 0x80-0xfe) at several per-group scales."""
    codes = torch.tensor([c for c in range(256) if c not in (0x7F, 0xFF)], dtype=torch.uint8)
    g = torch.Generator().manual_seed(seed)
    rows = torch.zeros(T, 656, dtype=torch.uint8)
    lat = codes.repeat((T * 512 + codes.numel() - 1) // codes.numel())[:T * 512]
    rows[:, :512] = lat[torch.randperm(T * 512, generator=g)].reshape(T, 512)
    # scales representable in bf16: the kernel applies the scale to P (as
    # bf16(P x scale)), so these make its one-key output bf16(code x scale)
    # exactly, as golden's on the fp32-dequantised row
    scales = torch.tensor([1.0, 0.037109375, 0.0034942626953125, 117.0], dtype=torch.float32)
    sc = scales[torch.randint(0, 4, (T, 4), generator=g)]
    rows[:, 512:528] = sc.contiguous().view(torch.uint8).reshape(T, 16)
    rows[:, 528:] = torch.randn(T, 64, generator=g).to(torch.bfloat16).view(torch.uint8).reshape(T, 128)
    return rows


@pytest.mark.parametrize("H,scenario,waves", [(64, 1, 0), (16, 3, 0), (16, 3, 8), (64, 3, 4), (64, 3, 8)],
                         ids=["exact_h64", "exact_h16", "stream_h16", "stream_h64", "stream8_h64"])
def test_fp8_dequant_bit_exact_through_one_row_windows(H, scenario, waves):
    """Each token attends to exactly one cache row (window of one row, no
    compressed rows, a sink at -3e4): P = 1, l = 1, so the output is that
    row's V channels as the kernel decoded them, bf16(e4m3 x scale),
    compared bit for bit with the codec over every non-NaN code. Covers the
    exact schedule (64 and 16 heads) and the streaming kernel (16 heads,
    selected by waves=8 past the exact schedule; 64 heads with 4 waves, and
    8 waves whose wave pairs split the channels)."""
    T, bs = 96, 16
    rows = _fp8_code_rows(T)
    cache = rows.reshape(T // bs, bs, 1, 656)
    bt = torch.arange(T // bs, dtype=torch.int32).reshape(1, -1)
    g = torch.Generator().manual_seed(1)
    q = torch.randn(T, H, 576, generator=g).to(torch.bfloat16)
    kw = dict(ori_kv=cache.cuda(), ori_block_table=bt.cuda(), cu_seqlens_q=torch.tensor([0, T], dtype=torch.int32),
              seqused_kv=torch.tensor([T], dtype=torch.int32), sinks=torch.full((H,), -3.0e4),
              softmax_scale=1 / 24.0, ori_win_left=0)
    if scenario == 3:
        kw.update(cmp_kv=cache.cuda(), cmp_block_table=bt.cuda(), cmp_ratio=4,
                  cmp_sparse_indices=torch.full((T, 1, 16), -1, dtype=torch.int32).cuda())
    call = prepare_sparse_attn_sharedkv(q.cuda(), waves=waves, **kw)
    call.launch()
    torch.cuda.synchronize()
    out = call.out
    want = paged.dequantize_kv_fp8(rows)[:, :512].to(torch.bfloat16)      # row t is token t's only key
    got = out.cpu()
    for h in range(H):   # by value: code 0x80 (-0.0) accumulates to +0.0
        assert torch.equal(got[:, h].float(), want.float()), \
            f"head {h}: {int((got[:, h].float() != want.float()).sum())} channels differ"
