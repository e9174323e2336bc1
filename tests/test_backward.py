"""Backward (sas_bwd_v1): the fp64 autograd oracle pinned by the golden
forward, finite differences and the closed-form sink gradient; the GPU
kernel against the oracle."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from dsv4_amd import cases, paged
from oracle import backward_ref as BR
from oracle import golden_ref as O


def _tiny(dtype=torch.float64, seed=0, scenario=3):
    """2 batches (q_lens 3 and 1, kv_lens 40 and 23), H = 2, D = 576, block
    size 8, window 15, ratio 4, top-k 6: every kind of row in a few keys."""
    g = torch.Generator().manual_seed(seed)
    q_lens, kv_lens, bs, H, D, K, ratio = [3, 1], [40, 23], 8, 2, 576, 6, 4
    T = sum(q_lens)
    ori_bt, ori_nb = paged.random_block_table(kv_lens, bs, g, extra_blocks=2)
    cmp_lens = [k // ratio for k in kv_lens]
    cmp_bt, cmp_nb = paged.random_block_table(cmp_lens, bs, g, extra_blocks=1)
    kw = dict(
        ori_kv=torch.randn(ori_nb, bs, 1, D, generator=g).to(dtype), ori_block_table=ori_bt,
        cu_seqlens_q=torch.tensor([0] + np.cumsum(q_lens).tolist(), dtype=torch.int32),
        seqused_kv=torch.tensor(kv_lens, dtype=torch.int32), sinks=torch.randn(H, generator=g).double(),
        softmax_scale=1 / math.sqrt(D), ori_win_left=15, dv=512)
    if scenario >= 2:
        kw.update(cmp_kv=torch.randn(cmp_nb, bs, 1, D, generator=g).to(dtype), cmp_block_table=cmp_bt,
                  cmp_ratio=ratio)
    if scenario == 3:
        kw["cmp_sparse_indices"] = cases.topk_indices(q_lens, kv_lens, K, ratio, g)
    q = torch.randn(T, H, D, generator=g).to(dtype)
    dout = torch.randn(T, H, 512, generator=g).to(dtype)
    return q, dout, kw


def test_oracle_forward_is_golden():
    q, dout, kw = _tiny()
    r = BR.backward_paged(q, dout, **kw)
    g = dict(kw)
    g.pop("dv")
    out, lse = O.golden_paged(q, dv=512, exact=True, **g)
    torch.testing.assert_close(r["out"], out, atol=1e-10, rtol=1e-10)
    torch.testing.assert_close(r["lse"], lse, atol=1e-10, rtol=1e-10)


def test_oracle_planted_dropped_sink_fails():
    q, dout, kw = _tiny()
    r = BR.backward_paged(q, dout, drop_sink=True, **kw)
    g = dict(kw)
    g.pop("dv")
    out, _ = O.golden_paged(q, dv=512, exact=True, **g)
    assert not torch.allclose(r["out"], out, atol=1e-6, rtol=1e-6)


def test_oracle_sink_gradient_closed_form():
    """d(sink_h) = -sum_t exp(sink_h - lse_th) (dO_th . O_th): the sink's value
    row is zero, so only the softmax normaliser depends on it."""
    q, dout, kw = _tiny()
    r = BR.backward_paged(q, dout, **kw)
    delta = (dout.double() * r["out"]).sum(-1)                       # [T, H]
    ref = -(torch.exp(kw["sinks"].view(1, -1) - r["lse"]) * delta).sum(0)
    torch.testing.assert_close(r["d_sinks"], ref, atol=1e-12, rtol=1e-10)


@pytest.mark.parametrize("scenario", [1, 2, 3])
def test_oracle_given_forward_equals_autograd(scenario):
    """The explicit FlashAttention-2 formulas from the exact forward's out /
    lse give the autograd gradients (dq, touched cache rows, sinks); a
    planted sign error in dS does not."""
    q, dout, kw = _tiny(scenario=scenario, seed=10 + scenario)
    r = BR.backward_paged(q, dout, **kw)
    e = BR.backward_given_forward(q, dout, r["out"], r["lse"], **kw)
    torch.testing.assert_close(e["dq"], r["dq"], atol=1e-10, rtol=1e-9)
    torch.testing.assert_close(e["d_sinks"], r["d_sinks"], atol=1e-10, rtol=1e-9)
    for key in ("d_ori", "d_cmp") if scenario >= 2 else ("d_ori",):
        assert torch.equal(e[key][0], r[key][0])
        torch.testing.assert_close(e[key][1], r[key][1], atol=1e-10, rtol=1e-9)
    bad = BR.backward_given_forward(q, dout, r["out"], r["lse"], plant_sign=True, **kw)
    assert not torch.allclose(bad["dq"], r["dq"], atol=1e-6, rtol=1e-6)


@pytest.mark.parametrize("scenario", [1, 2, 3])
def test_oracle_finite_differences(scenario):
    """Central differences of sum(dO * out) in fp64 match the autograd
    gradients of q, of cache rows (a V channel and a rope channel) and of the
    sinks."""
    q, dout, kw = _tiny(scenario=scenario, seed=scenario)
    r = BR.backward_paged(q, dout, **kw)
    eps = 1e-6

    def loss(qq=q, sinks=kw["sinks"], ori=kw["ori_kv"], cmp_=kw.get("cmp_kv")):
        k2 = dict(kw, sinks=sinks, ori_kv=ori)
        if cmp_ is not None:
            k2["cmp_kv"] = cmp_
        return BR.loss_fp64(qq, dout, **{k: v for k, v in k2.items() if k not in ("sinks", "ori_kv", "cmp_kv")},
                            sinks=k2["sinks"], ori_kv=k2["ori_kv"], cmp_kv=k2.get("cmp_kv"))

    def fd(name, tensor, index):
        hi, lo = tensor.clone(), tensor.clone()
        hi[index] += eps
        lo[index] -= eps
        return (loss(**{name: hi}) - loss(**{name: lo})) / (2 * eps)

    for t, h, c in [(0, 0, 3), (2, 1, 511), (3, 0, 570)]:
        assert abs(fd("qq", q, (t, h, c)) - float(r["dq"][t, h, c])) < 1e-6
    rows, grads = r["d_ori"]
    D = q.shape[-1]
    for i in (0, len(rows) // 2, len(rows) - 1):
        row = int(rows[i])
        for c in (5, 530):
            ix = (row // kw["ori_kv"].shape[1], row % kw["ori_kv"].shape[1], 0, c)
            assert abs(fd("ori", kw["ori_kv"], ix) - float(grads[i, c])) < 1e-6
    if scenario >= 2:
        rows, grads = r["d_cmp"]
        row = int(rows[0])
        ix = (row // kw["cmp_kv"].shape[1], row % kw["cmp_kv"].shape[1], 0, 100)
        assert abs(fd("cmp_", kw["cmp_kv"], ix) - float(grads[0, 100])) < 1e-6
    for h in range(2):
        assert abs(fd("sinks", kw["sinks"], (h,)) - float(r["d_sinks"][h])) < 1e-6


# ---------------------------------------------------------------------------
# GPU: the kernel against the oracle
# ---------------------------------------------------------------------------

def _gpu_case(name):
    from tests.test_gpu_parity import _small
    if name == "C1":
        return cases.make_inputs(cases.CONFIGS["C1"], device="cpu")
    spec = {
        "scfa_prefill": dict(B=2, H=32, q_lens=[40, 3], kv_lens=[300, 90], K=64, bs=16),
        "swa": dict(B=3, H=16, q_lens=[1, 5, 2], kv_lens=[50, 700, 128], K=0, scenario=1),
        "cfa": dict(B=2, H=16, q_lens=[2, 1], kv_lens=[500, 333], K=0, scenario=2, ratio=8),
        "fp16_d512": dict(B=2, H=16, q_lens=[1, 2], kv_lens=[900, 400], K=64, D=512, dtype=torch.float16),
        "decode_h64": dict(B=8, H=64, q_lens=[1] * 8, kv_lens=[4000, 900, 129, 2500, 60, 3000, 1000, 2048], K=128),
        # kv shorter than the query: early tokens attend to no row (sink only)
        "short_kv": dict(B=4, H=32, q_lens=[1, 3, 2, 5], kv_lens=[1, 3, 60, 3], K=32),
        # 128 + 2048 dense compressed slots per token: beyond one workgroup's
        # 1280-slot range, so the planner splits the key range
        "cfa_2176_slots": dict(B=2, H=16, q_lens=[2, 1], kv_lens=[8192, 6000], K=0, scenario=2, ratio=4),
        # the same beyond-1280-slot split through the 64-head kernel
        # (sas_bwd64_kernel: H a multiple of 64), with 64 and 128 heads
        "cfa_2176_slots_h64": dict(B=2, H=64, q_lens=[2, 1], kv_lens=[8192, 6000], K=0, scenario=2, ratio=4),
        "cfa_2176_slots_h128": dict(B=2, H=128, q_lens=[1, 2], kv_lens=[7000, 8192], K=0, scenario=2, ratio=4),
    }[name]
    return _small(**spec)


def _rel_err(got, ref):
    ref = ref.double()
    return float((got.double() - ref).abs().max() / max(float(ref.abs().max()), 1e-30))


GRAD_TOL = 2e-2


def _check_elem(got, ref, what, tol=GRAD_TOL):
    """Element-wise: |got - ref| <= tol |ref| + tol max|ref over the element's
    row| (the last dimension: a (token, head)'s dq channels, a cache row's
    gradient channels, the H sink gradients), so a wrong small row fails even
    when the largest gradients are right. Returns the worst err / bound."""
    got, ref = got.double().reshape(-1, got.shape[-1]), ref.double().reshape(-1, ref.shape[-1])
    if ref.numel() == 0:
        return 0.0
    rowmax = ref.abs().amax(dim=1, keepdim=True)
    bound = tol * ref.abs() + tol * rowmax
    err = (got - ref).abs()
    ratio = err / bound.clamp_min(1e-300)
    bad = err > bound
    worst = float(ratio.max())
    assert not bool(bad.any()), (f"{what}: {int(bad.sum())} of {err.numel()} elements beyond "
                                 f"{tol}|ref| + {tol} rowmax|ref| (worst err/bound {worst:.3g})")
    return worst


def _check_against_oracle(name, inp, dq, d_ori, d_cmp, d_sinks, r):
    """dq, the touched cache rows (untouched rows exactly zero) and d_sinks
    element-wise against the fp64 oracle result ``r``."""
    c = inp.cfg
    D = inp.q.shape[-1]
    worst = {"dq": _check_elem(dq.cpu(), r["dq"], f"{name} dq")}
    rows, grads = r["d_ori"]
    flat = d_ori.cpu().reshape(-1, D)
    worst["d_ori"] = _check_elem(flat[rows], grads, f"{name} d_ori")
    untouched = torch.ones(flat.shape[0], dtype=torch.bool)
    untouched[rows] = False
    if untouched.any():
        assert float(flat[untouched].abs().max()) == 0.0, f"{name}: untouched ori rows changed"
    if c.scenario >= 2:
        rows, grads = r["d_cmp"]
        cflat = d_cmp.cpu().reshape(-1, D)
        if rows.numel():
            worst["d_cmp"] = _check_elem(cflat[rows], grads, f"{name} d_cmp")
        untouched = torch.ones(cflat.shape[0], dtype=torch.bool)
        untouched[rows] = False
        if untouched.any():
            assert float(cflat[untouched].abs().max()) == 0.0, f"{name}: untouched cmp rows changed"
    worst["d_sinks"] = _check_elem(d_sinks.cpu().reshape(1, -1), r["d_sinks"].reshape(1, -1), f"{name} d_sinks")
    print(f"[bwd] {name}: worst err / bound = {worst}", flush=True)


def _oracle_bwd(inp, dout, out, lse, tokens=None):
    """The fp64 backward from the GPU forward's own out / lse (the inputs
    sas_bwd_v1 takes; the formulas are pinned to autograd above): the GPU
    result may then differ only by its bf16 operand roundings and fp32
    accumulation, element by element."""
    c = inp.cfg
    return BR.backward_given_forward(
        inp.q, dout, out, lse, ori_kv=inp.ori_kv, ori_block_table=inp.ori_bt, cu_seqlens_q=inp.cu_seqlens_q,
        seqused_kv=inp.seqused_kv, sinks=inp.sinks, softmax_scale=c.scale,
        cmp_kv=inp.cmp_kv if c.scenario >= 2 else None, cmp_block_table=inp.cmp_bt if c.scenario >= 2 else None,
        cmp_sparse_indices=inp.cmp_idx if c.scenario == 3 else None, cmp_ratio=c.cmp_ratio,
        ori_win_left=c.win_left, tokens=tokens)


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["C1", "scfa_prefill", "swa", "cfa", "fp16_d512", "decode_h64", "short_kv",
                                  "cfa_2176_slots", "cfa_2176_slots_h64", "cfa_2176_slots_h128"])
def test_gpu_backward_matches_oracle(name):
    from dsv4_amd.api import sparse_attn_sharedkv, sparse_attn_sharedkv_backward
    inp = _gpu_case(name)
    d = inp.to("cuda")
    kw = d.api_kwargs()
    out, lse = sparse_attn_sharedkv(d.q, return_softmax_lse=True, **kw)
    g = torch.Generator().manual_seed(5)
    dout = torch.randn(out.shape, generator=g).to(inp.q.dtype)
    dq, d_ori, d_cmp, d_sinks = sparse_attn_sharedkv_backward(dout.cuda(), d.q, out, lse, **kw)
    torch.cuda.synchronize()
    # tolerance: bf16 / fp16 rounding of the forward output (used in Delta),
    # of the MFMA operands dS / P and of dq; fp32 accumulation elsewhere
    _check_against_oracle(name, inp, dq, d_ori, d_cmp, d_sinks, _oracle_bwd(inp, dout, out, lse))


@pytest.mark.gpu
@pytest.mark.parametrize("i", range(24))
def test_gpu_backward_random_configurations(i):
    """Seeded random configurations (scenario, H, D, dtype, window, block
    size, ratio, top-k, decode or short prefill batches), every gradient
    element against the oracle from the GPU forward's own out / lse."""
    from dsv4_amd.api import sparse_attn_sharedkv, sparse_attn_sharedkv_backward
    from tests.test_gpu_parity import _fuzz_case, _small
    kw, _ = _fuzz_case(500 + i)
    kw["fp8"] = False   # the backward takes caches in the query dtype
    print(f"[bwd fuzz {i}] {kw}", flush=True)
    inp = _small(**kw)
    d = inp.to("cuda")
    akw = d.api_kwargs()
    out, lse = sparse_attn_sharedkv(d.q, return_softmax_lse=True, **akw)
    g = torch.Generator().manual_seed(7 + i)
    dout = torch.randn(out.shape, generator=g).to(inp.q.dtype)
    dq, d_ori, d_cmp, d_sinks = sparse_attn_sharedkv_backward(dout.cuda(), d.q, out, lse, **akw)
    torch.cuda.synchronize()
    _check_against_oracle(f"bwd fuzz {i}", inp, dq, d_ori, d_cmp, d_sinks, _oracle_bwd(inp, dout, out, lse))


@pytest.mark.gpu
def test_gpu_backward_c2_decode_full():
    """The C2 workload the bench times (32 tokens, H = 64, top-k 512 +
    window 128 over 8K-32K contexts), every gradient against the oracle."""
    from dsv4_amd.api import sparse_attn_sharedkv, sparse_attn_sharedkv_backward
    inp = cases.make_inputs(cases.CONFIGS["C2"], device="cpu")
    d = inp.to("cuda")
    kw = d.api_kwargs()
    out, lse = sparse_attn_sharedkv(d.q, return_softmax_lse=True, **kw)
    g = torch.Generator().manual_seed(21)
    dout = torch.randn(out.shape, generator=g).to(inp.q.dtype)
    dq, d_ori, d_cmp, d_sinks = sparse_attn_sharedkv_backward(dout.cuda(), d.q, out, lse, **kw)
    torch.cuda.synchronize()
    _check_against_oracle("C2", inp, dq, d_ori, d_cmp, d_sinks, _oracle_bwd(inp, dout, out, lse))


@pytest.mark.gpu
def test_gpu_backward_c3_prefill_sampled():
    """The C3 4096-token prefill the bench times, with dout nonzero on 48
    sampled tokens only (first, last, window and block edges, random): the
    other tokens then contribute nothing to any gradient, so the oracle on
    the sampled tokens gives the exact expected dq, cache and sink
    gradients of the whole launch."""
    from dsv4_amd.api import sparse_attn_sharedkv, sparse_attn_sharedkv_backward
    inp = cases.make_inputs(cases.CONFIGS["C3"], device="cpu")
    d = inp.to("cuda")
    kw = d.api_kwargs()
    out, lse = sparse_attn_sharedkv(d.q, return_softmax_lse=True, **kw)
    g = torch.Generator().manual_seed(22)
    toks = sorted(set([0, 1, 127, 128, 129, 511, 512, 2047, 4094, 4095] +
                      torch.randint(0, 4096, (38,), generator=g).tolist()))
    dout = torch.zeros(out.shape, dtype=inp.q.dtype)
    dout[toks] = torch.randn((len(toks),) + tuple(out.shape[1:]), generator=g).to(inp.q.dtype)
    dq, d_ori, d_cmp, d_sinks = sparse_attn_sharedkv_backward(dout.cuda(), d.q, out, lse, **kw)
    torch.cuda.synchronize()
    r = _oracle_bwd(inp, dout, out, lse, tokens=toks)
    _check_against_oracle("C3 sampled", inp, dq, d_ori, d_cmp, d_sinks, r)


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["prefill_2b", "prefill_bs16_h16", "swa", "short_kv", "decode_h64", "cfa",
                                  "fp16_d512", "prefill_wide_window", "prefill_swa_bs16"])
def test_gpu_backward_window_pass_both_ways(name):
    """Window rows' gradients summed per (token, row) and by the key-major
    window pass (forced both ways, whatever the library would choose): each
    element-wise against the fp64 oracle, on prefills (several batches, BSND
    pages of 16, a window wider than the 64-position tile) and on
    decode and short-KV batches (tokens with empty windows, rows past
    act_kv)."""
    from dsv4_amd.api import sparse_attn_sharedkv, sparse_attn_sharedkv_backward
    from tests.test_gpu_parity import _small
    extra = {
        "prefill_2b": dict(B=2, H=64, q_lens=[300, 170], kv_lens=[300, 420], K=64, bs=64),
        "prefill_bs16_h16": dict(B=3, H=16, q_lens=[90, 17, 64], kv_lens=[90, 200, 64], K=32, bs=16),
        "prefill_wide_window": dict(B=1, H=32, q_lens=[400], kv_lens=[400], K=48, win=300),
        "prefill_swa_bs16": dict(B=2, H=16, q_lens=[200, 70], kv_lens=[260, 70], K=0, scenario=1, bs=16),
    }
    inp = _small(**extra[name]) if name in extra else _gpu_case(name)
    d = inp.to("cuda")
    kw = d.api_kwargs()
    out, lse = sparse_attn_sharedkv(d.q, return_softmax_lse=True, **kw)
    g = torch.Generator().manual_seed(31)
    dout = torch.randn(out.shape, generator=g).to(inp.q.dtype)
    r = _oracle_bwd(inp, dout, out, lse)
    for wp in (False, True):
        dq, d_ori, d_cmp, d_sinks = sparse_attn_sharedkv_backward(dout.cuda(), d.q, out, lse, window_pass=wp, **kw)
        torch.cuda.synchronize()
        _check_against_oracle(f"{name} window_pass={wp}", inp, dq, d_ori, d_cmp, d_sinks, r)


@pytest.mark.gpu
def test_gpu_backward_window_pass_bsnd():
    """The key-major window pass with BSND queries (per-batch lengths, padded
    rows: the kernel reads act_q instead of a prefix difference) gives the
    TND per-token result up to summation order."""
    from tests.test_gpu_parity import _small
    from dsv4_amd.api import sparse_attn_sharedkv, sparse_attn_sharedkv_backward
    q_lens = [70, 30]
    inp = _small(B=2, H=64, q_lens=q_lens, kv_lens=[90, 30], K=16)
    d = inp.to("cuda")
    kw = d.api_kwargs()
    out, lse = sparse_attn_sharedkv(d.q, return_softmax_lse=True, **kw)
    g = torch.Generator().manual_seed(33)
    dout = torch.randn(out.shape, generator=g).to(out.dtype).cuda()
    ref = sparse_attn_sharedkv_backward(dout, d.q, out, lse, window_pass=False, **kw)
    S = max(q_lens)
    q_b = torch.zeros(2, S, 64, 576, dtype=torch.bfloat16, device="cuda")
    idx_b = torch.full((2, S, 1, 16), -1, dtype=torch.int32, device="cuda")
    o_b = torch.zeros(2, S, 64, 512, dtype=torch.bfloat16, device="cuda")
    l_b = torch.zeros(2, S, 64, dtype=torch.float32, device="cuda")
    do_b = torch.zeros(2, S, 64, 512, dtype=torch.bfloat16, device="cuda")
    t_ = 0
    for b, n in enumerate(q_lens):
        q_b[b, :n], idx_b[b, :n], o_b[b, :n], l_b[b, :n], do_b[b, :n] = (
            d.q[t_:t_ + n], d.cmp_idx[t_:t_ + n], out[t_:t_ + n], lse[t_:t_ + n], dout[t_:t_ + n])
        t_ += n
    kwb = dict(kw, layout_q="BSND", cmp_sparse_indices=idx_b)
    dq_b, d_ori, d_cmp, d_snk = sparse_attn_sharedkv_backward(do_b, q_b, o_b, l_b, window_pass=True, **kwb)
    torch.cuda.synchronize()
    assert _rel_err(dq_b[0, :70].float().cpu(), ref[0][:70].float().cpu()) < 1e-2
    assert _rel_err(dq_b[1, :30].float().cpu(), ref[0][70:].float().cpu()) < 1e-2
    assert torch.count_nonzero(dq_b[1, 30:].cpu().float()) == 0
    assert _rel_err(d_ori.cpu(), ref[1].cpu()) < 1e-4 and _rel_err(d_cmp.cpu(), ref[2].cpu()) < 1e-4
    assert _rel_err(d_snk.cpu(), ref[3].cpu()) < 1e-4


@pytest.mark.gpu
def test_gpu_backward_captured_in_a_graph():
    """The backward of a prefill captured in a HIP graph: eagerly the window
    pass runs beside the per-token kernel on the library's side stream;
    under capture it either gives way to per-token adds (the default) or,
    when asked for, runs after the per-token kernel on the captured stream.
    Every replay (with eager work between them) equals the eager run of the
    same mode up to fp32 summation order; the two modes differ from each
    other only by where the window keys' products are rounded."""
    from dsv4_amd.api import prepare_sparse_attn_sharedkv_backward, sparse_attn_sharedkv
    from tests.test_gpu_parity import _small
    inp = _small(B=2, H=64, q_lens=[300, 170], kv_lens=[300, 420], K=64)
    d = inp.to("cuda")
    kw = d.api_kwargs()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        out, lse = sparse_attn_sharedkv(d.q, return_softmax_lse=True, **kw)
        g = torch.Generator().manual_seed(35)
        dout = torch.randn(out.shape, generator=g).to(out.dtype).cuda()
        refs = {}
        for wp in (False, True):
            eager = prepare_sparse_attn_sharedkv_backward(dout, d.q, out, lse, window_pass=wp, **kw)
            eager.launch(side)
            torch.cuda.synchronize()
            refs[wp] = [t.clone() for t in (eager.dq, eager.d_ori_kv, eager.d_cmp_kv, eager.d_sinks)]
        for a, b in zip(refs[False], refs[True]):
            assert _rel_err(a.cpu(), b.cpu()) < 1e-4
        for wp, mode in ((None, False), (True, True)):
            pb = prepare_sparse_attn_sharedkv_backward(dout, d.q, out, lse, window_pass=wp, **kw)
            torch.cuda.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=side):
                pb.zero_grads()
                pb.launch(side)
            grads = (pb.dq, pb.d_ori_kv, pb.d_cmp_kv, pb.d_sinks)
            for i in range(3):
                for t in grads:
                    t.fill_(float(i + 7))             # eager work between replays
                graph.replay()
                torch.cuda.synchronize()
                for name, got, want in zip(("dq", "d_ori", "d_cmp", "d_sinks"), grads, refs[mode]):
                    assert _rel_err(got.cpu(), want.cpu()) < 1e-5, f"window_pass={wp} replay {i} {name}"
            del graph, pb


@pytest.mark.gpu
def test_gpu_backward_split_count_invariance():
    """The key range split over 1, 3 or 7 workgroups per (token, head group)
    (dq then accumulated atomically) gives the same gradients up to fp32
    summation order."""
    from dsv4_amd.api import sparse_attn_sharedkv, sparse_attn_sharedkv_backward
    inp = _gpu_case("decode_h64")
    d = inp.to("cuda")
    kw = d.api_kwargs()
    out, lse = sparse_attn_sharedkv(d.q, return_softmax_lse=True, **kw)
    g = torch.Generator().manual_seed(6)
    dout = torch.randn(out.shape, generator=g).to(inp.q.dtype).cuda()
    res = [sparse_attn_sharedkv_backward(dout, d.q, out, lse, num_splits=ns, **kw) for ns in (1, 3, 7)]
    torch.cuda.synchronize()
    for other in res[1:]:
        for a_, b_ in zip(res[0], other):
            if a_ is not None:
                assert _rel_err(b_.float().cpu(), a_.float().cpu()) < 1e-2 if a_.dtype != torch.float32 \
                    else _rel_err(b_.cpu(), a_.cpu()) < 1e-5


@pytest.mark.gpu
def test_gpu_autograd_binding():
    """loss.backward() through sparse_attn_sharedkv_autograd gives the
    gradients of sparse_attn_sharedkv_backward."""
    from dsv4_amd.api import sparse_attn_sharedkv_autograd, sparse_attn_sharedkv, sparse_attn_sharedkv_backward
    inp = _gpu_case("scfa_prefill")
    d = inp.to("cuda")
    kw = d.api_kwargs()
    q = d.q.clone().requires_grad_(True)
    ori = d.ori_kv.clone().requires_grad_(True)
    cmp_ = d.cmp_kv.clone().requires_grad_(True)
    snk = d.sinks.clone().requires_grad_(True)
    rest = {k: v for k, v in kw.items() if k not in ("ori_kv", "cmp_kv", "sinks")}
    out = sparse_attn_sharedkv_autograd(q, ori_kv=ori, cmp_kv=cmp_, sinks=snk, **rest)
    g = torch.Generator().manual_seed(8)
    dout = torch.randn(out.shape, generator=g).to(out.dtype).cuda()
    (out.float() * dout.float()).sum().backward()
    o2, lse2 = sparse_attn_sharedkv(d.q, return_softmax_lse=True, **kw)
    ref = sparse_attn_sharedkv_backward(dout, d.q, o2, lse2, **kw)
    torch.cuda.synchronize()
    assert torch.equal(out.detach().cpu(), o2.cpu())
    assert _rel_err(q.grad.float().cpu(), ref[0].float().cpu()) < 1e-2
    assert _rel_err(ori.grad.float().cpu(), ref[1].cpu()) < 1e-2
    assert _rel_err(cmp_.grad.float().cpu(), ref[2].cpu()) < 1e-2
    assert _rel_err(snk.grad.cpu(), ref[3].cpu()) < 1e-4


@pytest.mark.gpu
def test_gpu_backward_bsnd_padding_matches_tnd():
    """BSND q [B, S, N, D] with per-batch lengths: the valid rows' dq and the
    cache / sink gradients equal the TND backward of the same tokens up to
    summation order (the two layouts get different KV split counts, so bf16
    dq may differ by a rounding step), and the padded rows' dq is zero."""
    from tests.test_gpu_parity import _small
    from dsv4_amd.api import sparse_attn_sharedkv, sparse_attn_sharedkv_backward
    inp = _small(B=2, H=64, q_lens=[3, 1], kv_lens=[800, 400], K=64)
    d = inp.to("cuda")
    kw = d.api_kwargs()
    out, lse = sparse_attn_sharedkv(d.q, return_softmax_lse=True, **kw)
    g = torch.Generator().manual_seed(9)
    dout = torch.randn(out.shape, generator=g).to(out.dtype).cuda()
    ref = sparse_attn_sharedkv_backward(dout, d.q, out, lse, **kw)
    slot = [(0, 0), (0, 1), (0, 2), (1, 0)]                       # (b, s) of the 4 packed tokens
    q_b = torch.zeros(2, 3, 64, 576, dtype=torch.bfloat16, device="cuda")
    idx_b = torch.full((2, 3, 1, 64), -1, dtype=torch.int32, device="cuda")
    o_b = torch.zeros(2, 3, 64, 512, dtype=torch.bfloat16, device="cuda")
    l_b = torch.zeros(2, 3, 64, dtype=torch.float32, device="cuda")
    do_b = torch.zeros(2, 3, 64, 512, dtype=torch.bfloat16, device="cuda")
    for t_, (b, s_) in enumerate(slot):
        q_b[b, s_], idx_b[b, s_], o_b[b, s_], l_b[b, s_], do_b[b, s_] = (
            d.q[t_], d.cmp_idx[t_], out[t_], lse[t_], dout[t_])
    kwb = dict(kw, layout_q="BSND", cmp_sparse_indices=idx_b)
    dq_b, d_ori, d_cmp, d_snk = sparse_attn_sharedkv_backward(do_b, q_b, o_b, l_b, **kwb)
    torch.cuda.synchronize()
    assert dq_b.shape == q_b.shape
    for t_, (b, s_) in enumerate(slot):
        assert _rel_err(dq_b[b, s_].float().cpu(), ref[0][t_].float().cpu()) < 1e-2
    assert torch.count_nonzero(dq_b[1, 1:].cpu().float()) == 0
    assert _rel_err(d_ori.cpu(), ref[1].cpu()) < 1e-4 and _rel_err(d_cmp.cpu(), ref[2].cpu()) < 1e-4
    assert _rel_err(d_snk.cpu(), ref[3].cpu()) < 1e-4


@pytest.mark.gpu
def test_gpu_backward_h48_d512_matches_oracle():
    """H = 48 (three 16-head workgroups per token) at D = 512."""
    from tests.test_gpu_parity import _small
    from dsv4_amd.api import sparse_attn_sharedkv, sparse_attn_sharedkv_backward
    inp = _small(B=2, H=48, q_lens=[3, 1], kv_lens=[2000, 700], K=100, D=512)
    c = inp.cfg
    d = inp.to("cuda")
    kw = d.api_kwargs()
    out, lse = sparse_attn_sharedkv(d.q, return_softmax_lse=True, **kw)
    g = torch.Generator().manual_seed(10)
    dout = torch.randn(out.shape, generator=g).to(out.dtype)
    dq, d_ori, d_cmp, d_snk = sparse_attn_sharedkv_backward(dout.cuda(), d.q, out, lse, **kw)
    torch.cuda.synchronize()
    _check_against_oracle("h48_d512", inp, dq, d_ori, d_cmp, d_snk, _oracle_bwd(inp, dout, out, lse))
