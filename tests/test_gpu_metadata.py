"""Device scheduler (``sas_metadata_device_v1``, through
``sparse_attn_sharedkv_metadata(..., device="cuda")`` with device-resident
sequence lengths) against the reference's recorded vectors and the host
scheduler, bit for bit."""

from __future__ import annotations

import random

import pytest
import torch

from dsv4_amd import cases as C
from dsv4_amd.metadata import sparse_attn_sharedkv_metadata
from test_metadata import FIX, TENSOR_KEYS, _expected, _fuzz_kwargs, _kw

pytestmark = pytest.mark.gpu


def _on_device(kw):
    out = dict(kw)
    for k in TENSOR_KEYS:
        if isinstance(out.get(k), torch.Tensor):
            out[k] = out[k].cuda()
    out["device"] = "cuda"
    return out


@pytest.mark.parametrize("case", FIX["cases"], ids=[c["name"] for c in FIX["cases"]])
def test_device_scheduler_matches_reference_vectors(case):
    got = sparse_attn_sharedkv_metadata(**_on_device(_kw(case["kwargs"])))
    assert got.is_cuda and got.dtype == torch.int32
    assert got.cpu().tolist() == _expected(case)


def test_device_scheduler_matches_host_fuzz():
    rnd = random.Random(20261)
    n_dev = 0
    for i in range(400):
        kw = _fuzz_kwargs(rnd)
        try:
            host = sparse_attn_sharedkv_metadata(**kw).tolist()
        except ValueError:
            host = None   # a row scan the host rejects: the device marks out[0] = -1
        dev = sparse_attn_sharedkv_metadata(**_on_device(kw)).cpu().tolist()
        if host is None:
            assert dev[0] == -1, f"fuzz case {i}: {kw}"
        else:
            assert dev == host, f"fuzz case {i}: {kw}"
        n_dev += any(isinstance(kw.get(k), torch.Tensor) for k in TENSOR_KEYS)
    assert n_dev > 300   # most cases pass lengths, so they ran on the device


def _long_unit_kwargs(rnd):
    """Few batches of hundreds to thousands of query rows over few cores: the
    row phase scans many windows of rows within one unit, with runs of rows
    without blocks (short or empty KV, sliding windows that end early)."""
    B = rnd.choice([1, 2, 3])
    n2 = rnd.choice([1, 2])
    g = rnd.choice([1, 16, 64])
    ql = [rnd.choice([300, 1000, 3000]) for _ in range(B)]
    kl = [max(0, q + rnd.choice([-2900, -700, -1, 0, 1, 511, 4000])) for q in ql]
    cu = [0]
    for x in ql:
        cu.append(cu[-1] + x)
    kw = dict(num_heads_q=g * n2, num_heads_kv=n2, head_dim=576, batch_size=B, max_seqlen_q=max(ql),
              max_seqlen_kv=max(kl), layout_q="TND", cu_seqlens_q=torch.tensor(cu, dtype=torch.int32),
              seqused_kv=torch.tensor(kl, dtype=torch.int32), has_cmp_kv=rnd.random() < 0.7,
              aic_core_num=rnd.choice([1, 2, 3, 5, 24]), ori_win_left=rnd.choice([127, 0, 511, -1]),
              ori_mask_mode=rnd.choice([4, 4, 3, 0]))
    if kw["has_cmp_kv"]:
        kw["cmp_ratio"] = rnd.choice([1, 4, 128])
        kw["cmp_topk"] = rnd.choice([0, 64, 512])
    return kw


def test_device_scheduler_long_row_scans_match_host():
    rnd = random.Random(20262)
    for i in range(60):
        kw = _long_unit_kwargs(rnd)
        try:
            host = sparse_attn_sharedkv_metadata(**kw).tolist()
        except ValueError:
            host = None
        dev = sparse_attn_sharedkv_metadata(**_on_device(kw)).cpu().tolist()
        if host is None:
            assert dev[0] == -1, f"case {i}: {kw}"
        else:
            assert dev == host, f"case {i}: {kw}"


@pytest.mark.parametrize("name", ["C2", "C3", "scfa_prefill"])
def test_device_scheduler_at_benchmark_shapes(name):
    """The decode and prefill workloads (C3: 4096 query rows, the row phase
    over windows of rows; the reference's 8K prefill: rows past the 5120
    kept in LDS are computed on the spot): same rows as the host, and the
    time a call takes."""
    cfg = C.CONFIGS.get(name) or C.REF_SCENARIOS[name]
    ql, kl = C.seq_lengths(cfg)
    cu = [0]
    for x in ql:
        cu.append(cu[-1] + x)
    kw = dict(num_heads_q=cfg.H, num_heads_kv=1, head_dim=cfg.D,
              cu_seqlens_q=torch.tensor(cu, dtype=torch.int32),
              seqused_kv=torch.tensor(kl, dtype=torch.int32), batch_size=cfg.B,
              max_seqlen_q=max(ql), max_seqlen_kv=max(kl), layout_q="TND",
              has_cmp_kv=cfg.scenario >= 2, cmp_ratio=cfg.cmp_ratio if cfg.scenario >= 2 else -1,
              cmp_topk=cfg.K if cfg.scenario == 3 else 0)
    host = sparse_attn_sharedkv_metadata(**kw).tolist()
    dkw = _on_device(kw)
    dev = sparse_attn_sharedkv_metadata(**dkw)
    assert dev.cpu().tolist() == host
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(10):
        sparse_attn_sharedkv_metadata(**dkw)
    e1.record()
    torch.cuda.synchronize()
    print(f"[metadata] {name}: {sum(ql)} query rows, device schedule {e0.elapsed_time(e1) * 100:.1f} us per call",
          flush=True)


@pytest.mark.parametrize("batches", [1024, 1025, 3000])
def test_device_lengths_beyond_the_device_batch_bound_take_the_host(batches):
    """More batches than the device scheduler holds (1024): the call with
    device-resident lengths still returns the host schedule, on the device,
    instead of raising; at the bound itself the device computes it."""
    rnd = random.Random(batches)
    ql = [rnd.choice([1, 2, 4]) for _ in range(batches)]
    kl = [rnd.randint(1, 40000) for _ in range(batches)]
    cu = [0]
    for x in ql:
        cu.append(cu[-1] + x)
    kw = dict(num_heads_q=64, num_heads_kv=1, head_dim=576, batch_size=batches, max_seqlen_q=4,
              max_seqlen_kv=max(kl), layout_q="TND", cu_seqlens_q=torch.tensor(cu, dtype=torch.int32),
              seqused_kv=torch.tensor(kl, dtype=torch.int32), cmp_ratio=4, cmp_topk=512)
    host = sparse_attn_sharedkv_metadata(**kw).tolist()
    got = sparse_attn_sharedkv_metadata(**_on_device(kw))
    assert got.is_cuda and got.dtype == torch.int32
    assert got.cpu().tolist() == host
