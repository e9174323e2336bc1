"""Paged-KV cache writer (sas_cache_write_v1): the CPU oracle pinned by known
e4m3fn codes, error bounds and the block-table layout; the GPU kernel
bit-exact against the oracle (fp8 rows and plain copies)."""

from __future__ import annotations

import ctypes as C
import math

import numpy as np
import pytest
import torch

from dsv4_amd import _lib, paged
from oracle import cache_ref as R


def _kat_row():
    """Group 0: amax 448 (scale 1) with known codes; group 1: zeros; group 2:
    amax 896 (scale 2); group 3: random. Returns (row, {index: code})."""
    x = torch.zeros(576)
    vals = {0: (448.0, 0x7E), 1: (1.0, 0x38), 2: (2.0 ** -9, 0x01), 3: (1.0625, 0x38),
            4: (1.1875, 0x3A), 5: (-0.0, 0x80), 6: (-1.0, 0xB8), 7: (2.0 ** -6, 0x08),
            8: (3 * 2.0 ** -10, 0x02)}   # 1.5 x 2^-9: tie between codes 1 and 2 -> 2 (even)
    for i, (v, _) in vals.items():
        x[i] = v
    x[256] = 896.0
    x[257] = 2.0
    x[384:512] = torch.linspace(-3, 3, 128)
    x[512:] = torch.linspace(-1, 1, 64)
    codes = {i: c for i, (_, c) in vals.items()}
    codes.update({128: 0x00, 256: 0x7E, 257: 0x38})
    return x, codes


def _check_kat(row_bytes, codes):
    for i, c in codes.items():
        assert int(row_bytes[i]) == c, f"byte {i}: {int(row_bytes[i]):#x} != {c:#x}"
    sc = row_bytes[R.SCALE_OFF:R.ROPE_OFF].view(torch.float32)
    assert sc.tolist()[:3] == [1.0, 1.0, 2.0]


def test_oracle_known_codes():
    x, codes = _kat_row()
    _check_kat(R.quantize_row_fp8(x), codes)


def test_oracle_planted_wrong_scale_fails():
    x, codes = _kat_row()
    with pytest.raises(AssertionError):
        _check_kat(R.quantize_row_fp8(x, scale_div=240.0), codes)


def test_oracle_error_bound_and_agreement_with_codec():
    g = torch.Generator().manual_seed(3)
    rows = torch.randn(64, 576, generator=g) * torch.logspace(-4, 3, 64).unsqueeze(1)
    rows = rows.to(torch.bfloat16)
    q = torch.stack([R.quantize_row_fp8(r) for r in rows])
    # the product's torch codec writes the same bytes
    assert torch.equal(q, paged.quantize_kv_fp8(rows))
    deq = paged.dequantize_kv_fp8(q)
    x = rows.float()
    lat, dl = x[:, :512].reshape(64, 4, 128), deq[:, :512].reshape(64, 4, 128)
    scale = lat.abs().amax(-1, keepdim=True) / 448.0
    y = lat / scale
    # half a step of e4m3: 2^-4 relative in the normal range, 2^-10 absolute below 2^-6
    bound = torch.where(y.abs() >= 2.0 ** -6, y.abs() * 2.0 ** -4, torch.full_like(y, 2.0 ** -10)) * scale
    assert bool(((dl - lat).abs() <= bound * (1 + 1e-6)).all())
    assert torch.equal(deq[:, 512:], x[:, 512:])   # rope exact


def test_oracle_scatter_follows_block_table_layout():
    """Writing every row of dense sequences and unpacking the paged cache
    through the block table (golden.py:247-268's convention) gives the rows."""
    g = torch.Generator().manual_seed(4)
    lens, bs = [70, 5, 128], 16
    nblk = [math.ceil(n / bs) for n in lens]
    perm = np.random.default_rng(5).permutation(sum(nblk) + 3).astype(np.int32)
    table = torch.full((3, max(nblk)), -1, dtype=torch.int32)
    c = 0
    for b, n in enumerate(nblk):
        table[b, :n] = torch.from_numpy(perm[c:c + n]); c += n
    dense = torch.randn(3, max(lens), 576, generator=g).to(torch.bfloat16)
    sid = torch.cat([torch.full((n,), b, dtype=torch.int32) for b, n in enumerate(lens)])
    pos = torch.cat([torch.arange(n, dtype=torch.int32) for n in lens])
    kv = torch.cat([dense[b, :n] for b, n in enumerate(lens)])
    cache = torch.zeros(len(perm), bs, 1, 576, dtype=torch.bfloat16)
    out = R.write_kv_cache_ref(kv, cache, table, sid, pos)
    back = paged.unpack_paged_kv(out, table, max(lens))
    for b, n in enumerate(lens):
        assert torch.equal(back[b, 0, :n], dense[b, :n])


def test_abi_rejects_bad_arguments():
    L = _lib.lib()
    a = _lib.SasCacheWriteArgs(N=0, B=1, D=576, kv_stride=576, bt_stride=1, block_size=64, num_blocks=1,
                               kv_dtype=_lib.SAS_DT_BF16, cache_dtype=_lib.SAS_DT_BF16)
    assert L.sas_cache_write_v1(C.byref(a), None) == _lib.SAS_OK          # nothing to write
    a.N = 4
    assert L.sas_cache_write_v1(C.byref(a), None) == _lib.SAS_EINVAL      # null pointers
    fake = 1 << 20
    a.kv = a.seq_ids = a.positions = a.block_table = a.cache = fake
    a.cache_dtype = _lib.SAS_DT_FP8_E4M3_ROW656
    a.kv_dtype = _lib.SAS_DT_FP16
    assert L.sas_cache_write_v1(C.byref(a), None) == _lib.SAS_EINVAL      # fp8 rows need bf16 kv
    assert "bf16" in L.sas_last_error().decode()
    a.kv_dtype, a.D, a.kv_stride = _lib.SAS_DT_BF16, 512, 512
    assert L.sas_cache_write_v1(C.byref(a), None) == _lib.SAS_EINVAL      # fp8 rows need D = 576
    assert L.sas_cache_write_v1(None, None) == _lib.SAS_EINVAL


# ---------------------------------------------------------------------------
# GPU: the kernel against the oracle, bit for bit
# ---------------------------------------------------------------------------

def _case(dtype, fp8, N=600, B=4, bs=64, seed=7):
    g = torch.Generator().manual_seed(seed)
    maxblk = 6
    nb = B * maxblk + 5
    perm = torch.randperm(nb, generator=g)[:B * maxblk].to(torch.int32)
    table = perm.reshape(B, maxblk).clone()
    table[1, 3] = -1                                   # an unused table entry
    table[2, 5] = nb + 9                               # an out-of-range entry (skipped)
    # distinct (batch, position) targets, some skipped by position or table
    flat = torch.randperm(B * maxblk * bs, generator=g)[:N]
    sid = (flat // (maxblk * bs)).to(torch.int32)
    pos = (flat % (maxblk * bs)).to(torch.int32)
    pos[::37] = -1
    kv = torch.randn(N, 576, generator=g) * torch.logspace(-3, 2, N).unsqueeze(1)
    kv[5, :128] = 0.0                                  # an all-zero group
    kv[6, 128:256] = 1e-30                             # tiny values: subnormal codes / zeros
    kv[7, 256:384] = -3.0e35                           # huge values (within bf16)
    kv[8, 0] = -0.0
    kv = kv.to(dtype)
    row = 656 if fp8 else 576
    cdt = torch.uint8 if fp8 else dtype
    cache = torch.randint(0, 255, (nb, bs, 1, row * (1 if fp8 else 2)), generator=g, dtype=torch.uint8)
    cache = cache if fp8 else cache.view(cdt)
    return kv, cache, table, sid, pos


@pytest.mark.gpu
@pytest.mark.parametrize("mode", ["fp8", "bf16", "fp16"])
def test_gpu_cache_write_matches_oracle(mode):
    from dsv4_amd.cache import write_kv_cache
    fp8 = mode == "fp8"
    dtype = torch.float16 if mode == "fp16" else torch.bfloat16
    kv, cache, table, sid, pos = _case(dtype, fp8)
    ref = R.write_kv_cache_ref(kv, cache, table, sid, pos)
    d = cache.cuda()
    write_kv_cache(kv.cuda(), d, table.cuda(), sid.cuda(), pos.cuda())
    torch.cuda.synchronize()
    got = d.cpu()
    assert torch.equal(got.view(torch.uint8), ref.view(torch.uint8)), \
        f"{int((got.view(torch.uint8) != ref.view(torch.uint8)).sum())} bytes differ"


def every_bf16_rows():
    """Every bf16 value with |v| <= 448 (both signs, zeros, subnormals), 127
    per 128-channel group next to a 448 that makes inv = 1, so the quantiser
    sees each value exactly: an exhaustive check of the e4m3 rounding."""
    bits = torch.arange(0, 1 << 16, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
    v = bits.float()
    v = v[torch.isfinite(v) & (v.abs() <= 448.0)]
    per = 127
    n = (v.numel() + 4 * per - 1) // (4 * per)
    pad = torch.zeros(n * 4 * per - v.numel())
    body = torch.cat([v, pad]).reshape(n, 4, per)
    lat = torch.cat([torch.full((n, 4, 1), 448.0), body], dim=2).reshape(n, 512)
    return torch.cat([lat, torch.zeros(n, 64)], dim=1).to(torch.bfloat16)


@pytest.mark.gpu
def test_gpu_cache_write_every_bf16_value():
    from dsv4_amd.cache import write_kv_cache
    kv = every_bf16_rows()
    N = kv.shape[0]
    table = torch.arange(N, dtype=torch.int32).reshape(N, 1)
    sid = torch.arange(N, dtype=torch.int32)
    pos = torch.zeros(N, dtype=torch.int32)
    cache = torch.zeros(N, 1, 1, 656, dtype=torch.uint8)
    ref = R.write_kv_cache_ref(kv, cache, table, sid, pos)
    d = cache.cuda()
    write_kv_cache(kv.cuda(), d, table.cuda(), sid.cuda(), pos.cuda())
    torch.cuda.synchronize()
    got = d.cpu()
    assert torch.equal(got, ref), f"{int((got != ref).sum())} bytes differ"


@pytest.mark.gpu
def test_gpu_cache_write_strided_rows_and_empty_call():
    """kv rows with a row stride wider than D (a column slice of a larger
    tensor); N = 0 is a no-op."""
    from dsv4_amd.cache import write_kv_cache
    kv, cache, table, sid, pos = _case(torch.bfloat16, True, N=64, seed=9)
    wide = torch.zeros(64, 640, dtype=torch.bfloat16)
    wide[:, :576] = kv
    ref = R.write_kv_cache_ref(kv, cache, table, sid, pos)
    d = cache.cuda()
    dw = wide.cuda()
    write_kv_cache(dw[:, :576], d, table.cuda(), sid.cuda(), pos.cuda())
    write_kv_cache(dw[:0, :576], d, table.cuda(), sid.cuda()[:0], pos.cuda()[:0])
    torch.cuda.synchronize()
    assert torch.equal(d.cpu(), ref)


@pytest.mark.gpu
def test_gpu_cache_write_int64_indices_on_a_side_stream():
    """int64 seq_ids / positions (converted on the current stream) with the
    kernel launched on another stream: the launch waits for the conversions,
    and the converted temporaries stay allocated until it has run (the
    current stream's next allocations cannot reuse them meanwhile)."""
    from dsv4_amd.cache import write_kv_cache
    kv, cache, table, sid, pos = _case(torch.bfloat16, True, N=600, seed=11)
    ref = R.write_kv_cache_ref(kv, cache, table, sid, pos)
    d = cache.cuda()
    dkv, dt = kv.cuda(), table.cuda().to(torch.int64)
    dsid, dpos = sid.cuda().to(torch.int64), pos.cuda().to(torch.int64)
    side = torch.cuda.Stream()
    torch.cuda.synchronize()
    torch.cuda._sleep(2_000_000)            # the current stream is busy when the conversions queue
    write_kv_cache(dkv, d, dt, dsid, dpos, stream=side)
    junk = [torch.full((600,), -7, dtype=torch.int32, device="cuda") for _ in range(8)]
    side.synchronize()
    torch.cuda.synchronize()
    del junk
    assert torch.equal(d.cpu(), ref), f"{int((d.cpu() != ref).sum())} bytes differ"
