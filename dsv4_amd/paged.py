"""Paged shared-KV caches, sparse-index generators, layout converters and the
fp8-e4m3 cache row codec.

Paging convention (golden.py:315-408): a cache is ``[block_num, block_size,
N2, D]``; a per-batch block table ``[B, table_len]`` int32 maps logical block
``i`` of sequence ``b`` to a physical block, ``-1`` marking unused slots.
Logical row ``g`` of sequence ``b`` lives at
``cache[table[b, g // block_size], g % block_size]``.

Sparse indices (golden.py:411-473) are prefix-valid per query row: the first
``min(K, threshold)`` slots hold distinct compressed positions below the
row's causal threshold ``floor((act_kv - act_q + s + 1) / cmp_ratio)`` and the
rest are ``-1``.

fp8 cache rows (no counterpart in the reference, which has no quantised
path; TEST_SETUP.md:401): one 656-byte row per token::

    bytes [0, 512)    512 latent channels, float8 e4m3fn
    bytes [512, 528)  4 float32 dequant scales, one per 128 latent channels
    bytes [528, 656)  64 rope channels, bfloat16 (kept unquantised)

``value = e4m3(byte) * scale[channel // 128]`` for the latent part. The row
is a multiple of 16 bytes so a gather moves it with 41 aligned 16-byte loads.
"""

from __future__ import annotations

import math
from typing import Optional, Sequence

import numpy as np
import torch

FP8_ROW_BYTES = 656
FP8_LATENT = 512
FP8_GROUP = 128
FP8_NGROUPS = FP8_LATENT // FP8_GROUP
FP8_SCALE_OFF = 512
FP8_ROPE_OFF = 528
FP8_ROPE = 64
E4M3_MAX = 448.0


# ---------------------------------------------------------------------------
# Reference-compatible generators (uniform data, numpy-permuted block tables)
# ---------------------------------------------------------------------------


def gen_ori_kv_paged(
    *,
    B: int,
    N2: int,
    D: int,
    block_num: int,
    block_size: int,
    seqused_kv: Sequence[int],
    dtype: torch.dtype,
    data_range: tuple = (-10, 10),
    rng: Optional[np.random.Generator] = None,
):
    """Paged raw KV + block table + dense BNSD copy (golden.py:315-360).

    Same call order of the random sources as the reference generator
    (``torch.rand`` for data, then ``rng.permutation`` for the table), so
    with the same seeds it produces the same tensors.
    """
    rng = rng if rng is not None else np.random.default_rng(0)
    max_s = max(seqused_kv)
    lo, hi = data_range
    dense = (torch.rand((B, N2, max_s, D)) * (hi - lo) + lo).to(dtype)
    nblk = [math.ceil(s / block_size) for s in seqused_kv]
    if block_num < sum(nblk):
        raise ValueError(f"ori block_num too small: {block_num} < {sum(nblk)}")
    table = _table_from_perm(rng.permutation(block_num).astype(np.int32), nblk,
                             math.ceil(max_s / block_size))
    pa = torch.zeros((block_num, block_size, N2, D), dtype=dtype)
    _scatter_dense(pa, table, dense, [max_s] * B, nblk)
    return pa, torch.from_numpy(table), dense


def gen_cmp_kv_paged(
    *,
    B: int,
    N2: int,
    D: int,
    block_num: int,
    block_size: int,
    seqused_kv: Sequence[int],
    cmp_ratio: int,
    dtype: torch.dtype,
    data_range: tuple = (-5, 10),
    rng: Optional[np.random.Generator] = None,
):
    """Paged compressed KV (``floor(act_kv / cmp_ratio)`` rows per sequence),
    its block table, dense copy and per-sequence lengths (golden.py:363-408)."""
    rng = rng if rng is not None else np.random.default_rng(1)
    cmp_seqs = [s // cmp_ratio for s in seqused_kv]
    max_cmp = max(cmp_seqs) if cmp_seqs else 0
    lo, hi = data_range
    dense = (torch.rand((B, N2, max(max_cmp, 1), D)) * (hi - lo) + lo).to(dtype)
    nblk = [math.ceil(s / block_size) if s > 0 else 0 for s in cmp_seqs]
    if block_num < max(sum(nblk), 1):
        raise ValueError(f"cmp block_num too small: {block_num} < {sum(nblk)}")
    width = max(math.ceil(max_cmp / block_size) if max_cmp > 0 else 1, 1)
    table = _table_from_perm(rng.permutation(block_num).astype(np.int32), nblk, width)
    pa = torch.zeros((block_num, block_size, N2, D), dtype=dtype)
    _scatter_dense(pa, table, dense, cmp_seqs, nblk)
    return pa, torch.from_numpy(table), dense, cmp_seqs


def _table_from_perm(perm: np.ndarray, nblk: Sequence[int], width: int) -> np.ndarray:
    table = np.full((len(nblk), width), -1, dtype=np.int32)
    cur = 0
    for b, n in enumerate(nblk):
        table[b, :n] = perm[cur:cur + n]
        cur += n
    return table


def _scatter_dense(pa, table, dense, lens, nblk):
    bs = pa.shape[1]
    for b in range(len(nblk)):
        for i in range(nblk[b]):
            s0 = i * bs
            s1 = min(s0 + bs, lens[b])
            if s1 > s0:
                pa[int(table[b, i]), : s1 - s0] = dense[b, :, s0:s1, :].permute(1, 0, 2)


def gen_cmp_sparse_indices_tnd(
    *,
    B: int,
    T1: int,
    N2: int,
    K: int,
    cu_seqlens_q: torch.Tensor,
    seqused_kv: Sequence[int],
    cmp_ratio: int,
    cmp_mask_mode: int = 3,
    rng: Optional[torch.Generator] = None,
) -> torch.Tensor:
    """Prefix-valid random top-k indices per packed query row
    (golden.py:442-473): ``randperm(threshold)[:min(threshold, K)]`` then -1."""
    if cmp_mask_mode != 3:
        raise ValueError("only cmp_mask_mode=3 supported")
    out = torch.full((T1, N2, K), -1, dtype=torch.int32)
    cu = [int(x) for x in cu_seqlens_q.tolist()]
    for b in range(B):
        act_q = cu[b + 1] - cu[b]
        act_kv = int(seqused_kv[b])
        for n2 in range(N2):
            for s in range(act_q):
                thr = max(0, (act_kv - act_q + s + 1) // cmp_ratio)
                if thr > 0:
                    perm = torch.randperm(thr, generator=rng).to(torch.int32)
                    take = min(thr, K)
                    out[cu[b] + s, n2, :take] = perm[:take]
    return out


def gen_cmp_sparse_indices_bsnd(
    *,
    B: int,
    S1: int,
    N2: int,
    K: int,
    seqused_kv: Sequence[int],
    cmp_ratio: int,
    cmp_mask_mode: int = 3,
    rng: Optional[torch.Generator] = None,
) -> torch.Tensor:
    """BSND twin of :func:`gen_cmp_sparse_indices_tnd` (golden.py:411-439)."""
    if cmp_mask_mode != 3:
        raise ValueError("only cmp_mask_mode=3 supported")
    out = torch.full((B, S1, N2, K), -1, dtype=torch.int32)
    for b in range(B):
        act_kv = int(seqused_kv[b])
        for n2 in range(N2):
            for s in range(S1):
                thr = max(0, (act_kv - S1 + s + 1) // cmp_ratio)
                if thr > 0:
                    perm = torch.randperm(thr, generator=rng).to(torch.int32)
                    take = min(thr, K)
                    out[b, s, n2, :take] = perm[:take]
    return out


# ---------------------------------------------------------------------------
# Layout converters (golden.py:247-312)
# ---------------------------------------------------------------------------


def unpack_paged_kv(kv_pa: torch.Tensor, block_table: torch.Tensor, max_len: int):
    """Paged ``[nb, bs, N2, D]`` -> dense ``[B, N2, max_len, D]``."""
    _, bs, n2, d = kv_pa.shape
    B = block_table.shape[0]
    out = kv_pa.new_zeros((B, n2, max_len, d))
    bt = block_table.tolist()
    for b in range(B):
        for i, phys in enumerate(bt[b]):
            start = i * bs
            if start >= max_len:
                break
            if phys < 0:
                continue
            end = min(start + bs, max_len)
            out[b, :, start:end] = kv_pa[phys, : end - start].permute(1, 0, 2)
    return out


def tnd_to_bnsd_q(q_tnd: torch.Tensor, cu_seqlens_q: torch.Tensor) -> torch.Tensor:
    cu = [int(x) for x in cu_seqlens_q.tolist()]
    lens = [cu[i + 1] - cu[i] for i in range(len(cu) - 1)]
    T, N, D = q_tnd.shape
    out = q_tnd.new_zeros((len(lens), N, max(lens) if lens else 0, D))
    for b, L in enumerate(lens):
        out[b, :, :L] = q_tnd[cu[b]:cu[b] + L].permute(1, 0, 2)
    return out


def bnsd_to_tnd_out(out_bnsd: torch.Tensor, cu_seqlens_q: torch.Tensor) -> torch.Tensor:
    cu = [int(x) for x in cu_seqlens_q.tolist()]
    B, N, _, D = out_bnsd.shape
    out = out_bnsd.new_zeros((cu[-1], N, D))
    for b in range(B):
        L = cu[b + 1] - cu[b]
        out[cu[b]:cu[b] + L] = out_bnsd[b, :, :L].permute(1, 0, 2)
    return out


def bnsd_to_tnd_lse(lse_bnsd: torch.Tensor, cu_seqlens_q: torch.Tensor) -> torch.Tensor:
    cu = [int(x) for x in cu_seqlens_q.tolist()]
    B, N, _ = lse_bnsd.shape
    out = lse_bnsd.new_zeros((cu[-1], N))
    for b in range(B):
        L = cu[b + 1] - cu[b]
        out[cu[b]:cu[b] + L] = lse_bnsd[b, :, :L].permute(1, 0)
    return out


# ---------------------------------------------------------------------------
# Large-scale generators (normal data, torch-permuted tables, any device)
# ---------------------------------------------------------------------------


def random_block_table(seqlens: Sequence[int], block_size: int, gen: torch.Generator,
                       extra_blocks: int = 0, shuffle: bool = True):
    """Block table for ``seqlens`` over a pool of ``sum(blocks)+extra`` physical
    blocks; physical ids are a permutation of the pool (identity if not
    ``shuffle``). Returns ``(table int32 [B, width], block_num)``."""
    nblk = [(s + block_size - 1) // block_size for s in seqlens]
    block_num = max(sum(nblk) + extra_blocks, 1)
    if shuffle:
        perm = torch.randperm(block_num, generator=gen).to(torch.int32).numpy()
    else:
        perm = np.arange(block_num, dtype=np.int32)
    width = max(max(nblk) if nblk else 1, 1)
    return torch.from_numpy(_table_from_perm(perm, nblk, width)), block_num


def fill_normal(shape, dtype, gen: torch.Generator, device) -> torch.Tensor:
    """N(0,1) data in ``dtype``, drawn in fp32 on ``gen``'s device."""
    out = torch.empty(shape, dtype=dtype, device=device)
    flat = out.view(-1)
    step = 1 << 26
    for i in range(0, flat.numel(), step):
        n = min(step, flat.numel() - i)
        flat[i:i + n] = torch.randn(n, generator=gen, device=device).to(dtype)
    return out


# ---------------------------------------------------------------------------
# fp8-e4m3 cache rows
# ---------------------------------------------------------------------------


def quantize_kv_fp8(kv: torch.Tensor) -> torch.Tensor:
    """Pack ``[..., 576]`` KV rows (latent 512 + rope 64) into 656-byte rows.

    Per 128-channel group: ``scale = amax / 448`` is stored and
    ``byte = e4m3fn(clamp(x * inv, -448, 448))`` with ``inv = 448 / amax``
    (both 1 for an all-zero group), rounded to nearest even: one division per
    group, a multiply per value (the device writer computes the same fp32
    products, so both write the same bytes).
    """
    if kv.shape[-1] != FP8_LATENT + FP8_ROPE:
        raise ValueError(f"fp8 rows need 576 channels, got {kv.shape[-1]}")
    lead = kv.shape[:-1]
    x = kv.reshape(-1, FP8_LATENT + FP8_ROPE).float()
    lat = x[:, :FP8_LATENT].reshape(-1, FP8_NGROUPS, FP8_GROUP)
    amax = lat.abs().amax(dim=-1)
    nz = amax > 0
    scale = torch.where(nz, amax / E4M3_MAX, torch.ones_like(amax))
    # a tensor / tensor division (correctly rounded, as on the device); torch
    # evaluates `scalar / tensor` as reciprocal(tensor) * scalar
    inv = torch.where(nz, torch.full_like(amax, E4M3_MAX).div(torch.where(nz, amax, torch.ones_like(amax))),
                      torch.ones_like(amax))
    q8 = (lat * inv.unsqueeze(-1)).clamp(-E4M3_MAX, E4M3_MAX).to(torch.float8_e4m3fn)
    rows = torch.empty((x.shape[0], FP8_ROW_BYTES), dtype=torch.uint8, device=kv.device)
    rows[:, :FP8_LATENT] = q8.reshape(-1, FP8_LATENT).view(torch.uint8)
    rows[:, FP8_SCALE_OFF:FP8_ROPE_OFF] = scale.contiguous().view(torch.uint8).reshape(-1, 16)
    rope = x[:, FP8_LATENT:].to(torch.bfloat16).contiguous()
    rows[:, FP8_ROPE_OFF:] = rope.view(torch.uint8).reshape(-1, 2 * FP8_ROPE)
    return rows.reshape(*lead, FP8_ROW_BYTES)


def dequantize_kv_fp8(rows: torch.Tensor) -> torch.Tensor:
    """Inverse of :func:`quantize_kv_fp8`: 656-byte rows -> fp32 ``[..., 576]``."""
    if rows.dtype != torch.uint8 or rows.shape[-1] != FP8_ROW_BYTES:
        raise ValueError("expected uint8 rows of 656 bytes")
    lead = rows.shape[:-1]
    r = rows.reshape(-1, FP8_ROW_BYTES)
    lat = r[:, :FP8_LATENT].contiguous().view(torch.float8_e4m3fn).float()
    scale = r[:, FP8_SCALE_OFF:FP8_ROPE_OFF].contiguous().view(torch.float32)
    lat = (lat.reshape(-1, FP8_NGROUPS, FP8_GROUP) * scale.unsqueeze(-1)).reshape(-1, FP8_LATENT)
    rope = r[:, FP8_ROPE_OFF:].contiguous().view(torch.bfloat16).float()
    return torch.cat([lat, rope], dim=-1).reshape(*lead, FP8_LATENT + FP8_ROPE)
