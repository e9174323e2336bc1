"""ORACLE (test infrastructure only; never imported by the product path).

CPU restatement of the paged-KV cache writer (``sas_cache_write_v1``).

The reference has no cache writer; its tests place rows into paged caches on
the host (sparse_attn_sharedkv_tilelang/golden.py:315-408): row ``pos`` of
batch ``b`` lives in physical block ``table[b, pos // block_size]`` at offset
``pos % block_size``, and ``-1`` marks an unused table entry. This oracle
scatters rows the same way, one row at a time in plain Python, skipping rows
whose position is negative or whose table entry is missing / out of range.

fp8 rows (656 bytes): per 128 latent channels ``scale = amax / 448`` is
stored and ``byte = e4m3fn(clamp(x * inv, -448, 448))`` with
``inv = 448 / amax`` (both 1 for an all-zero group), using torch's own
float -> ``float8_e4m3fn`` conversion (round to nearest even); then the 4
fp32 scales, then the 64 rope channels as bf16.

Pins (tests/test_cache_writer.py): known e4m3fn codes (1.0 -> 0x38, 448 ->
0x7E, 2^-9 -> 0x01, ties 1.0625 -> 1.0 and 1.1875 -> 1.25, -0.0 -> 0x80);
the dequantised row is within half an e4m3 step of the input; a planted
mistake (a scale of amax / 240) fails them; writing every row of dense
sequences and unpacking the cache through the block table returns the rows.
"""

from __future__ import annotations

import torch

ROW656, LATENT, GROUP, SCALE_OFF, ROPE_OFF = 656, 512, 128, 512, 528
E4M3_MAX = 448.0


def quantize_row_fp8(x: torch.Tensor, scale_div: float = E4M3_MAX) -> torch.Tensor:
    """One ``[576]`` row (any float dtype) -> uint8 ``[656]``; ``scale_div``
    exists so a test can plant a wrong divisor."""
    x = x.float()
    out = torch.zeros(ROW656, dtype=torch.uint8)
    scales = torch.empty(LATENT // GROUP, dtype=torch.float32)
    for gi in range(LATENT // GROUP):
        g = x[gi * GROUP:(gi + 1) * GROUP]
        amax = float(g.abs().max())
        a32 = torch.tensor(amax, dtype=torch.float32)
        s = a32 / scale_div if amax > 0 else torch.tensor(1.0)
        # tensor / tensor: one correctly rounded division (torch computes
        # `float / tensor` as reciprocal(tensor) * float, two roundings)
        inv = torch.tensor(scale_div, dtype=torch.float32) / a32 if amax > 0 else torch.tensor(1.0)
        q = (g * inv).clamp(-E4M3_MAX, E4M3_MAX).to(torch.float8_e4m3fn)
        out[gi * GROUP:(gi + 1) * GROUP] = q.view(torch.uint8)
        scales[gi] = s
    out[SCALE_OFF:ROPE_OFF] = scales.view(torch.uint8)
    out[ROPE_OFF:] = x[LATENT:].to(torch.bfloat16).contiguous().view(torch.uint8)
    return out


def write_kv_cache_ref(kv: torch.Tensor, cache: torch.Tensor, block_table: torch.Tensor,
                       seq_ids: torch.Tensor, positions: torch.Tensor) -> torch.Tensor:
    """Returns a copy of ``cache`` (CPU) with ``kv``'s rows written."""
    out = cache.detach().cpu().clone()
    kv = kv.detach().cpu()
    bt = block_table.detach().cpu().tolist()
    nb, bs = out.shape[0], out.shape[1]
    fp8 = out.dtype == torch.uint8
    for r, (b, pos) in enumerate(zip(seq_ids.tolist(), positions.tolist())):
        if b < 0 or b >= len(bt) or pos < 0 or pos // bs >= len(bt[b]):
            continue
        blk = bt[b][pos // bs]
        if blk < 0 or blk >= nb:
            continue
        out[blk, pos % bs, 0] = quantize_row_fp8(kv[r]) if fp8 else kv[r]
    return out
