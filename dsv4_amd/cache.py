"""Paged-KV cache writer: new latent KV rows -> the paged cache the forward
reads, through the same block tables.

The reference builds its paged caches on the host in its tests
(sparse_attn_sharedkv_tilelang/golden.py:315-408): row ``pos`` of batch ``b``
is stored in physical block ``block_table[b, pos // block_size]`` at offset
``pos % block_size``; ``-1`` marks an unused table entry. This module writes
rows into that layout on the GPU with ``sas_cache_write_v1``, either as a
bf16/fp16 copy or quantised into the 656-byte fp8 rows of
:mod:`dsv4_amd.paged` (``quantize_kv_fp8``'s format and rounding, bit for bit).
"""

from __future__ import annotations

import ctypes as C
from typing import Optional

import torch

from . import _lib

_DT = {torch.bfloat16: _lib.SAS_DT_BF16, torch.float16: _lib.SAS_DT_FP16}
FP8_ROW_BYTES = 656


class PreparedCacheWrite:
    """Arguments of one cache write, validated once; :meth:`launch` runs the
    kernel on the current (or given) stream without host syncs."""

    def __init__(self, args: _lib.SasCacheWriteArgs, keep: list, device):
        self.args = args
        self._keep = keep
        self.device = device
        # the int32 / contiguous conversions were enqueued on this stream
        self._prep_stream = torch.cuda.current_stream(device)

    def launch(self, stream: Optional[torch.cuda.Stream] = None) -> None:
        st = stream if stream is not None else torch.cuda.current_stream(self.device)
        if st != self._prep_stream:
            # order the launch after the conversions, and keep every bound
            # tensor's memory from being reused by the caching allocator on
            # its own stream while the kernel on `st` may still touch it
            ev = torch.cuda.Event()
            ev.record(self._prep_stream)
            st.wait_event(ev)
            for t in self._keep:
                t.record_stream(st)
        _lib.check(_lib.lib().sas_cache_write_v1(C.byref(self.args), C.c_void_p(st.cuda_stream)),
                   "write_kv_cache")


def prepare_kv_cache_write(kv: torch.Tensor, cache: torch.Tensor, block_table: torch.Tensor,
                           seq_ids: torch.Tensor, positions: torch.Tensor) -> PreparedCacheWrite:
    """Validate the arguments of :func:`write_kv_cache` and bind them."""
    if kv.dim() != 2:
        raise ValueError(f"kv must be [N, D], got {tuple(kv.shape)}")
    if kv.dtype not in _DT:
        raise ValueError(f"kv dtype must be bf16 or fp16, got {kv.dtype}")
    if cache.dim() != 4 or cache.shape[2] != 1:
        raise ValueError(f"cache must be [num_blocks, block_size, 1, row], got {tuple(cache.shape)}")
    N, D = kv.shape
    fp8 = cache.dtype == torch.uint8
    if fp8:
        if cache.shape[-1] != FP8_ROW_BYTES or kv.dtype != torch.bfloat16 or D != 576:
            raise ValueError("fp8 cache rows need uint8 [..., 656] and bf16 kv with D = 576")
    elif cache.dtype != kv.dtype or cache.shape[-1] != D:
        raise ValueError("cache must hold rows of kv's dtype and width, or uint8 fp8 rows")
    if block_table.dim() != 2:
        raise ValueError("block_table must be [B, max_blocks]")
    for name, t in (("seq_ids", seq_ids), ("positions", positions)):
        if t.shape != (N,):
            raise ValueError(f"{name} must be [N] = [{N}], got {tuple(t.shape)}")
    dev = kv.device
    if any(t.device != dev for t in (cache, block_table, seq_ids, positions)):
        raise ValueError("all tensors must be on kv's device")
    if kv.stride(1) != 1 or not cache.is_contiguous():
        raise ValueError("kv rows and cache must be contiguous")
    bt = block_table.to(torch.int32).contiguous()
    sid = seq_ids.to(torch.int32).contiguous()
    pos = positions.to(torch.int32).contiguous()
    a = _lib.SasCacheWriteArgs(
        kv=kv.data_ptr(), seq_ids=sid.data_ptr(), positions=pos.data_ptr(),
        block_table=bt.data_ptr(), cache=cache.data_ptr(),
        N=N, B=bt.shape[0], D=D, kv_stride=kv.stride(0), bt_stride=bt.shape[1],
        block_size=cache.shape[1], num_blocks=cache.shape[0],
        kv_dtype=_DT[kv.dtype], cache_dtype=_lib.SAS_DT_FP8_E4M3_ROW656 if fp8 else _DT[kv.dtype])
    return PreparedCacheWrite(a, [kv, cache, bt, sid, pos], dev)


def write_kv_cache(kv: torch.Tensor, cache: torch.Tensor, block_table: torch.Tensor,
                   seq_ids: torch.Tensor, positions: torch.Tensor,
                   stream: Optional[torch.cuda.Stream] = None) -> None:
    """Scatter ``kv [N, D]`` into ``cache`` on the GPU (no host sync).

    ``cache`` is ``[num_blocks, block_size, 1, D]`` in ``kv``'s dtype (rows
    copied) or uint8 ``[num_blocks, block_size, 1, 656]`` (bf16 ``kv`` with
    D = 576, quantised to fp8 rows). ``seq_ids`` / ``positions`` (int32
    ``[N]``) give each row's batch and logical position; rows whose position
    is negative, or whose block-table entry is -1 or missing, are skipped.
    The rows of one call must go to distinct cache rows.
    """
    prepare_kv_cache_write(kv, cache, block_table, seq_ids, positions).launch(stream)
