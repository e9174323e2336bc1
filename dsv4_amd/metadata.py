"""Drop-in for ``sparse_attn_sharedkv_tilelang/metadata.py``.

Same public names, constants and keyword signature
(metadata.py:38-60, 1018-1045); the schedule is computed by libsas's C++
scheduler (``sas_metadata_v1``), bit-exact with the reference's Python
scheduler, in microseconds instead of milliseconds.

The int32[1024] output is ``fa[36][8] || fd[72][8] || zero pad`` with FA
rows ``(enable, bn2_start, m_start, s2_start, bn2_end, m_end, s2_end,
first_fd_ws)``. The FD rows stay zero: flash-decode splitting is disabled in
the reference scheduler.
"""

from __future__ import annotations

import ctypes as C
from typing import Optional

import torch

from . import _lib

AIC_CORE_NUM = 36
AIV_CORE_NUM = 72
SAS_META_SIZE = 1024
# batches the device scheduler holds (sas_sched.hip: kMaxB); larger batch
# counts take the host scheduler
DEVICE_MAX_BATCHES = 1024

FA_METADATA_SIZE = 8
FD_METADATA_SIZE = 8

FA_CORE_ENABLE_INDEX = 0
FA_BN2_START_INDEX = 1
FA_M_START_INDEX = 2
FA_S2_START_INDEX = 3
FA_BN2_END_INDEX = 4
FA_M_END_INDEX = 5
FA_S2_END_INDEX = 6
FA_FIRST_FD_DATA_WORKSPACE_IDX_INDEX = 7

FD_CORE_ENABLE_INDEX = 0
FD_BN2_IDX_INDEX = 1
FD_M_IDX_INDEX = 2
FD_WORKSPACE_IDX_INDEX = 3
FD_WORKSPACE_NUM_INDEX = 4
FD_M_START_INDEX = 5
FD_M_NUM_INDEX = 6


class SparseMode:
    DEFAULT_MASK = 0
    ALL_MASK = 1
    LEFT_UP_CAUSAL = 2
    RIGHT_DOWN_CAUSAL = 3
    BAND = 4
    SPARSE_BUTT = 5


def _int_array(t):
    """Host int32 copy of an optional tensor / sequence -> (keepalive, ptr, n)."""
    if t is None:
        return None, None, 0
    if isinstance(t, torch.Tensor):
        if t.numel() == 0:
            return None, None, 0
        a = t.detach().reshape(-1).to(device="cpu", dtype=torch.int32).contiguous()
    else:
        vals = [int(x) for x in t]
        if not vals:
            return None, None, 0
        a = torch.tensor(vals, dtype=torch.int32)
    return a, C.cast(a.data_ptr(), C.POINTER(C.c_int32)), a.numel()


def _params(*, num_heads_q, num_heads_kv, head_dim, batch_size, max_seqlen_q, max_seqlen_kv, ori_topk,
            cmp_topk, cmp_ratio, ori_mask_mode, cmp_mask_mode, ori_win_left, ori_win_right, layout_q,
            layout_kv, has_ori_kv, has_cmp_kv, aic_core_num, aiv_core_num, keep) -> _lib.SasMetaParams:
    """The scalar fields of SasMetaParams (the layout strings kept alive in ``keep``)."""
    p = _lib.SasMetaParams()
    p.num_heads_q, p.num_heads_kv, p.head_dim = int(num_heads_q), int(num_heads_kv), int(head_dim)
    p.batch_size, p.max_seqlen_q, p.max_seqlen_kv = int(batch_size), int(max_seqlen_q), int(max_seqlen_kv)
    p.ori_topk, p.cmp_topk, p.cmp_ratio = int(ori_topk), int(cmp_topk), int(cmp_ratio)
    p.ori_mask_mode, p.cmp_mask_mode = int(ori_mask_mode), int(cmp_mask_mode)
    p.ori_win_left, p.ori_win_right = int(ori_win_left), int(ori_win_right)
    lq, lkv = str(layout_q).encode(), str(layout_kv).encode()
    keep += [lq, lkv]
    p.layout_q, p.layout_kv = lq, lkv
    p.has_ori_kv, p.has_cmp_kv = int(bool(has_ori_kv)), int(bool(has_cmp_kv))
    p.aic_core_num, p.aiv_core_num = int(aic_core_num), int(aiv_core_num)
    return p


def _metadata_device(dev, tensors, **scalars) -> torch.Tensor:
    """sas_metadata_device_v1: the lengths stay on ``dev`` (int32 views or
    copies made there), the result is a device tensor; nothing synchronises."""
    keep = []
    p = _params(keep=keep, **scalars)
    names = ("cu_seqlens_q", "cu_seqlens_ori_kv", "cu_seqlens_cmp_kv", "seqused_q", "seqused_kv")
    for name, t in zip(names, tensors):
        n = 0
        if t is not None and t.numel() > 0:
            a = t.detach().reshape(-1).to(dtype=torch.int32).contiguous()
            keep.append(a)
            setattr(p, name, C.cast(a.data_ptr(), C.POINTER(C.c_int32)))
            n = a.numel()
        setattr(p, "n_" + name, n)
    out = torch.empty(SAS_META_SIZE, dtype=torch.int32, device=dev)
    with torch.cuda.device(dev):
        st = torch.cuda.current_stream(dev)
        rc = _lib.lib().sas_metadata_device_v1(C.byref(p), C.c_void_p(out.data_ptr()), C.c_void_p(st.cuda_stream))
        _lib.check(rc, "sparse_attn_sharedkv_metadata")
        # int32 copies made for the launch must outlive it on the stream
        for a in keep:
            if isinstance(a, torch.Tensor):
                a.record_stream(st)
    return out


def _batch_count(layout_q, cu_seqlens_q, seqused_q, batch_size) -> int:
    """The scheduler's batch count from tensor sizes only (no device read):
    seqused_q's length, else cu_seqlens_q's minus one under TND, else
    ``batch_size`` (metadata.py:345-350; the same rule as both entry
    points)."""
    def n(t):
        return 0 if t is None else (t.numel() if isinstance(t, torch.Tensor) else len(t))
    if n(seqused_q) > 0:
        return n(seqused_q)
    if (layout_q or "BSND") == "TND" and n(cu_seqlens_q) > 0:
        return n(cu_seqlens_q) - 1
    return int(batch_size)


def sparse_attn_sharedkv_metadata(
    *,
    num_heads_q: int,
    num_heads_kv: int,
    head_dim: int,
    cu_seqlens_q: Optional[torch.Tensor] = None,
    cu_seqlens_ori_kv: Optional[torch.Tensor] = None,
    cu_seqlens_cmp_kv: Optional[torch.Tensor] = None,
    seqused_q: Optional[torch.Tensor] = None,
    seqused_kv: Optional[torch.Tensor] = None,
    batch_size: int = 0,
    max_seqlen_q: int = 0,
    max_seqlen_kv: int = 0,
    ori_topk: int = 0,
    cmp_topk: int = 0,
    cmp_ratio: int = -1,
    ori_mask_mode: int = 4,
    cmp_mask_mode: int = 3,
    ori_win_left: int = 127,
    ori_win_right: int = 0,
    layout_q: str = "BSND",
    layout_kv: str = "PA_ND",
    has_ori_kv: bool = True,
    has_cmp_kv: bool = True,
    aic_core_num: int = 24,
    aiv_core_num: int = 48,
    device: Optional[str] = None,
) -> torch.Tensor:
    """Return the scheduler's INT32 ``[SAS_META_SIZE]`` tensor (CPU, or on
    ``device`` when given), as metadata.py:1018-1086 does.

    When ``device`` is a GPU, every sequence-length tensor given lives on it
    and the batch count (from the tensors' sizes or ``batch_size``, known
    without reading them) is at most ``DEVICE_MAX_BATCHES``, the schedule is
    computed there (``sas_metadata_device_v1``: one kernel on the current
    stream, no host copy, no synchronisation), bit for bit the host
    schedule; else on the host (``sas_metadata_v1``).

    The device path cannot raise on values it never reads back: where the
    host scheduler raises ``ValueError`` for the lengths given (a row scan
    past a batch's last row that finds no work), or where they exceed the
    device scheduler's own bound (more than 2^22 query rows in all), the
    returned tensor holds ``-1`` in element 0 and zeros elsewhere. Element 0
    of a valid schedule is the first core's enable flag, 0 or 1."""
    tensors = (cu_seqlens_q, cu_seqlens_ori_kv, cu_seqlens_cmp_kv, seqused_q, seqused_kv)
    dev = torch.device(device) if device is not None else None
    if (dev is not None and dev.type == "cuda"
            and _batch_count(layout_q, cu_seqlens_q, seqused_q, batch_size) <= DEVICE_MAX_BATCHES
            and all(isinstance(t, torch.Tensor) for t in tensors if t is not None)
            and any(t is not None for t in tensors)
            and all(t.is_cuda for t in tensors if t is not None)):
        tdev = next(t.device for t in tensors if t is not None)
        if all(t.device == tdev for t in tensors if t is not None) and (dev.index is None or dev.index == tdev.index):
            return _metadata_device(tdev, tensors, num_heads_q=num_heads_q, num_heads_kv=num_heads_kv,
                                    head_dim=head_dim, batch_size=batch_size, max_seqlen_q=max_seqlen_q,
                                    max_seqlen_kv=max_seqlen_kv, ori_topk=ori_topk, cmp_topk=cmp_topk,
                                    cmp_ratio=cmp_ratio, ori_mask_mode=ori_mask_mode,
                                    cmp_mask_mode=cmp_mask_mode, ori_win_left=ori_win_left,
                                    ori_win_right=ori_win_right, layout_q=layout_q, layout_kv=layout_kv,
                                    has_ori_kv=has_ori_kv, has_cmp_kv=has_cmp_kv, aic_core_num=aic_core_num,
                                    aiv_core_num=aiv_core_num)
    keep = []
    p = _params(num_heads_q=num_heads_q, num_heads_kv=num_heads_kv, head_dim=head_dim, batch_size=batch_size,
                max_seqlen_q=max_seqlen_q, max_seqlen_kv=max_seqlen_kv, ori_topk=ori_topk, cmp_topk=cmp_topk,
                cmp_ratio=cmp_ratio, ori_mask_mode=ori_mask_mode, cmp_mask_mode=cmp_mask_mode,
                ori_win_left=ori_win_left, ori_win_right=ori_win_right, layout_q=layout_q, layout_kv=layout_kv,
                has_ori_kv=has_ori_kv, has_cmp_kv=has_cmp_kv, aic_core_num=aic_core_num,
                aiv_core_num=aiv_core_num, keep=keep)
    for name, t in (("cu_seqlens_q", cu_seqlens_q), ("cu_seqlens_ori_kv", cu_seqlens_ori_kv),
                    ("cu_seqlens_cmp_kv", cu_seqlens_cmp_kv), ("seqused_q", seqused_q),
                    ("seqused_kv", seqused_kv)):
        a, ptr, n = _int_array(t)
        keep.append(a)
        if ptr is not None:
            setattr(p, name, ptr)
        setattr(p, "n_" + name, n)
    out = torch.zeros(SAS_META_SIZE, dtype=torch.int32)
    rc = _lib.lib().sas_metadata_v1(C.byref(p), C.cast(out.data_ptr(), C.POINTER(C.c_int32)))
    _lib.check(rc, "sparse_attn_sharedkv_metadata")
    if device is not None:
        out = out.to(device)
    return out
