"""Drop-in for ``sparse_attn_sharedkv_tilelang/api.py``: ``sparse_attn_sharedkv``.

Same signature, argument meaning, scenario routing and return convention as
api.py:129-397; the computation runs in libsas's gfx950 HIP kernels.

Scenario (api.py:196-202): ``cmp_kv is None`` -> SWA (window only);
``cmp_sparse_indices is None`` -> CFA (window + every compressed row below
the causal threshold); otherwise SCFA (window + top-k compressed rows).

Relaxations of the reference's shape guard (api.py:279-282), which are not
signature changes: the query head count may be any multiple of 16; the
head dim may be 512 or 576 (576 = 512 latent + 64 rope; the output and V are
the first 512 channels, so ``out`` is ``[..., 512]``); any top-k width; any
block size; and an fp8 cache given as uint8 ``[num_blocks, block_size, 1,
656]`` rows (see :mod:`dsv4_amd.paged`) with a bf16 query.

``metadata`` is validated (int32, 1024 entries). The GPU kernel does not
need it for scheduling: it launches one workgroup per (token, head group,
KV split) and covers every valid token by construction; an omitted one is
built with the bit-exact scheduler on request (:meth:`PreparedCall.metadata`).

Host cost of a call: the argument resolution (routing, checks, launch
arguments, split plan) is cached per call signature (shapes, dtypes, device
pointers, scalars, stream), so a repeated call allocates ``out`` / ``lse``,
copies host-side sequence lengths through a reused pinned buffer, and
launches. Device ``cu_seqlens_q`` is passed to the kernel as it is.
"""

from __future__ import annotations

import ctypes as C
import threading
from collections import OrderedDict
from typing import Optional, Tuple, Union

import torch

from . import _lib
from .metadata import SAS_META_SIZE, sparse_attn_sharedkv_metadata

DEFAULT_CORE_NUM = 24
_DT = {torch.bfloat16: _lib.SAS_DT_BF16, torch.float16: _lib.SAS_DT_FP16}
FP8_ROW_BYTES = 656


# ---------------------------------------------------------------------------
# per-call helpers: pinned staging of host int32 arrays, workspaces
# ---------------------------------------------------------------------------

class _Staging:
    """A ring of pinned host slots for the small int32 arrays a call copies
    to the device (host-side sequence lengths), so no call pins memory. A
    slot is reused only after the copy that last read it has completed."""

    SLOTS, SLOT_INTS = 64, 8192

    def __init__(self):
        self.buf = torch.empty(self.SLOTS * self.SLOT_INTS, dtype=torch.int32, pin_memory=True)
        self.events = [torch.cuda.Event() for _ in range(self.SLOTS)]
        self.used = [False] * self.SLOTS
        self.next = 0
        self.lock = threading.Lock()

    def to_device(self, parts, device, stream) -> torch.Tensor:
        """Concatenation of ``parts`` (host int32 tensors) as a new device
        tensor, copied on ``stream`` without blocking the host."""
        n = sum(int(t.numel()) for t in parts)
        if n > self.SLOT_INTS:
            return torch.cat([t.reshape(-1) for t in parts]).to(device)
        with self.lock:
            slot = self.next
            self.next = (slot + 1) % self.SLOTS
            ev = self.events[slot]
            if self.used[slot]:
                ev.synchronize()
            host = self.buf[slot * self.SLOT_INTS: slot * self.SLOT_INTS + n]
            if len(parts) == 1:
                host.copy_(parts[0].reshape(-1))
            else:
                torch.cat([t.reshape(-1) for t in parts], out=host)
            dev = torch.empty(n, dtype=torch.int32, device=device)
            if stream == torch.cuda.current_stream(device):
                dev.copy_(host, non_blocking=True)
            else:
                with torch.cuda.stream(stream):
                    dev.copy_(host, non_blocking=True)
            ev.record(stream)
            self.used[slot] = True
        return dev


_staging = None
_staging_lock = threading.Lock()


def _stage(parts, device, stream) -> torch.Tensor:
    global _staging
    if _staging is None:
        with _staging_lock:
            if _staging is None:
                _staging = _Staging()
    return _staging.to_device(parts, device, stream)


def _raw_stream(dev: torch.device) -> int:
    """The current stream of ``dev`` as a hipStream_t value (no Stream object)."""
    f = getattr(torch._C, "_cuda_getCurrentRawStream", None)
    if f is not None:
        return int(f(dev.index if dev.index is not None else torch.cuda.current_device()))
    return torch.cuda.current_stream(dev).cuda_stream


def _hip_check(rc: int, what: str) -> None:
    if rc != 0:
        raise RuntimeError(f"{what} failed (hipError {rc})")


def _hip_runtime():
    """The HIP runtime entry points of the library libsas.so runs on (the
    runtime torch loaded), resolved through libsas's handle."""
    L = _lib.lib()
    if not getattr(L, "_sas_hip_bound", False):
        L.hipMemcpyAsync.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int, C.c_void_p]
        L.hipMemcpyAsync.restype = C.c_int
        L.hipEventCreateWithFlags.argtypes = [C.POINTER(C.c_void_p), C.c_uint]
        L.hipEventCreateWithFlags.restype = C.c_int
        L.hipEventRecord.argtypes = [C.c_void_p, C.c_void_p]
        L.hipEventRecord.restype = C.c_int
        L.hipEventSynchronize.argtypes = [C.c_void_p]
        L.hipEventSynchronize.restype = C.c_int
        L._sas_hip_bound = True
    return L


class _SeqlenRing:
    """Host-side sequence lengths of the drop-in call reach the device
    through two rings of SLOTS slots per device: pinned host memory, filled
    with memmove, and device memory, filled by one hipMemcpyAsync on the
    call's stream; no tensor is created per call. A slot is handed out again
    once the event recorded after the launch that read it (so after its copy
    and its kernels) has completed; a slot between its copy and that record
    is skipped."""

    SLOTS, SLOT_INTS = 64, 1024
    FREE, PENDING, RECORDED = 0, 1, 2

    def __init__(self, device: torch.device):
        self.host = torch.empty(self.SLOTS * self.SLOT_INTS, dtype=torch.int32, pin_memory=True)
        self.dev = torch.empty(self.SLOTS * self.SLOT_INTS, dtype=torch.int32, device=device)
        self.hbase, self.dbase = self.host.data_ptr(), self.dev.data_ptr()
        self.hip = _hip_runtime()
        self.events = []
        with torch.cuda.device(device):
            for _ in range(self.SLOTS):
                ev = C.c_void_p()
                _hip_check(self.hip.hipEventCreateWithFlags(C.byref(ev), 2), "hipEventCreateWithFlags")
                self.events.append(ev)
        self.state = [self.FREE] * self.SLOTS
        self.next = 0
        self.lock = threading.Lock()

    def stage(self, parts, stream_ptr: int):
        """Copy the host int32 arrays ``parts`` ((address, count) pairs) into
        one device slot on the stream. Returns (device address, slot), or
        None when they do not fit a slot or every slot is pending."""
        n = sum(cnt for _, cnt in parts)
        if n > self.SLOT_INTS:
            return None
        with self.lock:
            for _ in range(self.SLOTS):
                slot = self.next
                self.next = (slot + 1) % self.SLOTS
                if self.state[slot] != self.PENDING:
                    break
            else:
                return None
            if self.state[slot] == self.RECORDED:
                _hip_check(self.hip.hipEventSynchronize(self.events[slot]), "hipEventSynchronize")
            self.state[slot] = self.PENDING
        off = slot * self.SLOT_INTS * 4
        o = 0
        for addr, cnt in parts:
            C.memmove(self.hbase + off + o, addr, 4 * cnt)
            o += 4 * cnt
        rc = self.hip.hipMemcpyAsync(self.dbase + off, self.hbase + off, 4 * n, 1, stream_ptr)
        if rc != 0:
            with self.lock:
                self.state[slot] = self.FREE
            _hip_check(rc, "hipMemcpyAsync")
        return self.dbase + off, slot

    def release(self, slot: int, stream_ptr: int) -> None:
        """After the launch that reads the slot: its reuse waits for this."""
        rc = self.hip.hipEventRecord(self.events[slot], stream_ptr)
        with self.lock:
            self.state[slot] = self.RECORDED if rc == 0 else self.FREE
        _hip_check(rc, "hipEventRecord")


_rings = {}
_rings_lock = threading.Lock()


def _seqlen_ring(dev: torch.device) -> _SeqlenRing:
    key = dev.index
    ring = _rings.get(key)
    if ring is None:
        with _rings_lock:
            ring = _rings.get(key)
            if ring is None:
                ring = _rings[key] = _SeqlenRing(dev)
    return ring


# split-KV workspaces, one growing buffer per (device, stream): the calls of
# one stream run in order, so they can share it. At most _WS_MAX streams keep
# one (least recently used first out); a dropped or outgrown buffer returns
# to torch's caching allocator on its own stream, which orders its next use
# after the kernels already queued there.
_WS_MAX = 16
_workspaces = OrderedDict()
_ws_lock = threading.Lock()


def _workspace(device, stream_ptr: int, nbytes: int) -> torch.Tensor:
    """A workspace of at least ``nbytes`` for a call on ``device``'s current
    stream (``stream_ptr``)."""
    if torch.cuda.is_current_stream_capturing():
        # A captured call bakes the buffer's address into the graph: it gets
        # its own, from the graph's private pool (kept for the graph's
        # lifetime), never the shared per-stream buffer that a later, larger
        # eager call may replace and free.
        return torch.empty(nbytes, dtype=torch.uint8, device=device)
    key = (device, stream_ptr)
    with _ws_lock:
        ws = _workspaces.get(key)
        if ws is None or ws.numel() < nbytes:
            # allocated on the current stream (the call's), in the caching
            # allocator's pool of that stream
            ws = torch.empty(nbytes, dtype=torch.uint8, device=device)
            _workspaces[key] = ws
        _workspaces.move_to_end(key)
        while len(_workspaces) > _WS_MAX:
            _workspaces.popitem(last=False)
    return ws


# ---------------------------------------------------------------------------
# argument resolution (api.py:186-366)
# ---------------------------------------------------------------------------

class _Resolved:
    """A call's launch arguments with everything except its outputs, its
    workspace and host-side sequence lengths (staged per call)."""

    __slots__ = ("args", "keep", "device", "dtype", "T1", "N1", "layout_q", "B", "S_max", "host_parts",
                 "num_splits", "ws_bytes", "cacheable", "metadata_fn")


def _resolve(q, *, ori_kv, cmp_kv, cmp_sparse_indices, ori_block_table, cmp_block_table, cu_seqlens_q,
             seqused_q, seqused_kv, sinks, metadata, softmax_scale, cmp_ratio, ori_mask_mode, cmp_mask_mode,
             ori_win_left, ori_win_right, layout_q, layout_kv, core_num, topk_cmp, num_splits, head_waves,
             waves) -> _Resolved:
    del seqused_q  # API-parity placeholder, as in the reference (api.py:186)
    assert ori_mask_mode == 4, "only ori_mask_mode=4 supported"
    assert cmp_mask_mode == 3 or cmp_kv is None, "only cmp_mask_mode=3 supported"
    assert ori_win_right == 0, "only ori_win_right=0 supported"
    assert layout_kv == "PA_ND", "only layout_kv=PA_ND supported"
    assert layout_q in ("TND", "BSND"), f"unsupported layout_q={layout_q!r}"
    if q.dtype not in _DT:
        raise ValueError(f"unsupported torch dtype {q.dtype}")
    if not q.is_cuda:
        raise ValueError("sparse_attn_sharedkv runs on the GPU: q must be a device tensor")
    dev = q.device
    r = _Resolved()
    r.cacheable = True

    scenario = _lib.SAS_SWA if cmp_kv is None else (
        _lib.SAS_CFA if cmp_sparse_indices is None else _lib.SAS_SCFA)

    # ---- flat [total_tokens, N1, D] view + per-batch token offsets ----------
    # TND: the kernel takes cu_seqlens_q itself (q_prefix = cu_seqlens_q,
    # act_q = NULL), on the device as given or copied there per call.
    # BSND: q_prefix = b * S_max and the lengths, copied per call.
    if layout_q == "TND":
        assert cu_seqlens_q is not None, "cu_seqlens_q is required for TND"
        B = cu_seqlens_q.numel() - 1
        S_max = None   # not needed for TND outputs
        T1, N1, D = q.shape
        q_flat = q
        idx_flat = cmp_sparse_indices if scenario == _lib.SAS_SCFA else None
        seq_parts = [("cu", cu_seqlens_q)]
    else:
        B, S_max, N1, D = q.shape
        T1 = B * S_max
        q_flat = q.reshape(T1, N1, D)
        q_prefix = torch.arange(B, dtype=torch.int32) * S_max
        if cu_seqlens_q is not None:
            cu = cu_seqlens_q.to(torch.int32).cpu()
            act_q = cu[1:] - cu[:-1]
        else:
            act_q = torch.full((B,), S_max, dtype=torch.int32)
        idx_flat = None
        if scenario == _lib.SAS_SCFA:
            ci = cmp_sparse_indices
            idx_flat = ci.reshape(T1, ci.shape[2], ci.shape[3])
        seq_parts = [("qp", q_prefix), ("aq", act_q)]
        r.cacheable = False
    if B < 1:
        raise ValueError("batch must be at least 1")

    # ---- top-k / scenario tensors (api.py:244-277) ---------------------------
    fp8 = ori_kv.dtype == torch.uint8
    if scenario == _lib.SAS_SCFA:
        N2 = idx_flat.shape[1]
        K = topk_cmp if topk_cmp is not None else idx_flat.shape[2]
        assert K == idx_flat.shape[2], "topk_cmp does not match cmp_sparse_indices last dim"
        if idx_flat.shape[0] != T1:
            raise ValueError(f"cmp_sparse_indices has {idx_flat.shape[0]} rows, q has {T1} tokens")
    elif scenario == _lib.SAS_CFA:
        N2 = cmp_kv.shape[2]
        if cmp_ratio is None:
            cmp_ratio = 4
        # api.py:259-261: the slot count follows the longest sequence
        K = int(seqused_kv.max().item()) // cmp_ratio if seqused_kv.numel() else 0
    else:
        N2 = ori_kv.shape[2]
        K = 0
    row = ori_kv.shape[-1]
    if N2 != 1 or N1 % 16 != 0 or D not in (512, 576) or (fp8 and (D != 576 or row != FP8_ROW_BYTES)):
        raise ValueError(
            f"supported: N1 a multiple of 16, N2=1, D in (512, 576), fp8 rows of "
            f"{FP8_ROW_BYTES} bytes with D=576 (got N1={N1}, N2={N2}, D={D}, kv row={row})")
    if fp8 and q.dtype != torch.bfloat16:
        raise ValueError("fp8 caches need a bfloat16 query")
    if not fp8 and (ori_kv.dtype != q.dtype or row != D):
        raise ValueError(f"ori_kv must be {q.dtype} rows of {D} (got {ori_kv.dtype}, {row})")
    if cmp_kv is not None and (cmp_kv.dtype != ori_kv.dtype or cmp_kv.shape[-1] != row):
        raise ValueError("cmp_kv must use the same row format as ori_kv")
    cmp_ratio_eff = cmp_ratio if cmp_ratio is not None else 4
    if scenario >= _lib.SAS_CFA and cmp_ratio_eff < 1:
        raise ValueError("cmp_ratio must be >= 1")
    if seqused_kv.numel() != B:
        raise ValueError(f"seqused_kv has {seqused_kv.numel()} entries, batch is {B}")

    # ---- metadata (api.py:335-366) -------------------------------------------
    # A given tensor is validated. The kernel covers every (token, head group,
    # split) by construction and does not consume it, so an absent one is not
    # synthesised on the call path (about 25 us of host time per call);
    # PreparedCall.metadata() builds it with the bit-exact scheduler on demand.
    if metadata is not None:
        assert metadata.numel() == SAS_META_SIZE, (
            f"metadata must have {SAS_META_SIZE} int32 entries (got {metadata.numel()})")

    def _metadata():
        if metadata is not None:
            return metadata
        kv_max = int(seqused_kv.max().item()) if seqused_kv.numel() else 0
        if layout_q == "TND":
            cu_h = cu_seqlens_q.to(torch.int32).cpu()
            sq = int((cu_h[1:] - cu_h[:-1]).max().item()) if B else 0
        else:
            sq = int(S_max)
        meta_kwargs = dict(
            num_heads_q=N1, num_heads_kv=N2, head_dim=D,
            cu_seqlens_q=cu_seqlens_q if layout_q == "TND" else None,
            seqused_kv=seqused_kv, batch_size=int(B), max_seqlen_q=sq, max_seqlen_kv=kv_max,
            ori_mask_mode=ori_mask_mode, ori_win_left=ori_win_left, ori_win_right=ori_win_right,
            layout_q=layout_q, layout_kv=layout_kv, has_ori_kv=True,
            has_cmp_kv=cmp_kv is not None, aic_core_num=core_num)
        if scenario >= _lib.SAS_CFA:
            meta_kwargs["cmp_ratio"] = cmp_ratio_eff
            meta_kwargs["cmp_mask_mode"] = cmp_mask_mode
        if scenario == _lib.SAS_SCFA:
            meta_kwargs["cmp_topk"] = K
        return sparse_attn_sharedkv_metadata(**meta_kwargs)

    # ---- device operands ------------------------------------------------------
    # Used as given when already int32 / contiguous on the device; otherwise
    # converted (kept alive with the call, which is then not cached: the
    # converted copies are new tensors each time).
    keep = []

    def d(t, dtype=None):
        if t is None:
            return None
        if t.device == dev and (dtype is None or t.dtype == dtype) and t.is_contiguous():
            return t
        r.cacheable = False
        t = t.to(device=dev, dtype=dtype) if dtype is not None else t.to(device=dev)
        t = t.contiguous()
        keep.append(t)
        return t

    qd = d(q_flat)
    okv = d(ori_kv)
    obt = d(ori_block_table, torch.int32)
    ckv = d(cmp_kv) if scenario >= _lib.SAS_CFA else None
    cbt = d(cmp_block_table, torch.int32) if scenario >= _lib.SAS_CFA else None
    cidx = d(idx_flat, torch.int32) if scenario == _lib.SAS_SCFA else None
    snk = d(sinks, torch.float32)
    if snk.numel() != N1:
        raise ValueError(f"sinks must have {N1} entries (got {snk.numel()})")

    a = _lib.SasFwdArgs()
    host_parts = []
    for name, t in seq_parts + [("kv", seqused_kv.reshape(-1))]:
        if t.is_cuda:
            td = d(t, torch.int32)
            if name == "cu":
                a.q_prefix, a.act_q = td.data_ptr(), None
            elif name == "qp":
                a.q_prefix = td.data_ptr()
            elif name == "aq":
                a.act_q = td.data_ptr()
            else:
                a.act_kv = td.data_ptr()
        else:
            host_parts.append((name, t.to(torch.int32).reshape(-1)))

    a.q, a.ori_kv, a.ori_block_table = qd.data_ptr(), okv.data_ptr(), obt.data_ptr()
    a.cmp_kv = ckv.data_ptr() if ckv is not None else None
    a.cmp_block_table = cbt.data_ptr() if cbt is not None else None
    a.cmp_indices = cidx.data_ptr() if cidx is not None else None
    a.sinks = snk.data_ptr()
    a.T, a.B, a.H, a.D, a.DV = T1, B, N1, D, 512
    a.ori_block_size, a.ori_bt_stride, a.ori_num_blocks = okv.shape[1], obt.shape[1], okv.shape[0]
    if ckv is not None:
        a.cmp_block_size, a.cmp_bt_stride, a.cmp_num_blocks = ckv.shape[1], cbt.shape[1], ckv.shape[0]
    a.K = int(K)
    a.scenario = scenario
    a.q_dtype = _DT[q.dtype]
    a.kv_dtype = _lib.SAS_DT_FP8_E4M3_ROW656 if fp8 else _DT[q.dtype]
    a.cmp_ratio = int(cmp_ratio_eff)
    a.win_left = int(ori_win_left)
    a.softmax_scale = float(softmax_scale)
    a.num_splits = int(num_splits)
    a.head_waves = int(head_waves)
    a.waves = int(waves)
    ns = C.c_int32(0)
    ws = C.c_size_t(0)
    _lib.check(_lib.lib().sas_fwd_plan(C.byref(a), C.byref(ns), C.byref(ws)), "sparse_attn_sharedkv")
    a.num_splits = ns.value
    r.args, r.keep, r.device, r.dtype = a, keep, dev, q.dtype
    r.T1, r.N1, r.layout_q, r.B, r.S_max = T1, N1, layout_q, B, S_max
    r.host_parts = host_parts
    r.num_splits, r.ws_bytes = ns.value, ws.value
    r.metadata_fn = _metadata
    return r


def _host_i32(t: torch.Tensor) -> torch.Tensor:
    """A host tensor as contiguous int32 (itself when it already is)."""
    if t.dtype is not torch.int32 or not t.is_contiguous():
        t = t.to(torch.int32).contiguous()
    return t


def _point_seqlens(parts, a: _lib.SasFwdArgs, base: int) -> None:
    """Point the launch arguments at ``parts`` ((name, tensor) pairs) laid
    out one after the other from device address ``base``."""
    o = 0
    for name, t in parts:
        ptr = base + 4 * o
        if name == "cu":
            a.q_prefix, a.act_q = ptr, None
        elif name == "qp":
            a.q_prefix = ptr
        elif name == "aq":
            a.act_q = ptr
        else:
            a.act_kv = ptr
        o += int(t.numel())


def _bind_seqlens(r: _Resolved, parts, a: _lib.SasFwdArgs, stream, keep: list) -> None:
    """Copy the call's host-side sequence lengths ``parts`` ((name, int32
    tensor) pairs, the names of ``r.host_parts``) to the device through the
    pinned ring and point the launch arguments at them."""
    if not parts:
        return
    dev = _stage([t for _, t in parts], r.device, stream)
    keep.append(dev)
    _point_seqlens(parts, a, dev.data_ptr())


class PreparedCall:
    """Arguments of one forward, resolved and allocated; :meth:`launch` runs
    the kernels on the current (or given) stream without host syncs."""

    def __init__(self, r: _Resolved):
        self._r = r
        dev = r.device
        self.out = torch.empty((r.T1, r.N1, 512), dtype=r.dtype, device=dev)
        self.lse = torch.empty((r.T1, r.N1), dtype=torch.float32, device=dev)
        self.layout_q, self.B, self.S_max = r.layout_q, r.B, r.S_max
        self.num_splits = r.num_splits
        self._prep_stream = torch.cuda.current_stream(dev)
        self._keep = list(r.keep)
        self.args = _lib.SasFwdArgs.from_buffer_copy(r.args)
        self.args.out, self.args.lse = self.out.data_ptr(), self.lse.data_ptr()
        _bind_seqlens(r, r.host_parts, self.args, self._prep_stream, self._keep)
        self.workspace = None
        if r.ws_bytes:
            self.workspace = torch.empty(r.ws_bytes, dtype=torch.uint8, device=dev)
            self.args.workspace = self.workspace.data_ptr()
            self.args.workspace_bytes = r.ws_bytes

    def _stream(self, stream):
        st = stream if stream is not None else torch.cuda.current_stream(self.out.device)
        if st != self._prep_stream:
            # the device-side copies were enqueued on the stream that was
            # current when the call was prepared
            ev = torch.cuda.Event()
            ev.record(self._prep_stream)
            st.wait_event(ev)
        return C.c_void_p(st.cuda_stream)

    def launch(self, stream: Optional[torch.cuda.Stream] = None) -> None:
        """Split kernel, then (with more than one split) the LSE combine."""
        self.args.flags = 0
        _lib.check(_lib.lib().sas_fwd_v1(C.byref(self.args), self._stream(stream)),
                   "sparse_attn_sharedkv")

    def launch_split(self, stream: Optional[torch.cuda.Stream] = None) -> None:
        """Split kernel only; with more than one split the result is the
        partials in :attr:`workspace` until :meth:`launch_combine` runs."""
        self.args.flags = _lib.SAS_FWD_NO_COMBINE
        try:
            _lib.check(_lib.lib().sas_fwd_v1(C.byref(self.args), self._stream(stream)),
                       "sparse_attn_sharedkv")
        finally:
            self.args.flags = 0

    def combine_args(self) -> _lib.SasCombineArgs:
        a = self.args
        ca = _lib.SasCombineArgs()
        ca.part_o = a.workspace
        pb = 4 if a.q_dtype == _lib.SAS_DT_FP16 else 2   # part_o element: fp32 under fp16 out, else fp16
        ca.part_ml = a.workspace + a.T * self.num_splits * a.H * a.DV * pb
        ca.sinks, ca.out, ca.lse = a.sinks, a.out, a.lse
        ca.T, ca.S, ca.H, ca.DV = a.T, self.num_splits, a.H, a.DV
        ca.out_dtype = a.q_dtype
        return ca

    def launch_combine(self, stream: Optional[torch.cuda.Stream] = None) -> None:
        """LSE combine of the partials left by :meth:`launch_split`."""
        if self.num_splits <= 1:
            return
        ca = self.combine_args()
        _lib.check(_lib.lib().sas_combine_v1(C.byref(ca), self._stream(stream)),
                   "sparse_attn_sharedkv combine")

    def metadata(self) -> torch.Tensor:
        """The reference's int32[1024] scheduler metadata for this call: the
        tensor passed in, else synthesised with the bit-exact scheduler
        (metadata.py:258-1086). The kernels do not need it."""
        return self._r.metadata_fn()

    def result(self, return_softmax_lse: bool):
        return _result(self.out, self.lse, self.layout_q, self.B, self.S_max, return_softmax_lse)


def _result(out, lse, layout_q, B, S_max, return_softmax_lse):
    if layout_q == "BSND":
        out = out.reshape(B, S_max, out.shape[1], out.shape[2])
        lse = lse.reshape(B, S_max, lse.shape[1])
    return (out, lse) if return_softmax_lse else out


_FWD_DEFAULTS = dict(cmp_kv=None, cmp_sparse_indices=None, cmp_block_table=None, cu_seqlens_q=None,
                     seqused_q=None, metadata=None, cmp_ratio=None, ori_mask_mode=4, cmp_mask_mode=3,
                     ori_win_left=127, ori_win_right=0, layout_q="TND", layout_kv="PA_ND",
                     core_num=DEFAULT_CORE_NUM, topk_cmp=None, num_splits=0, head_waves=0, waves=0)


def prepare_sparse_attn_sharedkv(
    q: torch.Tensor,
    *,
    ori_kv: torch.Tensor,
    cmp_kv: Optional[torch.Tensor] = None,
    cmp_sparse_indices: Optional[torch.Tensor] = None,
    ori_block_table: torch.Tensor,
    cmp_block_table: Optional[torch.Tensor] = None,
    cu_seqlens_q: Optional[torch.Tensor] = None,
    seqused_q: Optional[torch.Tensor] = None,
    seqused_kv: torch.Tensor,
    sinks: torch.Tensor,
    metadata: Optional[torch.Tensor] = None,
    softmax_scale: float,
    cmp_ratio: Optional[int] = None,
    ori_mask_mode: int = 4,
    cmp_mask_mode: int = 3,
    ori_win_left: int = 127,
    ori_win_right: int = 0,
    layout_q: str = "TND",
    layout_kv: str = "PA_ND",
    core_num: int = DEFAULT_CORE_NUM,
    topk_cmp: Optional[int] = None,
    num_splits: int = 0,
    head_waves: int = 0,
    waves: int = 0,
) -> PreparedCall:
    """Validate and resolve the arguments of :func:`sparse_attn_sharedkv`
    (api.py:186-366) and allocate outputs and workspace; see that function."""
    r = _resolve(q, ori_kv=ori_kv, cmp_kv=cmp_kv, cmp_sparse_indices=cmp_sparse_indices,
                 ori_block_table=ori_block_table, cmp_block_table=cmp_block_table,
                 cu_seqlens_q=cu_seqlens_q, seqused_q=seqused_q, seqused_kv=seqused_kv, sinks=sinks,
                 metadata=metadata, softmax_scale=softmax_scale, cmp_ratio=cmp_ratio,
                 ori_mask_mode=ori_mask_mode, cmp_mask_mode=cmp_mask_mode, ori_win_left=ori_win_left,
                 ori_win_right=ori_win_right, layout_q=layout_q, layout_kv=layout_kv, core_num=core_num,
                 topk_cmp=topk_cmp, num_splits=num_splits, head_waves=head_waves, waves=waves)
    return PreparedCall(r)


# ---------------------------------------------------------------------------
# the drop-in entry point, with its per-signature cache
# ---------------------------------------------------------------------------

_CACHE_MAX = 64
_cache: "OrderedDict[tuple, _Resolved]" = OrderedDict()
_cache_lock = threading.Lock()


def _sig(t):
    """What a launch depends on for a tensor: device tensors by address and
    geometry (their values are read by the kernel), host tensors by geometry
    (their values are copied per call)."""
    if t is None:
        return None
    if t.is_cuda:
        return (t.data_ptr(), t.shape, t.stride(), t.dtype, t.device.index)
    return ("host", t.shape, t.dtype)


def sparse_attn_sharedkv(
    q: torch.Tensor,
    *,
    ori_kv: torch.Tensor,
    cmp_kv: Optional[torch.Tensor] = None,
    cmp_sparse_indices: Optional[torch.Tensor] = None,
    ori_block_table: torch.Tensor,
    cmp_block_table: Optional[torch.Tensor] = None,
    cu_seqlens_q: Optional[torch.Tensor] = None,
    seqused_q: Optional[torch.Tensor] = None,
    seqused_kv: torch.Tensor,
    sinks: torch.Tensor,
    metadata: Optional[torch.Tensor] = None,
    softmax_scale: float,
    cmp_ratio: Optional[int] = None,
    ori_mask_mode: int = 4,
    cmp_mask_mode: int = 3,
    ori_win_left: int = 127,
    ori_win_right: int = 0,
    layout_q: str = "TND",
    layout_kv: str = "PA_ND",
    return_softmax_lse: bool = False,
    core_num: int = DEFAULT_CORE_NUM,
    topk_cmp: Optional[int] = None,
) -> Union[torch.Tensor, Tuple[torch.Tensor, torch.Tensor]]:
    """Forward pass; returns ``attention_out`` in ``q``'s layout, or
    ``(attention_out, lse)`` when ``return_softmax_lse`` (api.py:129-397).

    ``attention_out`` is ``[T1, N1, 512]`` (TND) or ``[B, S1, N1, 512]``
    (BSND) in q's dtype; ``lse`` is fp32 ``[T1, N1]`` / ``[B, S1, N1]`` with
    ``lse = max + ln(sum)`` over all attended keys and the sink.
    """
    dev = q.device
    stream = _raw_stream(dev) if q.is_cuda else None
    # CFA's slot count follows the longest sequence (api.py:259-261): part of
    # the signature, read from the host copy, or through a sync as the
    # reference does for device lengths
    cfa_k = None
    if cmp_kv is not None and cmp_sparse_indices is None and seqused_kv.numel():
        cfa_k = int(seqused_kv.max().item())
    key = (_sig(q), _sig(ori_kv), _sig(cmp_kv), _sig(cmp_sparse_indices), _sig(ori_block_table),
           _sig(cmp_block_table), _sig(cu_seqlens_q), _sig(seqused_kv), _sig(sinks),
           None if metadata is None else metadata.numel(), float(softmax_scale), cmp_ratio, ori_mask_mode,
           cmp_mask_mode, ori_win_left, ori_win_right, layout_q, layout_kv, core_num, topk_cmp, cfa_k, stream)
    with _cache_lock:
        r = _cache.get(key)
        if r is not None:
            _cache.move_to_end(key)
    hit = r is not None
    if not hit:
        r = _resolve(q, ori_kv=ori_kv, cmp_kv=cmp_kv, cmp_sparse_indices=cmp_sparse_indices,
                     ori_block_table=ori_block_table, cmp_block_table=cmp_block_table,
                     cu_seqlens_q=cu_seqlens_q, seqused_q=seqused_q, seqused_kv=seqused_kv, sinks=sinks,
                     metadata=metadata, softmax_scale=softmax_scale, cmp_ratio=cmp_ratio,
                     ori_mask_mode=ori_mask_mode, cmp_mask_mode=cmp_mask_mode, ori_win_left=ori_win_left,
                     ori_win_right=ori_win_right, layout_q=layout_q, layout_kv=layout_kv,
                     core_num=core_num, topk_cmp=topk_cmp, num_splits=0, head_waves=0, waves=0)
        if r.cacheable:
            with _cache_lock:
                _cache[key] = r
                if len(_cache) > _CACHE_MAX:
                    _cache.popitem(last=False)
    out = torch.empty((r.T1, r.N1, 512), dtype=r.dtype, device=dev)
    lse = torch.empty((r.T1, r.N1), dtype=torch.float32, device=dev)
    a = _lib.SasFwdArgs.from_buffer_copy(r.args)
    a.out, a.lse = out.data_ptr(), lse.data_ptr()
    keep = []
    staged = None
    if r.host_parts:
        parts = r.host_parts
        if hit:
            # this call's host lengths (a cached resolution, TND only, holds
            # an earlier call's)
            cur = {"cu": cu_seqlens_q, "kv": seqused_kv}
            parts = [(name, _host_i32(cur[name])) for name, _ in r.host_parts]
        if not torch.cuda.is_current_stream_capturing():
            ring = _seqlen_ring(dev)
            staged = ring.stage([(t.data_ptr(), t.numel()) for _, t in parts], stream)
        if staged is not None:
            _point_seqlens(parts, a, staged[0])
        else:
            _bind_seqlens(r, parts, a, torch.cuda.current_stream(dev), keep)
    try:
        if r.ws_bytes:
            ws = _workspace(dev, stream, r.ws_bytes)
            a.workspace, a.workspace_bytes = ws.data_ptr(), r.ws_bytes
        _lib.check(_lib.lib().sas_fwd_v1(C.byref(a), C.c_void_p(stream)), "sparse_attn_sharedkv")
    finally:
        if staged is not None:
            ring.release(staged[1], stream)
    return _result(out, lse, r.layout_q, r.B, r.S_max, return_softmax_lse)


class PreparedBackward:
    """Arguments and gradient buffers of one backward, resolved once;
    :meth:`launch` enqueues the kernel (the gradients accumulate:
    :meth:`zero_grads` clears them), :meth:`result` returns them."""

    def __init__(self, call: PreparedCall, ba, keep, q, dq, d_ori, d_cmp, d_sinks):
        self._call, self.args, self._keep, self._q = call, ba, keep, q
        self.dq, self.d_ori_kv, self.d_cmp_kv, self.d_sinks = dq, d_ori, d_cmp, d_sinks

    def launch(self, stream: Optional[torch.cuda.Stream] = None) -> None:
        _lib.check(_lib.lib().sas_bwd_v1(C.byref(self.args), self._call._stream(stream)),
                   "sparse_attn_sharedkv_backward")

    def zero_grads(self) -> None:
        for t in (self.dq, self.d_ori_kv, self.d_cmp_kv, self.d_sinks):
            if t is not None:
                t.zero_()

    def result(self):
        return (self.dq.to(self._q.dtype).reshape(self._q.shape), self.d_ori_kv, self.d_cmp_kv,
                self.d_sinks)


def prepare_sparse_attn_sharedkv_backward(dout: torch.Tensor, q: torch.Tensor, out: torch.Tensor,
                                          lse: torch.Tensor, **kwargs) -> PreparedBackward:
    """Validate and bind the arguments of :func:`sparse_attn_sharedkv_backward`
    and allocate its (zeroed) gradient buffers. ``window_pass`` (keyword,
    default None: the library's choice, the key-major pass for prefills)
    selects how window rows' gradients are summed: True, the key-major pass
    (each row's gradient summed over the tokens whose window holds it, one
    add per 16 heads, beside the per-token kernel on a side stream); False,
    one add per (token, row); the results agree up to fp32 summation
    order."""
    kwargs.pop("return_softmax_lse", None)
    window_pass = kwargs.pop("window_pass", None)
    call = prepare_sparse_attn_sharedkv(q, **kwargs)
    # a copy: the forward's resolved split count stays with the forward. The
    # backward takes the caller's count, or plans its own (0); the forward's
    # plan (C2: 4 splits, 128 workgroups of 64 heads) would leave half the
    # CUs idle.
    a = _lib.SasFwdArgs.from_buffer_copy(call.args)
    a.num_splits = int(kwargs.get("num_splits", 0))
    if window_pass is not None:
        a.flags = _lib.SAS_BWD_WINDOW_KEYS if window_pass else _lib.SAS_BWD_WINDOW_TOKENS
    if a.kv_dtype != a.q_dtype:
        raise ValueError("the backward needs caches in the query dtype (fp8 rows are not differentiated)")
    T1, H = int(a.T), int(a.H)
    dev = q.device
    dout_f = dout.reshape(T1, H, 512)
    out_f = out.reshape(T1, H, 512)
    lse_f = lse.reshape(T1, H)
    for name, t_, dt in (("dout", dout_f, q.dtype), ("out", out_f, q.dtype), ("lse", lse_f, torch.float32)):
        if t_.dtype != dt or t_.device != dev:
            raise ValueError(f"{name} must be a {dt} tensor on {dev}")
    dout_f, out_f, lse_f = dout_f.contiguous(), out_f.contiguous(), lse_f.contiguous()
    ori_kv = kwargs["ori_kv"]
    cmp_kv = kwargs.get("cmp_kv")
    dq = torch.zeros((T1, H, int(a.D)), dtype=torch.float32, device=dev)
    d_ori = torch.zeros(ori_kv.shape, dtype=torch.float32, device=dev)
    d_cmp = torch.zeros(cmp_kv.shape, dtype=torch.float32, device=dev) if cmp_kv is not None else None
    d_sinks = torch.zeros(H, dtype=torch.float32, device=dev)
    a.out, a.lse = out_f.data_ptr(), lse_f.data_ptr()
    ba = _lib.SasBwdArgs(fwd=a, dout=dout_f.data_ptr(), dq=dq.data_ptr(), d_ori_kv=d_ori.data_ptr(),
                         d_cmp_kv=d_cmp.data_ptr() if d_cmp is not None else None,
                         d_sinks=d_sinks.data_ptr())
    return PreparedBackward(call, ba, [dout_f, out_f, lse_f], q, dq, d_ori, d_cmp, d_sinks)


def sparse_attn_sharedkv_backward(
    dout: torch.Tensor,
    q: torch.Tensor,
    out: torch.Tensor,
    lse: torch.Tensor,
    **kwargs,
) -> Tuple[torch.Tensor, torch.Tensor, Optional[torch.Tensor], torch.Tensor]:
    """Gradients of :func:`sparse_attn_sharedkv` (the reference has no
    backward; its LSE output is documented as this pass's input, api.py:32-35).

    ``dout``, ``out`` (``[..., 512]``) and ``lse`` are in the forward's layout;
    ``kwargs`` are the forward's keyword arguments (same caches, tables,
    indices, seqlens, sinks, scale, scenario). Caches must be in q's dtype.
    Returns ``(dq, d_ori_kv, d_cmp_kv, d_sinks)``: ``dq`` in q's dtype and
    layout; the cache gradients fp32 in the caches' shapes (zero for rows no
    token attends; ``d_cmp_kv`` is None without ``cmp_kv``); ``d_sinks`` fp32
    ``[H]``. Key sets are the forward's: window rows and the valid top-k (or
    dense compressed) rows; V is the first 512 channels of each row.
    """
    pb = prepare_sparse_attn_sharedkv_backward(dout, q, out, lse, **kwargs)
    pb.launch()
    return pb.result()


class _SparseAttnSharedkvFn(torch.autograd.Function):
    """Autograd binding: forward = :func:`sparse_attn_sharedkv` (keeping
    out / LSE), backward = :func:`sparse_attn_sharedkv_backward`."""

    @staticmethod
    def forward(ctx, q, ori_kv, cmp_kv, sinks, kw):
        kwargs = dict(kw, ori_kv=ori_kv, cmp_kv=cmp_kv, sinks=sinks)
        out, lse = sparse_attn_sharedkv(q, return_softmax_lse=True, **kwargs)
        ctx.save_for_backward(q, ori_kv, cmp_kv if cmp_kv is not None else torch.empty(0), sinks, out, lse)
        ctx.kw = kw
        ctx.has_cmp = cmp_kv is not None
        ctx.mark_non_differentiable(lse)
        return out, lse

    @staticmethod
    def backward(ctx, dout, dlse):
        q, ori_kv, cmp_kv, sinks, out, lse = ctx.saved_tensors
        kwargs = dict(ctx.kw, ori_kv=ori_kv, cmp_kv=cmp_kv if ctx.has_cmp else None, sinks=sinks)
        dq, d_ori, d_cmp, d_sinks = sparse_attn_sharedkv_backward(
            dout.to(q.dtype).contiguous(), q, out, lse, **kwargs)
        return (dq, d_ori.to(ori_kv.dtype), d_cmp.to(cmp_kv.dtype) if ctx.has_cmp else None,
                d_sinks.to(sinks.dtype), None)


def sparse_attn_sharedkv_autograd(q: torch.Tensor, *, ori_kv: torch.Tensor,
                                  cmp_kv: Optional[torch.Tensor] = None, sinks: torch.Tensor,
                                  return_softmax_lse: bool = False, **kwargs):
    """:func:`sparse_attn_sharedkv` recorded for autograd: gradients flow to
    ``q``, ``ori_kv``, ``cmp_kv`` and ``sinks`` (through
    :func:`sparse_attn_sharedkv_backward`; the LSE output is not
    differentiable). Other arguments as for :func:`sparse_attn_sharedkv`."""
    out, lse = _SparseAttnSharedkvFn.apply(q, ori_kv, cmp_kv, sinks, kwargs)
    return (out, lse) if return_softmax_lse else out
