"""ctypes binding of libsas.so (declared in include/sas.h).

The library is loaded from this package directory only; there is no Python
or CPU fallback for the kernels. Loading fails loudly when the library has
not been built (``python -m dsv4_amd.build``).
"""

from __future__ import annotations

import ctypes as C
import os
import threading

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libsas.so")

SAS_OK, SAS_EINVAL, SAS_ELAUNCH, SAS_ENOWS = 0, 1, 2, 3
SAS_DT_BF16, SAS_DT_FP16, SAS_DT_FP8_E4M3_ROW656 = 0, 1, 2
SAS_SWA, SAS_CFA, SAS_SCFA = 1, 2, 3
SAS_META_SIZE = 1024
SAS_FWD_NO_COMBINE = 1
SAS_BWD_WINDOW_TOKENS = 2   # backward: per-token adds for window rows
SAS_BWD_WINDOW_KEYS = 4     # backward: the key-major window pass

EXPORTED = ("sas_metadata_v1", "sas_metadata_device_v1", "sas_fwd_plan", "sas_fwd_v1", "sas_fwd_noalloc_v1", "sas_combine_v1",
            "sas_cache_write_v1", "sas_bwd_v1", "sas_last_error", "sas_version",
            "sas_bench_atomic_add_v1")

_i32p = C.POINTER(C.c_int32)


class SasMetaParams(C.Structure):
    _fields_ = [
        ("num_heads_q", C.c_int64), ("num_heads_kv", C.c_int64), ("head_dim", C.c_int64),
        ("batch_size", C.c_int64), ("max_seqlen_q", C.c_int64), ("max_seqlen_kv", C.c_int64),
        ("ori_topk", C.c_int64), ("cmp_topk", C.c_int64), ("cmp_ratio", C.c_int64),
        ("ori_mask_mode", C.c_int64), ("cmp_mask_mode", C.c_int64),
        ("ori_win_left", C.c_int64), ("ori_win_right", C.c_int64),
        ("layout_q", C.c_char_p), ("layout_kv", C.c_char_p),
        ("has_ori_kv", C.c_int32), ("has_cmp_kv", C.c_int32),
        ("aic_core_num", C.c_int64), ("aiv_core_num", C.c_int64),
        ("cu_seqlens_q", _i32p), ("n_cu_seqlens_q", C.c_int64),
        ("cu_seqlens_ori_kv", _i32p), ("n_cu_seqlens_ori_kv", C.c_int64),
        ("cu_seqlens_cmp_kv", _i32p), ("n_cu_seqlens_cmp_kv", C.c_int64),
        ("seqused_q", _i32p), ("n_seqused_q", C.c_int64),
        ("seqused_kv", _i32p), ("n_seqused_kv", C.c_int64),
    ]


class SasFwdArgs(C.Structure):
    _fields_ = [
        ("q", C.c_void_p), ("ori_kv", C.c_void_p), ("ori_block_table", C.c_void_p),
        ("cmp_kv", C.c_void_p), ("cmp_block_table", C.c_void_p), ("cmp_indices", C.c_void_p),
        ("q_prefix", C.c_void_p), ("act_q", C.c_void_p), ("act_kv", C.c_void_p),
        ("sinks", C.c_void_p), ("out", C.c_void_p), ("lse", C.c_void_p),
        ("workspace", C.c_void_p), ("workspace_bytes", C.c_size_t),
        ("T", C.c_int64), ("B", C.c_int64), ("H", C.c_int64), ("D", C.c_int64), ("DV", C.c_int64),
        ("ori_block_size", C.c_int64), ("ori_bt_stride", C.c_int64), ("ori_num_blocks", C.c_int64),
        ("cmp_block_size", C.c_int64), ("cmp_bt_stride", C.c_int64), ("cmp_num_blocks", C.c_int64),
        ("K", C.c_int64),
        ("scenario", C.c_int32), ("q_dtype", C.c_int32), ("kv_dtype", C.c_int32),
        ("cmp_ratio", C.c_int32), ("win_left", C.c_int32),
        ("softmax_scale", C.c_float),
        ("num_splits", C.c_int32),
        ("head_waves", C.c_int32),
        ("flags", C.c_int32),
        ("waves", C.c_int32),
    ]


class SasCombineArgs(C.Structure):
    _fields_ = [
        ("part_o", C.c_void_p), ("part_ml", C.c_void_p), ("sinks", C.c_void_p),
        ("out", C.c_void_p), ("lse", C.c_void_p),
        ("T", C.c_int64), ("S", C.c_int64), ("H", C.c_int64), ("DV", C.c_int64),
        ("out_dtype", C.c_int32),
    ]


class SasBwdArgs(C.Structure):
    _fields_ = [
        ("fwd", SasFwdArgs), ("dout", C.c_void_p), ("dq", C.c_void_p),
        ("d_ori_kv", C.c_void_p), ("d_cmp_kv", C.c_void_p), ("d_sinks", C.c_void_p),
    ]


class SasCacheWriteArgs(C.Structure):
    _fields_ = [
        ("kv", C.c_void_p), ("seq_ids", C.c_void_p), ("positions", C.c_void_p),
        ("block_table", C.c_void_p), ("cache", C.c_void_p),
        ("N", C.c_int64), ("B", C.c_int64), ("D", C.c_int64), ("kv_stride", C.c_int64),
        ("bt_stride", C.c_int64), ("block_size", C.c_int64), ("num_blocks", C.c_int64),
        ("kv_dtype", C.c_int32), ("cache_dtype", C.c_int32),
    ]


_lock = threading.Lock()
_lib = None


def lib() -> C.CDLL:
    """The loaded libsas.so (raises if it is missing)."""
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not os.path.exists(LIB_PATH):
                    raise RuntimeError(
                        f"{LIB_PATH} is missing: build it with `python -m dsv4_amd.build` "
                        "(the HIP library is the only implementation; there is no fallback)")
                L = C.CDLL(LIB_PATH)
                L.sas_metadata_v1.argtypes = [C.POINTER(SasMetaParams), _i32p]
                L.sas_metadata_v1.restype = C.c_int
                L.sas_metadata_device_v1.argtypes = [C.POINTER(SasMetaParams), C.c_void_p, C.c_void_p]
                L.sas_metadata_device_v1.restype = C.c_int
                L.sas_fwd_plan.argtypes = [C.POINTER(SasFwdArgs), _i32p, C.POINTER(C.c_size_t)]
                L.sas_fwd_plan.restype = C.c_int
                L.sas_fwd_v1.argtypes = [C.POINTER(SasFwdArgs), C.c_void_p]
                L.sas_fwd_v1.restype = C.c_int
                L.sas_fwd_noalloc_v1.argtypes = [C.POINTER(SasFwdArgs), C.c_void_p]
                L.sas_fwd_noalloc_v1.restype = C.c_int
                L.sas_combine_v1.argtypes = [C.POINTER(SasCombineArgs), C.c_void_p]
                L.sas_combine_v1.restype = C.c_int
                L.sas_bwd_v1.argtypes = [C.POINTER(SasBwdArgs), C.c_void_p]
                L.sas_bwd_v1.restype = C.c_int
                L.sas_cache_write_v1.argtypes = [C.POINTER(SasCacheWriteArgs), C.c_void_p]
                L.sas_cache_write_v1.restype = C.c_int
                L.sas_bench_atomic_add_v1.argtypes = [C.c_void_p, C.c_int32, C.c_int32, C.c_int32, C.c_int32,
                                                      C.c_void_p]
                L.sas_bench_atomic_add_v1.restype = C.c_int
                L.sas_last_error.argtypes = []
                L.sas_last_error.restype = C.c_char_p
                L.sas_version.argtypes = []
                L.sas_version.restype = C.c_char_p
                _lib = L
    return _lib


def check(rc: int, what: str) -> None:
    """Raise the reference-style exception for a non-zero status."""
    if rc == SAS_OK:
        return
    msg = lib().sas_last_error().decode(errors="replace")
    if rc in (SAS_EINVAL, SAS_ENOWS):
        raise ValueError(f"{what}: {msg}")
    raise RuntimeError(f"{what}: {msg}")
