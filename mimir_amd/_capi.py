"""ctypes binding of libmimir_prefixlm.so (include/mimir_prefixlm.h).

The binding mirrors the C structs field for field and maps the library's status
codes onto the exception types the reference raises for the same conditions
(``ValueError`` for bad lengths / GQA, flash_attention_prefixlm_dense.py:14,54-55;
``TypeError`` for an unsupported dtype, flash_attention_prefixlm_mps.py:1390-1391;
``ImportError`` when the backend library is missing, flash_attention_prefixlm_fa4.py:32-35).
"""

from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

# MIMIR_PREFIXLM_LIB overrides the in-tree library (e.g. to A/B two builds).
LIB_PATH = Path(os.environ.get("MIMIR_PREFIXLM_LIB") or Path(__file__).resolve().parent / "_lib" / "libmimir_prefixlm.so")
ABI_VERSION = 8

DTYPE_FLOAT32 = 0
DTYPE_BFLOAT16 = 1

SPLIT_AUTO = 0
SPLIT_ALWAYS = 1
SPLIT_NEVER = 2

OK = 0
ERR_INVALID_ARGUMENT = 1
ERR_UNSUPPORTED_DTYPE = 2
ERR_UNSUPPORTED_SHAPE = 3
ERR_HIP = 4

_i64 = ctypes.c_int64
_i32 = ctypes.c_int32
_vp = ctypes.c_void_p


class FwdParams(ctypes.Structure):
    _fields_ = [
        ("q", _vp), ("k", _vp), ("v", _vp), ("out", _vp), ("lse", _vp),
        ("prefix_lens", _vp), ("causal_lens", _vp), ("cu_seqlens", _vp),
        ("q_stride_token", _i64), ("q_stride_head", _i64),
        ("k_stride_token", _i64), ("k_stride_head", _i64),
        ("v_stride_token", _i64), ("v_stride_head", _i64),
        ("out_stride_token", _i64), ("out_stride_head", _i64),
        ("lse_stride_head", _i64),
        ("total_tokens", _i32), ("num_q_heads", _i32), ("num_kv_heads", _i32), ("head_dim", _i32),
        ("numseqs", _i32), ("total_seqlen", _i32), ("max_seqlen_all", _i32), ("is_causal", _i32),
        ("dtype", _i32), ("softmax_scale", ctypes.c_float),
        ("workspace", _vp), ("workspace_bytes", ctypes.c_size_t),
        ("gate", _vp), ("gate_stride_token", _i64), ("gate_stride_head", _i64),
        ("gated_out", _vp), ("gated_out_stride_token", _i64), ("gated_out_stride_head", _i64),
        ("out_lo", _vp), ("out_lo_stride_token", _i64), ("out_lo_stride_head", _i64),
        ("split_mode", _i32), ("split_flag", _vp),
        ("rope_cos", _vp), ("rope_sin", _vp), ("rope_stride_token", _i64),
        ("q_rope", _vp), ("q_rope_stride_token", _i64), ("q_rope_stride_head", _i64),
    ]


class BwdParams(ctypes.Structure):
    _fields_ = [
        ("q", _vp), ("k", _vp), ("v", _vp), ("out", _vp), ("dout", _vp), ("lse", _vp),
        ("dq", _vp), ("dk", _vp), ("dv", _vp),
        ("prefix_lens", _vp), ("causal_lens", _vp), ("cu_seqlens", _vp),
        ("q_stride_token", _i64), ("q_stride_head", _i64),
        ("k_stride_token", _i64), ("k_stride_head", _i64),
        ("v_stride_token", _i64), ("v_stride_head", _i64),
        ("out_stride_token", _i64), ("out_stride_head", _i64),
        ("dout_stride_token", _i64), ("dout_stride_head", _i64),
        ("dq_stride_token", _i64), ("dq_stride_head", _i64),
        ("dk_stride_token", _i64), ("dk_stride_head", _i64),
        ("dv_stride_token", _i64), ("dv_stride_head", _i64),
        ("lse_stride_head", _i64),
        ("total_tokens", _i32), ("num_q_heads", _i32), ("num_kv_heads", _i32), ("head_dim", _i32),
        ("numseqs", _i32), ("total_seqlen", _i32), ("max_seqlen_all", _i32), ("is_causal", _i32),
        ("dtype", _i32), ("softmax_scale", ctypes.c_float),
        ("workspace", _vp), ("workspace_bytes", ctypes.c_size_t),
        ("gate", _vp), ("gate_stride_token", _i64), ("gate_stride_head", _i64),
        ("dgate", _vp), ("dgate_stride_token", _i64), ("dgate_stride_head", _i64),
        ("dscore_limit_bytes", ctypes.c_size_t),
        ("out_lo", _vp), ("out_lo_stride_token", _i64), ("out_lo_stride_head", _i64),
        ("split_mode", _i32), ("split_flag", _vp),
        ("rope_cos", _vp), ("rope_sin", _vp), ("rope_stride_token", _i64),
        ("dq_key_chunks", _i32),
    ]


class RopeParams(ctypes.Structure):
    _fields_ = [
        ("x", _vp), ("y", _vp), ("cos", _vp), ("sin", _vp),
        ("x_stride_token", _i64), ("x_stride_head", _i64),
        ("y_stride_token", _i64), ("y_stride_head", _i64),
        ("cs_stride_token", _i64),
        ("total_tokens", _i32), ("num_heads", _i32), ("head_dim", _i32), ("dtype", _i32), ("inverse", _i32),
    ]


class CacheAttnParams(ctypes.Structure):
    _fields_ = [
        ("q", _vp), ("k_new", _vp), ("v_new", _vp), ("cache_k", _vp), ("cache_v", _vp), ("out", _vp),
        ("cache_lengths", _vp), ("batch_indices", _vp),
        ("q_stride_batch", _i64), ("q_stride_token", _i64), ("q_stride_head", _i64),
        ("kn_stride_batch", _i64), ("kn_stride_token", _i64), ("kn_stride_head", _i64),
        ("vn_stride_batch", _i64), ("vn_stride_token", _i64), ("vn_stride_head", _i64),
        ("ck_stride_batch", _i64), ("ck_stride_token", _i64), ("ck_stride_head", _i64),
        ("cv_stride_batch", _i64), ("cv_stride_token", _i64), ("cv_stride_head", _i64),
        ("out_stride_batch", _i64), ("out_stride_token", _i64), ("out_stride_head", _i64),
        ("batch", _i32), ("seqlen", _i32), ("cache_len", _i32), ("cache_rows", _i32), ("max_kv_len", _i32),
        ("num_q_heads", _i32), ("num_kv_heads", _i32), ("head_dim", _i32), ("causal", _i32), ("dtype", _i32),
        ("softmax_scale", ctypes.c_float), ("workspace", _vp), ("workspace_bytes", ctypes.c_size_t),
        ("index_int64", _i32),
    ]


BWD_STAGE_DELTA = 1
BWD_STAGE_DKDV = 2
BWD_STAGE_DQ = 4
BWD_STAGE_FILL = 8
BWD_STAGE_ALL = 15

EXPORTED_SYMBOLS = (
    "mimir_prefixlm_fwd",
    "mimir_prefixlm_fwd_noalloc",
    "mimir_prefixlm_bwd",
    "mimir_prefixlm_bwd_stages",
    "mimir_prefixlm_fwd_workspace_bytes",
    "mimir_prefixlm_fwd_workspace_size",
    "mimir_prefixlm_bwd_workspace_bytes",
    "mimir_prefixlm_bwd_workspace_size",
    "mimir_prefixlm_bwd_dscore_bytes",
    "mimir_prefixlm_rope",
    "mimir_prefixlm_cache_attn",
    "mimir_prefixlm_cache_attn_workspace_bytes",
    "mimir_prefixlm_check_metadata",
    "mimir_prefixlm_last_error",
    "mimir_prefixlm_abi_version",
)

_lib = None
_lock = threading.Lock()


def library_path() -> Path:
    return LIB_PATH


def load() -> ctypes.CDLL:
    """Load the HIP library once; ImportError if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise ImportError(
                f"mimir_amd prefix-LM attention requires the HIP library {LIB_PATH}; "
                "build it with `python -m mimir_amd.build`"
            )
        lib = ctypes.CDLL(str(LIB_PATH))
        lib.mimir_prefixlm_fwd.argtypes = [ctypes.POINTER(FwdParams), _vp]
        lib.mimir_prefixlm_fwd.restype = ctypes.c_int
        lib.mimir_prefixlm_fwd_noalloc.argtypes = [ctypes.POINTER(FwdParams), _vp]
        lib.mimir_prefixlm_fwd_noalloc.restype = ctypes.c_int
        lib.mimir_prefixlm_bwd.argtypes = [ctypes.POINTER(BwdParams), _vp]
        lib.mimir_prefixlm_bwd.restype = ctypes.c_int
        lib.mimir_prefixlm_bwd_stages.argtypes = [ctypes.POINTER(BwdParams), ctypes.c_int, _vp]
        lib.mimir_prefixlm_bwd_stages.restype = ctypes.c_int
        lib.mimir_prefixlm_fwd_workspace_bytes.argtypes = [_i32, _i32, _i32]
        lib.mimir_prefixlm_fwd_workspace_bytes.restype = ctypes.c_size_t
        lib.mimir_prefixlm_fwd_workspace_size.argtypes = [ctypes.POINTER(FwdParams)]
        lib.mimir_prefixlm_fwd_workspace_size.restype = ctypes.c_size_t
        lib.mimir_prefixlm_bwd_workspace_bytes.argtypes = [_i32, _i32, _i32, _i32]
        lib.mimir_prefixlm_bwd_workspace_bytes.restype = ctypes.c_size_t
        lib.mimir_prefixlm_bwd_workspace_size.argtypes = [ctypes.POINTER(BwdParams)]
        lib.mimir_prefixlm_bwd_workspace_size.restype = ctypes.c_size_t
        lib.mimir_prefixlm_bwd_dscore_bytes.argtypes = [ctypes.POINTER(BwdParams)]
        lib.mimir_prefixlm_bwd_dscore_bytes.restype = ctypes.c_size_t
        lib.mimir_prefixlm_rope.argtypes = [ctypes.POINTER(RopeParams), _vp]
        lib.mimir_prefixlm_rope.restype = ctypes.c_int
        lib.mimir_prefixlm_cache_attn.argtypes = [ctypes.POINTER(CacheAttnParams), _vp]
        lib.mimir_prefixlm_cache_attn.restype = ctypes.c_int
        lib.mimir_prefixlm_cache_attn_workspace_bytes.argtypes = [ctypes.POINTER(CacheAttnParams)]
        lib.mimir_prefixlm_cache_attn_workspace_bytes.restype = ctypes.c_size_t
        lib.mimir_prefixlm_check_metadata.argtypes = [_vp, _vp, _vp, _i32, _i32, _vp, _vp]
        lib.mimir_prefixlm_check_metadata.restype = ctypes.c_int
        lib.mimir_prefixlm_last_error.argtypes = []
        lib.mimir_prefixlm_last_error.restype = ctypes.c_char_p
        lib.mimir_prefixlm_abi_version.argtypes = []
        lib.mimir_prefixlm_abi_version.restype = ctypes.c_int
        version = lib.mimir_prefixlm_abi_version()
        if version != ABI_VERSION:
            raise ImportError(f"{LIB_PATH} has ABI version {version}, expected {ABI_VERSION}; rebuild it")
        _lib = lib
        return lib


def raise_for_status(lib: ctypes.CDLL, status: int) -> None:
    if status == OK:
        return
    msg = lib.mimir_prefixlm_last_error().decode(errors="replace")
    if status == ERR_UNSUPPORTED_DTYPE:
        raise TypeError(msg)
    if status in (ERR_INVALID_ARGUMENT, ERR_UNSUPPORTED_SHAPE):
        raise ValueError(msg)
    raise RuntimeError(msg)
