"""ctypes binding of the C ABI in ``include/simplicial_mi355x.h``.

The shared library ``libsimplicial_mi355x.so`` is built in-tree by
``archlab_amd.build`` (hipcc, gfx950).  There is no fallback: if the library
is missing or the device is not a ROCm GPU, every entry point raises.
"""

from __future__ import annotations

import ctypes
import os
import threading

import torch  # noqa: F401  -- loads torch's HIP runtime first; the library binds to it

LIB_NAME = "libsimplicial_mi355x.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)

SA_OK, SA_ERR_INVALID, SA_ERR_UNSUPPORTED, SA_ERR_HIP = 0, 1, 2, 3
SA_DTYPE_F32, SA_DTYPE_BF16, SA_DTYPE_F16 = 0, 1, 2
SA_INDEX_I32, SA_INDEX_I64 = 0, 1
SA_FLAG_FORCE_GENERIC = 1
SA_FLAG_SEPARATE_DK1 = 2
# SIMPLICIAL_MI355X_ABI_VERSION of the header these struct layouts mirror
ABI_VERSION = 3

_i64, _i32, _f32, _vp = ctypes.c_int64, ctypes.c_int32, ctypes.c_float, ctypes.c_void_p


class PrefillArgs(ctypes.Structure):
    _fields_ = [
        ("q", _vp), ("k1", _vp), ("k2", _vp), ("v1", _vp), ("v2", _vp),
        ("out", _vp), ("lse", _vp), ("cu_seqlens", _vp),
        ("q_stride_t", _i64), ("q_stride_h", _i64),
        ("k_stride_t", _i64), ("k_stride_h", _i64),
        ("v_stride_t", _i64), ("v_stride_h", _i64),
        ("o_stride_t", _i64), ("o_stride_h", _i64),
        ("lse_stride_t", _i64),
        ("num_seqs", _i32), ("seqlen", _i32), ("total_tokens", _i32),
        ("heads_q", _i32), ("heads_kv", _i32), ("head_dim", _i32), ("value_dim", _i32),
        ("short_window", _i32), ("long_window", _i32),
        ("scale", _f32), ("dtype", _i32), ("flags", _i32),
        ("workspace", _vp), ("workspace_bytes", ctypes.c_size_t),
    ]


class PagedArgs(ctypes.Structure):
    _fields_ = [
        ("q", _vp), ("q_stride_t", _i64), ("q_stride_h", _i64),
        ("short_cache", _vp), ("sc_stride", _i64 * 4),
        ("long_cache", _vp), ("lc_stride", _i64 * 4),
        ("short_table", _vp), ("st_stride", _i64),
        ("long_table", _vp), ("lt_stride", _i64),
        ("token_seq", _vp), ("token_pos", _vp),
        ("out", _vp), ("o_stride_t", _i64), ("o_stride_h", _i64),
        ("lse", _vp),
        ("tokens", _i32), ("heads_q", _i32), ("heads_kv", _i32), ("head_dim", _i32), ("block_size", _i32),
        ("num_seqs", _i32), ("short_table_width", _i32), ("long_table_width", _i32),
        ("short_blocks", _i32), ("long_blocks", _i32),
        ("short_window", _i32), ("long_window", _i32),
        ("splits", _i32), ("scale", _f32),
        ("q_dtype", _i32), ("cache_dtype", _i32),
        ("table_index_dtype", _i32), ("token_index_dtype", _i32),
        ("flags", _i32),
        ("long_cache_dtype", _i32), ("long_table_index_dtype", _i32), ("token_pos_index_dtype", _i32),
        ("token_window_caps", _vp),
    ]


class PrefillBwdArgs(ctypes.Structure):
    _fields_ = [
        ("fwd", PrefillArgs),
        ("dout", _vp), ("do_stride_t", _i64), ("do_stride_h", _i64),
        ("dq", _vp), ("dq_stride_t", _i64), ("dq_stride_h", _i64),
        ("dk1", _vp), ("dk2", _vp), ("dk_stride_t", _i64), ("dk_stride_h", _i64),
        ("dv1", _vp), ("dv2", _vp), ("dv_stride_t", _i64), ("dv_stride_h", _i64),
        ("dlse", _vp), ("dlse_stride_t", _i64),
    ]


EXPORTS = ("sa_prefill_fwd", "sa_paged_fwd", "sa_paged_workspace_bytes", "sa_paged_splits",
           "sa_prefill_kernel", "sa_paged_kernel", "sa_last_error", "sa_version",
           "sa_prefill_bwd", "sa_prefill_bwd_workspace_bytes", "sa_paged_fwd_noalloc",
           "sa_prefill_workspace_bytes", "sa_abi_version")

_lib = None
_lock = threading.Lock()


def library_path() -> str:
    return LIB_PATH


def load():
    """Load the shared library (once).  Raises RuntimeError if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_NAME} is not built ({LIB_PATH}); run `python -m archlab_amd.build` "
                "or __graft_entry__.build() first")
        lib = ctypes.CDLL(LIB_PATH, mode=ctypes.RTLD_GLOBAL)
        lib.sa_prefill_fwd.argtypes = [ctypes.POINTER(PrefillArgs), _vp]
        lib.sa_prefill_fwd.restype = ctypes.c_int
        lib.sa_prefill_workspace_bytes.argtypes = [ctypes.POINTER(PrefillArgs)]
        lib.sa_prefill_workspace_bytes.restype = ctypes.c_size_t
        lib.sa_paged_fwd.argtypes = [ctypes.POINTER(PagedArgs), _vp, ctypes.c_size_t, _vp]
        lib.sa_paged_fwd.restype = ctypes.c_int
        lib.sa_paged_fwd_noalloc.argtypes = [ctypes.POINTER(PagedArgs), _vp]
        lib.sa_paged_fwd_noalloc.restype = ctypes.c_int
        lib.sa_paged_workspace_bytes.argtypes = [ctypes.POINTER(PagedArgs)]
        lib.sa_paged_workspace_bytes.restype = ctypes.c_size_t
        lib.sa_paged_splits.argtypes = [ctypes.POINTER(PagedArgs)]
        lib.sa_paged_splits.restype = ctypes.c_int
        lib.sa_prefill_kernel.argtypes = [ctypes.POINTER(PrefillArgs)]
        lib.sa_prefill_kernel.restype = ctypes.c_char_p
        lib.sa_paged_kernel.argtypes = [ctypes.POINTER(PagedArgs)]
        lib.sa_paged_kernel.restype = ctypes.c_char_p
        lib.sa_prefill_bwd.argtypes = [ctypes.POINTER(PrefillBwdArgs), _vp, ctypes.c_size_t, _vp]
        lib.sa_prefill_bwd.restype = ctypes.c_int
        lib.sa_prefill_bwd_workspace_bytes.argtypes = [ctypes.POINTER(PrefillBwdArgs)]
        lib.sa_prefill_bwd_workspace_bytes.restype = ctypes.c_size_t
        lib.sa_last_error.argtypes = []
        lib.sa_last_error.restype = ctypes.c_char_p
        lib.sa_version.argtypes = []
        lib.sa_version.restype = ctypes.c_char_p
        lib.sa_abi_version.argtypes = []
        lib.sa_abi_version.restype = ctypes.c_int
        if lib.sa_abi_version() != ABI_VERSION:
            raise RuntimeError(
                f"{LIB_NAME} implements ABI {lib.sa_abi_version()}, this binding expects {ABI_VERSION}; "
                "rebuild the library (`python -m archlab_amd.build`)")
        _lib = lib
    return _lib


def check(rc: int) -> None:
    """Map a C status code onto the reference's exception types."""
    if rc == SA_OK:
        return
    msg = load().sa_last_error().decode()
    if rc in (SA_ERR_INVALID, SA_ERR_UNSUPPORTED):
        raise ValueError(msg)
    raise RuntimeError(f"HIP error in simplicial kernel: {msg}")


INT32_MAX = 2 ** 31 - 1


def window(w) -> int:
    """A window length for an int32 ABI field.  Lengths beyond int32 select
    the same keys as INT32_MAX (no sequence or table reaches that far; the
    library clips further, to the sequence length or the table capacity)."""
    return min(int(w), INT32_MAX)


def dtype_code(dtype) -> int:
    if dtype == torch.float32:
        return SA_DTYPE_F32
    if dtype == torch.bfloat16:
        return SA_DTYPE_BF16
    raise ValueError("kernel supports float32/bfloat16")


def cache_dtype_code(dtype) -> int:
    """Element type of a paged cache: float32, bfloat16 or float16 (the
    reference's paged loads read any float cache, simplicial_paged.py:42-52)."""
    if dtype == torch.float16:
        return SA_DTYPE_F16
    if dtype in (torch.float32, torch.bfloat16):
        return dtype_code(dtype)
    raise ValueError("kernel supports float32/bfloat16/float16 caches")


def index_code(dtype) -> int:
    if dtype == torch.int32:
        return SA_INDEX_I32
    if dtype == torch.int64:
        return SA_INDEX_I64
    raise ValueError("invalid paged simplicial inputs")


def stream_handle(device) -> int:
    return torch.cuda.current_stream(device).cuda_stream
