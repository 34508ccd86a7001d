"""2-simplicial attention over paged K/V caches (serving form) on MI355X.

Drop-in for ``archlab.architectures.simplicial_paged.simplicial_paged_attention``
(simplicial_paged.py:68-128).  Each query token carries its own sequence index
and absolute position, so one launch serves prefill, chunked prefill, decode
and mixed batches.  Short-window (k1/v1) and long-window (k2/v2) keys are
gathered through one block table per cache.  Cache layout per branch:
[2 (K, V), blocks, block_size, kv_heads, head_dim] with arbitrary strides.

Launch shapes depend only on tensor metadata and nothing is read back to the
host, so the call can be captured into a CUDA/HIP graph.
"""

from __future__ import annotations

import ctypes

import torch

from .. import _native
from .simplicial_attention import _kernel_flag


def _paged_args(q, short_cache, long_cache, block_table, long_block_table, token_seq, token_pos,
                short_window, long_window, scale, splits, out, lse, flags, plan_only=False, window_caps=None):
    tokens, heads, dim = q.shape
    return _native.PagedArgs(
        q=q.data_ptr(), q_stride_t=q.stride(0), q_stride_h=q.stride(1),
        short_cache=short_cache.data_ptr(), sc_stride=(ctypes.c_int64 * 4)(*short_cache.stride()[:4]),
        long_cache=long_cache.data_ptr(), lc_stride=(ctypes.c_int64 * 4)(*long_cache.stride()[:4]),
        short_table=block_table.data_ptr(), st_stride=block_table.stride(0),
        long_table=long_block_table.data_ptr(), lt_stride=long_block_table.stride(0),
        token_seq=token_seq.data_ptr(), token_pos=token_pos.data_ptr(),
        out=out.data_ptr() if out is not None else (256 if plan_only else None),
        o_stride_t=out.stride(0) if out is not None else heads * dim,
        o_stride_h=out.stride(1) if out is not None else dim,
        lse=lse.data_ptr() if lse is not None else None,
        tokens=tokens, heads_q=heads, heads_kv=short_cache.shape[3], head_dim=dim,
        block_size=short_cache.shape[2], num_seqs=min(block_table.shape[0], long_block_table.shape[0]),
        short_table_width=block_table.shape[1], long_table_width=long_block_table.shape[1],
        short_blocks=short_cache.shape[1], long_blocks=long_cache.shape[1],
        short_window=_native.window(short_window), long_window=_native.window(long_window),
        splits=0 if splits is None else min(int(splits), _native.INT32_MAX), scale=float(scale),
        q_dtype=_native.dtype_code(q.dtype), cache_dtype=_native.cache_dtype_code(short_cache.dtype),
        long_cache_dtype=_native.cache_dtype_code(long_cache.dtype),
        table_index_dtype=_native.index_code(block_table.dtype),
        long_table_index_dtype=_native.index_code(long_block_table.dtype),
        token_index_dtype=_native.index_code(token_seq.dtype),
        token_pos_index_dtype=_native.index_code(token_pos.dtype), flags=flags,
        token_window_caps=window_caps.data_ptr() if window_caps is not None else None)


def simplicial_paged_attention(q, short_cache, long_cache, block_table, token_seq, token_pos, *,
                               short_window, long_window, scale, long_block_table=None, splits=None,
                               return_lse=False, kernel="auto"):
    """q [tokens, query_heads, D]; returns FP32 [tokens, query_heads, D].

    ``long_window`` bounds the K2/V2 axis (pass a value >= the longest sequence
    for global layers).  ``block_table`` indexes the short cache and, unless
    ``long_block_table`` is given, also the long cache.  Block zero may be the
    null block; every slot inside a token's windows must be allocated.
    ``splits`` fixes the number of long-window partitions (default: chosen
    from the launch size); results for different split counts agree to
    rounding and, for a fixed split count, are bitwise reproducible.  With
    ``return_lse=True`` also returns the natural-log LSE [tokens, heads] fp32.
    """
    long_block_table = block_table if long_block_table is None else long_block_table
    if q.ndim != 3 or short_cache.ndim != 5 or long_cache.ndim != 5:
        raise ValueError("expected q [T,H,D] and caches [2,blocks,block,Hk,D]")
    tokens, heads, dim = q.shape
    if (short_cache.shape[0] != 2 or long_cache.shape[0] != 2
            or short_cache.shape[2:] != long_cache.shape[2:]
            or short_cache.shape[-1] != dim or heads % short_cache.shape[3]
            or dim not in (16, 32, 64, 128, 256)):
        raise ValueError("incompatible paged simplicial geometry")
    if not 1 <= short_window <= long_window:
        raise ValueError("require 1 <= short_window <= long_window")
    if (q.device.type != "cuda" or q.dtype not in (torch.float32, torch.bfloat16)
            or any(x.device != q.device for x in (short_cache, long_cache, block_table, long_block_table,
                                                   token_seq, token_pos))
            or any(x.dtype not in (torch.int32, torch.int64)
                   for x in (block_table, long_block_table, token_seq, token_pos))
            or token_seq.shape != (tokens,) or token_pos.shape != (tokens,)
            or block_table.ndim != 2 or long_block_table.ndim != 2):
        raise ValueError("invalid paged simplicial inputs")
    # the reference reads the caches in any float dtype its loads accept
    # (simplicial_paged.py:42-52); this library takes float32, bfloat16 and
    # float16 caches, each axis on its own
    if any(x.dtype not in (torch.float32, torch.bfloat16, torch.float16) for x in (short_cache, long_cache)):
        raise ValueError("kernel supports float32/bfloat16/float16 caches")
    if (q.stride(-1) != 1 or short_cache.stride(-1) != 1 or long_cache.stride(-1) != 1
            or block_table.stride(-1) != 1 or long_block_table.stride(-1) != 1):
        raise ValueError("innermost dimensions must be contiguous")
    kv_heads = short_cache.shape[3]
    if heads // kv_heads > 128:
        raise ValueError("at most 128 query heads per KV group")
    if splits is not None and int(splits) < 1:
        raise ValueError("splits must be a positive integer")
    if torch.is_grad_enabled() and q.requires_grad:
        raise ValueError("simplicial_paged_attention is inference-only")
    return _paged_launch(q, short_cache, long_cache, block_table, long_block_table, token_seq, token_pos,
                         short_window, long_window, scale, splits, return_lse, kernel)


def _paged_launch(q, short_cache, long_cache, block_table, long_block_table, token_seq, token_pos,
                  short_window, long_window, scale, splits, return_lse, kernel, window_caps=None):
    """The launch behind ``simplicial_paged_attention`` on validated inputs.
    The caches may be any objects with ``data_ptr()``, ``stride()``,
    ``shape`` and ``dtype`` describing [2, blocks, block_size, HK, D]
    (``window_decode`` passes separate K and V tensors that way).
    ``window_caps`` (int32 [tokens, 2] on the device, optional) limits each
    token's short and long windows further."""
    tokens, heads, dim = q.shape
    flags = _kernel_flag(kernel)
    if tokens == 0:
        out = torch.empty((0, heads, dim), device=q.device, dtype=torch.float32)
        return (out, torch.empty((0, heads), device=q.device, dtype=torch.float32)) if return_lse else out
    token_seq, token_pos = token_seq.contiguous(), token_pos.contiguous()
    lib = _native.load()
    out = torch.empty((tokens, heads, dim), device=q.device, dtype=torch.float32)
    lse = torch.empty((tokens, heads), device=q.device, dtype=torch.float32) if return_lse else None
    if window_caps is not None:
        window_caps = window_caps.to(torch.int32).contiguous()
    args = _paged_args(q, short_cache, long_cache, block_table, long_block_table, token_seq, token_pos,
                       short_window, long_window, scale, splits, out, lse, flags, window_caps=window_caps)
    if kernel == "mfma" and lib.sa_paged_kernel(ctypes.byref(args)) != b"mfma":
        raise ValueError("the MFMA kernel does not cover this dtype / head_dim / layout")
    nbytes = lib.sa_paged_workspace_bytes(ctypes.byref(args))
    workspace = torch.empty(max(nbytes, 1) + 256, device=q.device, dtype=torch.uint8)
    base = workspace.data_ptr()
    aligned = (base + 255) & ~255
    with torch.cuda.device(q.device):
        _native.check(lib.sa_paged_fwd(ctypes.byref(args), aligned, nbytes,
                                       _native.stream_handle(q.device)))
    return (out, lse) if return_lse else out


def paged_plan(q, short_cache, long_cache, block_table, token_seq, token_pos, *, short_window,
               long_window, scale=1.0, long_block_table=None, splits=None, kernel="auto"):
    """(kernel family, splits, workspace bytes) a call with these tensors would use."""
    long_block_table = block_table if long_block_table is None else long_block_table
    lib = _native.load()
    args = _paged_args(q, short_cache, long_cache, block_table, long_block_table, token_seq, token_pos,
                       short_window, long_window, scale, splits, None, None, _kernel_flag(kernel), plan_only=True)
    name = lib.sa_paged_kernel(ctypes.byref(args))
    return (None if name is None else name.decode(), lib.sa_paged_splits(ctypes.byref(args)),
            lib.sa_paged_workspace_bytes(ctypes.byref(args)))
