"""2-simplicial (trilinear) sliding-window attention on MI355X: prefill forms.

Drop-in for ``archlab.architectures.simplicial_attention`` on the forward
path.  Tensor layout is [batch, sequence, heads, head_dim]; the score is
``scale * sum_d q_i[d] * k1_j[d] * k2_k[d]`` with ``j`` in the causal short
window and ``k`` in the causal long window, one joint softmax over all valid
(j, k) pairs, and the output ``sum_jk P_ijk * (v1_j ⊙ v2_k)``.

The computation runs in hand-written gfx950 HIP kernels
(``libsimplicial_mi355x.so``, C ABI in ``include/simplicial_mi355x.h``); this
module only validates, allocates outputs with torch's caching allocator and
passes pointers.  There is no CPU path here: non-GPU tensors raise, exactly
as the reference does.
"""

from __future__ import annotations

import ctypes
import math
from numbers import Real

import torch

from .. import _native


def validate_inputs(q, k1, k2, v1, v2, short_window, long_window, *,
                    allow_scaled_query=False, allow_value_dim=False):
    """Contract checks with the reference's messages (simplicial_attention.py:17-38)."""
    if q.ndim != 4 or any(x.ndim != 4 for x in (k1, k2, v1, v2)):
        raise ValueError("expected [batch, sequence, heads, head_dim]")
    if min(short_window, long_window) < 1 or short_window > long_window:
        raise ValueError("require 1 <= short_window <= long_window")
    b, n, heads, d = q.shape
    if min(b, n, heads, d) < 1:
        raise ValueError("empty attention dimensions are unsupported")
    if k2.shape != k1.shape or v2.shape != v1.shape or v1.shape[:3] != k1.shape[:3]:
        raise ValueError("both key/value branches must have matching batch, sequence and heads")
    if v1.shape[-1] < 1 or (not allow_value_dim and v1.shape[-1] != d):
        raise ValueError("unsupported value head dimension")
    if k1.shape[2] < 1 or k1.shape[:2] != (b, n) or k1.shape[-1] != d or heads % k1.shape[2]:
        raise ValueError("incompatible grouped-query geometry")
    dtype = (
        k1.dtype
        if allow_scaled_query and q.dtype == torch.float32 and k1.dtype == torch.bfloat16
        else q.dtype
    )
    if any(x.dtype != dtype or x.device != q.device for x in (k1, k2, v1, v2)):
        raise ValueError("all inputs must have the same dtype and device")


def _score_scale(scale, dim):
    """simplicial_attention.py:41-46: None -> 1/sqrt(score_dim), else a finite real."""
    if scale is None:
        return 1 / math.sqrt(dim)
    if not isinstance(scale, Real) or not math.isfinite(scale):
        raise ValueError("scale must be a finite real number")
    return float(scale)


def _kernel_checks(q, v_dim, score_dim):
    """simplicial_attention.py:87-92 device / dtype / head-dim contract."""
    if q.device.type != "cuda" or q.dtype not in (torch.float32, torch.bfloat16):
        raise ValueError("kernel supports CUDA float32/bfloat16")
    if score_dim not in (16, 32, 64, 128, 256, 512):
        raise ValueError("unsupported score head dimension")
    if v_dim not in (16, 32, 64, 128, 256):
        raise ValueError("unsupported value head dimension")


def _forward_only(*tensors):
    if torch.is_grad_enabled() and any(t.requires_grad for t in tensors):
        raise ValueError("this entry point is forward-only: no backward kernel is provided for it")


def _needs_grad(*tensors):
    return torch.is_grad_enabled() and any(t.requires_grad for t in tensors)


def _kernel_flag(kernel):
    if kernel not in ("auto", "mfma", "generic"):
        raise ValueError("kernel must be 'auto', 'mfma' or 'generic'")
    return _native.SA_FLAG_FORCE_GENERIC if kernel == "generic" else 0


def _prefill(q, k1, k2, v1, v2, short_window, long_window, scale, cu_seqlens, num_seqs, seqlen,
             return_lse, kernel):
    """q [T,HQ,D], k [T,HK,D], v [T,HK,DV] contiguous -> out [T,HQ,DV], lse [T,HQ]."""
    lib = _native.load()
    tokens, hq, d = q.shape
    hk, dv = k1.shape[1], v1.shape[-1]
    if hq // hk > 128:
        raise ValueError("at most 128 query heads per KV group")
    out = torch.empty((tokens, hq, dv), device=q.device, dtype=q.dtype)
    lse = torch.empty((tokens, hq), device=q.device, dtype=torch.float32) if return_lse else None
    args = _native.PrefillArgs(
        q=q.data_ptr(), k1=k1.data_ptr(), k2=k2.data_ptr(), v1=v1.data_ptr(), v2=v2.data_ptr(),
        out=out.data_ptr(), lse=lse.data_ptr() if lse is not None else None,
        cu_seqlens=cu_seqlens.data_ptr() if cu_seqlens is not None else None,
        q_stride_t=q.stride(0), q_stride_h=q.stride(1),
        k_stride_t=k1.stride(0), k_stride_h=k1.stride(1),
        v_stride_t=v1.stride(0), v_stride_h=v1.stride(1),
        o_stride_t=out.stride(0), o_stride_h=out.stride(1), lse_stride_t=hq,
        num_seqs=num_seqs, seqlen=seqlen, total_tokens=tokens,
        heads_q=hq, heads_kv=hk, head_dim=d, value_dim=dv,
        short_window=_native.window(short_window), long_window=_native.window(long_window),
        scale=scale, dtype=_native.dtype_code(q.dtype), flags=_kernel_flag(kernel))
    workspace = None
    if q.dtype == torch.float32:
        # fp32 inputs run on the matrix cores with a workspace for the hi/lo
        # split of k2, v2, v1 (torch's caching allocator; freed with the call's
        # stream order preserved)
        nbytes = lib.sa_prefill_workspace_bytes(ctypes.byref(args))
        if nbytes:
            workspace = torch.empty(nbytes + 256, device=q.device, dtype=torch.uint8)
            args.workspace = (workspace.data_ptr() + 255) & ~255
            args.workspace_bytes = nbytes
    if kernel == "mfma" and lib.sa_prefill_kernel(ctypes.byref(args)) != b"mfma":
        raise ValueError("the MFMA kernel does not cover this dtype / head_dim / layout")
    with torch.cuda.device(q.device):
        _native.check(lib.sa_prefill_fwd(ctypes.byref(args), _native.stream_handle(q.device)))
    return out, lse


def _backward(q, k1, k2, v1, v2, out, lse, dout, dlse, short_window, long_window, scale, cu_seqlens, num_seqs,
              seqlen, kernel="auto"):
    """Gradients of q, k1, k2, v1, v2 ([T,H,*] contiguous) through the C ABI."""
    lib = _native.load()
    tokens, hq, d = q.shape
    hk, dv = k1.shape[1], v1.shape[-1]
    dout = dout.contiguous()
    grads = [torch.empty_like(x) for x in (q, k1, k2, v1, v2)]
    dq, dk1, dk2, dv1, dv2 = grads
    fwd = _native.PrefillArgs(
        q=q.data_ptr(), k1=k1.data_ptr(), k2=k2.data_ptr(), v1=v1.data_ptr(), v2=v2.data_ptr(),
        out=out.data_ptr(), lse=lse.data_ptr(),
        cu_seqlens=cu_seqlens.data_ptr() if cu_seqlens is not None else None,
        q_stride_t=q.stride(0), q_stride_h=q.stride(1), k_stride_t=k1.stride(0), k_stride_h=k1.stride(1),
        v_stride_t=v1.stride(0), v_stride_h=v1.stride(1), o_stride_t=out.stride(0), o_stride_h=out.stride(1),
        lse_stride_t=hq, num_seqs=num_seqs, seqlen=seqlen, total_tokens=tokens,
        heads_q=hq, heads_kv=hk, head_dim=d, value_dim=dv,
        short_window=_native.window(short_window), long_window=_native.window(long_window), scale=scale,
        dtype=_native.dtype_code(q.dtype), flags=_kernel_flag(kernel))
    if dlse is not None:
        dlse = dlse.float().contiguous()
    args = _native.PrefillBwdArgs(
        fwd=fwd, dout=dout.data_ptr(), do_stride_t=dout.stride(0), do_stride_h=dout.stride(1),
        dq=dq.data_ptr(), dq_stride_t=dq.stride(0), dq_stride_h=dq.stride(1),
        dk1=dk1.data_ptr(), dk2=dk2.data_ptr(), dk_stride_t=dk1.stride(0), dk_stride_h=dk1.stride(1),
        dv1=dv1.data_ptr(), dv2=dv2.data_ptr(), dv_stride_t=dv1.stride(0), dv_stride_h=dv1.stride(1),
        dlse=dlse.data_ptr() if dlse is not None else None, dlse_stride_t=hq)
    nbytes = lib.sa_prefill_bwd_workspace_bytes(ctypes.byref(args))
    try:
        workspace = torch.empty(max(nbytes, 1) + 256, device=q.device, dtype=torch.uint8)
    except torch.cuda.OutOfMemoryError:
        # the dq pass's dk1 partials (16-17.5x the bytes of q) do not fit:
        # compute dk1 in its own pass, with the small workspace
        args.fwd.flags |= _native.SA_FLAG_SEPARATE_DK1
        nbytes = lib.sa_prefill_bwd_workspace_bytes(ctypes.byref(args))
        workspace = torch.empty(max(nbytes, 1) + 256, device=q.device, dtype=torch.uint8)
    aligned = (workspace.data_ptr() + 255) & ~255
    with torch.cuda.device(q.device):
        _native.check(lib.sa_prefill_bwd(ctypes.byref(args), aligned, nbytes, _native.stream_handle(q.device)))
    return grads


class _SimplicialFunction(torch.autograd.Function):
    """Forward kernels + the atomics-free backward (sa_prefill_bwd) on [T, H, *] tensors."""

    @staticmethod
    def forward(ctx, q, k1, k2, v1, v2, short_window, long_window, scale, cu_seqlens, num_seqs, seqlen, kernel):
        out, lse = _prefill(q, k1, k2, v1, v2, short_window, long_window, scale, cu_seqlens, num_seqs, seqlen,
                            True, kernel)
        ctx.save_for_backward(q, k1, k2, v1, v2, out, lse)
        ctx.cu_seqlens = cu_seqlens
        ctx.meta = (short_window, long_window, scale, num_seqs, seqlen, kernel)
        return out, lse

    @staticmethod
    def backward(ctx, dout, dlse):
        q, k1, k2, v1, v2, out, lse = ctx.saved_tensors
        short_window, long_window, scale, num_seqs, seqlen, kernel = ctx.meta
        if dout is None:
            dout = torch.zeros_like(out)
        grads = _backward(q, k1, k2, v1, v2, out, lse, dout, dlse, short_window, long_window, scale,
                          ctx.cu_seqlens, num_seqs, seqlen, "generic" if kernel == "generic" else "auto")
        return (*grads, None, None, None, None, None, None, None)


def _prefill_autograd(q, k1, k2, v1, v2, short_window, long_window, scale, cu_seqlens, num_seqs, seqlen,
                      return_lse, kernel):
    if _needs_grad(q, k1, k2, v1, v2):
        out, lse = _SimplicialFunction.apply(q, k1, k2, v1, v2, short_window, long_window, scale, cu_seqlens,
                                             num_seqs, seqlen, kernel)
        return out, (lse if return_lse else None)
    return _prefill(q, k1, k2, v1, v2, short_window, long_window, scale, cu_seqlens, num_seqs, seqlen,
                    return_lse, kernel)


def _padded_width(d, dv, dtype, kernel):
    """Width to which a call with score width ``d`` and value width ``dv``
    is zero-padded to run on the matrix cores, or None.  Widths 16 and 32
    (the reference's qualification gate runs D = 32,
    qualification/simplicial_attention.py:42-44; its scratch-scaling recipes
    use D = 16) pad to 64 (or to the other width): zero coordinates add
    exactly nothing to a score, padded value columns are sliced off, and the
    backward reaches the unpadded tensors through the pad.  Only for
    ``kernel="auto"``; "mfma" and "generic" take the shapes as given."""
    if kernel != "auto" or (d >= 64 and dv >= 64):
        return None
    w = max(64, d, dv)
    if w not in (64, 128, 256) or (dtype == torch.float32 and w > 128):
        return None
    return w


def _pad_last(x, w):
    return x if x.shape[-1] == w else torch.nn.functional.pad(x, (0, w - x.shape[-1]))


def simplicial_attention(q, k1, k2, v1, v2, short_window, long_window, *, scale=None,
                         return_lse=False, kernel="auto"):
    """Drop-in for ``simplicial_attention`` (simplicial_attention.py:77-97), forward only.

    q [B,N,HQ,D]; k1, k2 [B,N,HK,D]; v1, v2 [B,N,HK,DV].  Returns O
    [B,N,HQ,DV] in q's dtype and, with ``return_lse=True``, also the
    natural-log LSE [B,N,HQ] in float32.  ``kernel`` selects the
    implementation: "auto" (bf16 with D == DV in {64,128,256}, or with
    (D, DV) = (128, 64) / (256, 128) as the determinant expansion produces,
    and fp32 with D == DV in {64, 128} run on the MFMA kernel; widths 16 and
    32 are zero-padded to 64 to run there too; everything else on the
    portable kernel), "mfma" (raise if not covered) or "generic".

    Inputs that require grad get gradients from the library's backward
    (``sa_prefill_bwd``: atomics-free, bitwise reproducible; MFMA tiles for
    bf16 with D and DV each 64 or 128, or D = 256 over DV = 128 / 256,
    portable kernels otherwise and with
    ``kernel="generic"``).  Deviation from
    the reference: forward and backward are deterministic, so
    ``torch.use_deterministic_algorithms(True)`` is allowed.
    """
    validate_inputs(q, k1, k2, v1, v2, short_window, long_window, allow_value_dim=True)
    scale = _score_scale(scale, q.shape[-1])
    _kernel_checks(q, v1.shape[-1], q.shape[-1])
    b, n, hq, d = q.shape
    hk, dv = k1.shape[2], v1.shape[-1]
    w = _padded_width(d, dv, q.dtype, kernel)
    if w is not None:
        q, k1, k2, v1, v2 = (_pad_last(x, w) for x in (q, k1, k2, v1, v2))
    dp, dvp = q.shape[-1], v1.shape[-1]
    q_, k1_, k2_ = (x.contiguous().view(b * n, -1, dp) for x in (q, k1, k2))
    v1_, v2_ = (x.contiguous().view(b * n, hk, dvp) for x in (v1, v2))
    out, lse = _prefill_autograd(q_, k1_, k2_, v1_, v2_, short_window, long_window, scale, None, b, n,
                                 return_lse, kernel)
    out = out.view(b, n, hq, dvp)[..., :dv]
    if return_lse:
        return out, lse.view(b, n, hq)
    return out


def simplicial_varlen_attention(q, k1, k2, v1, v2, cu_seqlens, short_window, long_window, *,
                                scale=None, return_lse=False, kernel="auto"):
    """Packed variable-length prefill: q [T,HQ,D], k1/k2 [T,HK,D], v1/v2 [T,HK,DV].

    ``cu_seqlens`` is int32 [num_seqs + 1] on q's device (cu[0] = 0,
    cu[-1] = T, non-decreasing).  Each sequence is attended on its own, i.e.
    the result equals ``simplicial_attention`` applied to every
    ``[cu[s], cu[s+1])`` slice ("same-document" visibility,
    recipes/deepseek_v41/proposals.yaml:76).  The offsets are not read back to
    the host; a malformed ``cu_seqlens`` yields meaningless values but never
    addresses memory outside the tensors.
    """
    if q.ndim != 3 or any(x.ndim != 3 for x in (k1, k2, v1, v2)):
        raise ValueError("expected packed [tokens, heads, head_dim]")
    validate_inputs(q[None], k1[None], k2[None], v1[None], v2[None], short_window, long_window,
                    allow_value_dim=True)
    scale = _score_scale(scale, q.shape[-1])
    _kernel_checks(q, v1.shape[-1], q.shape[-1])
    if (cu_seqlens.ndim != 1 or cu_seqlens.dtype != torch.int32 or cu_seqlens.numel() < 2
            or cu_seqlens.device != q.device):
        raise ValueError("cu_seqlens must be int32 [num_seqs + 1] on the input device")
    t, hq, d = q.shape
    dv = v1.shape[-1]
    w = _padded_width(d, dv, q.dtype, kernel)
    if w is not None:
        q, k1, k2, v1, v2 = (_pad_last(x, w) for x in (q, k1, k2, v1, v2))
    q_, k1_, k2_, v1_, v2_ = (x.contiguous() for x in (q, k1, k2, v1, v2))
    out, lse = _prefill_autograd(q_, k1_, k2_, v1_, v2_, short_window, long_window, scale,
                                 cu_seqlens.contiguous(), cu_seqlens.numel() - 1, 0, return_lse, kernel)
    out = out[..., :dv]
    return (out, lse) if return_lse else out


def prefill_kernel_name(q, k1, v1, *, kernel="auto"):
    """Which kernel family ('mfma' or 'generic') a dense call with these shapes
    runs ('mfma' also for widths the shim zero-pads onto the matrix cores)."""
    lib = _native.load()
    b, n, hq, d = q.shape
    hk, dv = k1.shape[2], v1.shape[-1]
    w = _padded_width(d, dv, q.dtype, kernel)
    if w is not None:
        d = dv = w
    args = _native.PrefillArgs(
        q=16, k1=16, k2=16, v1=16, v2=16, out=16,
        q_stride_t=hq * d, q_stride_h=d, k_stride_t=hk * d, k_stride_h=d,
        v_stride_t=hk * dv, v_stride_h=dv, o_stride_t=hq * dv, o_stride_h=dv, lse_stride_t=hq,
        num_seqs=b, seqlen=n, total_tokens=b * n, heads_q=hq, heads_kv=hk, head_dim=d,
        value_dim=dv, short_window=1, long_window=1, scale=1.0,
        dtype=_native.dtype_code(q.dtype), flags=_kernel_flag(kernel))
    # a call passes the workspace the fp32 matrix-core path asks for
    args.workspace_bytes = lib.sa_prefill_workspace_bytes(ctypes.byref(args))
    args.workspace = 256 if args.workspace_bytes else None
    name = lib.sa_prefill_kernel(ctypes.byref(args))
    return None if name is None else name.decode()
