"""Drop-ins for the packed fp32 entry points of
``archlab.architectures.simplicial_packed``:

* ``packed_simplicial_attention`` (simplicial_packed.py:227-235): prefill with
  short window w1 <= 16, long window w2, head_dim 128, scale 1/sqrt(D),
  computed in fp32 (bf16 inputs are widened, as the reference does with its
  fp32 forward buffers) and returned in fp32;
* ``packed_simplicial_decode`` (simplicial_packed.py:290-338): one fp32 query
  against explicit windows of at most 16 short rows.

Both keep the reference's argument checks and messages.  The prefill runs on
the matrix cores with every fp32 operand split into hi + lo bf16 terms
(fp32-accurate, within 1e-4 of the fp64 oracle); its backward and the
decode's fp32 windows run on the library's kernels for fp32 inputs.
"""

from __future__ import annotations

import torch

from .simplicial_attention import _prefill_autograd, validate_inputs
from .window_decode import window_decode


def packed_simplicial_attention(q, k1, k2, v1, v2, w1, w2):
    """q [B,N,HQ,128] (fp32, or bf16); k1/k2/v1/v2 [B,N,HK,128] -> fp32 [B,N,HQ,128].

    Gradients flow through the library's backward (fp32, as the reference's
    fp32 buffers); being deterministic, the call is allowed under
    ``torch.use_deterministic_algorithms`` (a deviation: the reference raises).
    """
    validate_inputs(q, k1, k2, v1, v2, w1, w2, allow_scaled_query=True)
    if not q.is_cuda:
        raise ValueError("packed kernel requires CUDA")
    b, n, hq, d = q.shape
    if q.dtype not in (torch.float32, torch.bfloat16) or w1 > 16 or d != 128:
        raise ValueError("packed kernel requires FP32/BF16, head_dim=128, short window <=16")
    hk = k1.shape[2]
    xs = [x.float().contiguous() for x in (q, k1, k2, v1, v2)]
    q_ = xs[0].view(b * n, hq, d)
    k1_, k2_, v1_, v2_ = (x.view(b * n, hk, d) for x in xs[1:])
    out, _ = _prefill_autograd(q_, k1_, k2_, v1_, v2_, w1, w2, d ** -0.5, None, b, n, False, "auto")
    return out.view(b, n, hq, d)


def packed_simplicial_decode(q, k1, k2, v1, v2):
    """q [B,1,H,128] fp32; k1/v1 [B,N1<=16,HK,128]; k2/v2 [B,N2,HK,128] -> [B,1,H,128]."""
    if (
        q.ndim != 4
        or q.shape[1] != 1
        or q.shape[-1] != 128
        or q.dtype != torch.float32
        or not q.is_cuda
    ):
        raise ValueError("native packed decode requires CUDA FP32 [B,1,H,128]")
    if (
        k1.shape != v1.shape
        or k2.shape != v2.shape
        or k1.shape[0] != q.shape[0]
        or k2.shape[0] != q.shape[0]
        or k1.shape[2:] != k2.shape[2:]
        or k1.shape[-1] != 128
        or q.shape[2] % k1.shape[2]
        or not 1 <= k1.shape[1] <= min(16, k2.shape[1])
    ):
        raise ValueError("incompatible native decode windows")
    if any(x.dtype != q.dtype or x.device != q.device for x in (k1, k2, v1, v2)):
        raise ValueError("native decode inputs must share dtype/device")
    if torch.is_grad_enabled() and any(x.requires_grad for x in (q, k1, k2, v1, v2)):
        raise ValueError("decode is inference-only")
    out = window_decode(q[:, 0], k1, k2, v1, v2, 128 ** -0.5)
    return out[:, None]
