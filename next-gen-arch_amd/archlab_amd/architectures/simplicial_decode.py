"""One-token contiguous decode: drop-in for
``archlab.architectures.simplicial_decode.simplicial_decode_attention``
(simplicial_decode.py:47-72).

The query attends to every pair of its explicit windows: the N1 short rows
(k1, v1) and the N2 long rows (k2, v2), scale 1/sqrt(D), fp32 throughout.
It runs on the paged kernel (``window_decode``).
"""

from __future__ import annotations

import torch

from .window_decode import window_decode


def simplicial_decode_attention(q, k1, k2, v1, v2):
    """q [B,1,HQ,D], k1/v1 [B,N1,HK,D], k2/v2 [B,N2,HK,D] (N1 <= N2), fp32 -> [B,1,HQ,D]."""
    if (q.ndim != 4 or q.shape[1] != 1 or any(x.ndim != 4 for x in (k1, k2, v1, v2))
            or min(q.shape) < 1 or min(k1.shape) < 1 or min(k2.shape) < 1
            or k1.shape != v1.shape or k2.shape != v2.shape
            or k1.shape[0] != q.shape[0] or k2.shape[0] != q.shape[0]
            or k1.shape[2:] != k2.shape[2:] or q.shape[-1] != k1.shape[-1]
            or q.shape[2] % k1.shape[2] or min(k1.shape[1], k2.shape[1]) < 1
            or k1.shape[1] > k2.shape[1]):
        raise ValueError("incompatible one-query simplicial windows")
    if (q.device.type != "cuda" or q.dtype != torch.float32 or q.shape[-1] not in (16, 32, 64, 128, 256)
            or any(x.device != q.device or x.dtype != q.dtype for x in (k1, k2, v1, v2))):
        raise ValueError("simplicial decode requires CUDA FP32 projections")
    if torch.is_grad_enabled() and any(x.requires_grad for x in (q, k1, k2, v1, v2)):
        raise ValueError("simplicial decode has no backward; use the training kernel")
    if q.shape[2] // k1.shape[2] > 128:
        raise ValueError("at most 128 query heads per KV group")
    out = window_decode(q[:, 0], k1, k2, v1, v2, q.shape[-1] ** -0.5)
    return out[:, None]
