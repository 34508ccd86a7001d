"""Drop-in for ``archlab.architectures.simplicial_deterministic.deterministic_simplicial_attention``
(simplicial_deterministic.py:107-111), forward only.

The reference's forward is the same computation as ``simplicial_attention``
in fp32 (simplicial_deterministic.py:83-84); its deterministic part is the
backward.  Here the forward kernels are deterministic by construction (fixed
reduction order, no atomics), so the call is ``simplicial_attention`` with
the reference's checks.  The reference forward passes no score scale to the
shared forward; the documented default of the equal-width API, 1/sqrt(D), is
used.
"""

from __future__ import annotations

import torch

from .simplicial_attention import simplicial_attention, validate_inputs


def deterministic_simplicial_attention(q, k1, k2, v1, v2, short_window, long_window):
    validate_inputs(q, k1, k2, v1, v2, short_window, long_window)
    if q.device.type != "cuda" or q.dtype != torch.float32 or q.shape[-1] not in (16, 32, 64, 128, 256):
        raise ValueError("deterministic simplicial core requires supported CUDA FP32 head geometry")
    return simplicial_attention(q, k1, k2, v1, v2, short_window, long_window)
