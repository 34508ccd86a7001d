"""Determinant-score 2-simplicial attention on the same kernels.

Drop-ins for ``determinant_operands``, ``determinant_simplicial_attention``
and ``oriented_determinant_simplicial_attention``
(archlab/architectures/simplicial_attention.py:100-202).

The score of (q, k1_j, k2_k) is the sum, over consecutive chunks of three
coordinates, of the signed determinant det([q; k1_j; k2_k]) (Fast and
Simplex, sec. 5, eq. 9; the trailing ``dim % 3`` coordinates take no part).
By Sarrus' rule each chunk's determinant is

    sum_c a_c b_{c+1} d_{c+2}  -  sum_c a_c b_{c+2} d_{c+1}      (indices mod 3)

so the whole score is one elementwise trilinear form over 2 * used
coordinates: the operands below are that expansion, zero-padded to a power
of two (at least 16), and the attention itself is the ordinary
``simplicial_attention`` with score width DS = padded width and the value
width DV unchanged.  Gradients flow through the expansion into the library's
backward.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from .simplicial_attention import _score_scale, simplicial_attention, validate_inputs


def _sarrus_indices(dim, device):
    """(used, first, second): per 3-chunk, coordinate c maps to c+1 (first) and c+2 (second), mod 3."""
    if dim < 3:
        raise ValueError("determinant scores require at least 3 coordinates")
    used = dim - dim % 3
    coord = torch.arange(used, device=device)
    chunk_base = coord - coord % 3
    first = chunk_base + (coord % 3 + 1) % 3
    second = chunk_base + (coord % 3 + 2) % 3
    return used, first, second


def determinant_operands(q, k1, k2):
    """Expanded (q, k1, k2) whose elementwise trilinear form is the chunked determinant sum.

    Layout (last dimension, width = max(16, next power of two >= 2*used)):
    q -> [q_c, -q_c, 0...], k1 -> [k1_{c+1}, k1_{c+2}, 0...],
    k2 -> [k2_{c+2}, k2_{c+1}, 0...], c over the first ``used`` coordinates
    (simplicial_attention.py:111-129).
    """
    used, first, second = _sarrus_indices(q.shape[-1], q.device)
    if k1.shape[-1] != q.shape[-1] or k2.shape[-1] != q.shape[-1]:
        raise ValueError("determinant operands must have matching score widths")
    width = max(16, 1 << (2 * used - 1).bit_length())
    tail = width - 2 * used

    def expand(x, lo, hi, neg_hi):
        a = x.index_select(-1, lo)
        b = x.index_select(-1, hi)
        return F.pad(torch.cat((a, -b if neg_hi else b), dim=-1), (0, tail))

    keep = torch.arange(used, device=q.device)
    return expand(q, keep, keep, True), expand(k1, first, second, False), expand(k2, second, first, False)


def determinant_simplicial_attention(q, k1, k2, v1, v2, short_window, long_window, *, scale=None,
                                     return_lse=False, kernel="auto"):
    """simplicial_attention.py:132-148: causal attention with chunked 3x3 determinants as scores.

    q [B,N,HQ,D], k1/k2 [B,N,HK,D], v1/v2 [B,N,HK,DV]; D >= 3.  The default
    scale is 1/sqrt(D) of the original score width (not of the padded
    expansion).  Returns O [B,N,HQ,DV] (and the natural-log LSE with
    ``return_lse``); differentiable in all five inputs.
    """
    validate_inputs(q, k1, k2, v1, v2, short_window, long_window, allow_value_dim=True)
    scale = _score_scale(scale, q.shape[-1])
    qs, k1s, k2s = determinant_operands(q, k1, k2)
    return simplicial_attention(qs, k1s, k2s, v1, v2, short_window, long_window, scale=scale,
                                return_lse=return_lse, kernel=kernel)


def oriented_determinant_simplicial_attention(q, k1, k2, v1, v2, window_1, window_2, *, scale=None,
                                              backend="kernel"):
    """simplicial_attention.py:181-202: determinant attention for any positive (window_1, window_2).

    ``window_1`` bounds the (k1, v1) causal prefix and ``window_2`` the
    (k2, v2) one.  When window_1 > window_2 the axes are exchanged using
    det([-q; k2; k1]) == det([q; k1; k2]) and v2 * v1 == v1 * v2, so that the
    shorter window is always the kernel's short axis.

    Deviation: only ``backend="kernel"`` is provided.  The reference's
    ``backend="reference"`` runs its torch determinant oracle, which is test
    infrastructure and not part of this library; it raises ``ValueError``.
    """
    if type(window_1) is not int or type(window_2) is not int or min(window_1, window_2) < 1:
        raise ValueError("window_1 and window_2 must be positive integers")
    if backend not in ("kernel", "reference"):
        raise ValueError("backend must be kernel or reference")
    if backend == "reference":
        raise ValueError("backend='reference' (the torch determinant oracle) is not shipped by this library")
    if window_1 <= window_2:
        return determinant_simplicial_attention(q, k1, k2, v1, v2, window_1, window_2, scale=scale)
    return determinant_simplicial_attention(-q, k2, k1, v2, v1, window_2, window_1, scale=scale)
