"""One query per sequence against explicit key windows, on the paged kernel.

The reference's contiguous decode entry points (``simplicial_decode_attention``,
``packed_simplicial_decode``, ``tilelang_decode``) take, per batch row, the
short-axis rows (k1, v1) [B, N1, HK, D] and the long-axis rows (k2, v2)
[B, N2, HK, D] that the single query attends to: every (j, k) pair of those
rows is valid.  This module expresses that as a paged call: the rows become
caches with a block size of one row, the query sits at position P, the long
rows occupy positions P-L+1 .. P and the short rows P-N1+1 .. P, and the two
block tables map each position to its row.  No data is rearranged on the
device beyond stacking K with V, and nothing is read back to the host.
"""

from __future__ import annotations

import torch

from .simplicial_paged import simplicial_paged_attention


def window_decode(q, k1, k2, v1, v2, scale, key_lower=0, kernel="auto"):
    """q [B, HQ, D]; k1/v1 [B, N1, HK, D]; k2/v2 [B, N2, HK, D].

    Returns the fp32 output [B, HQ, D] of one joint softmax over all pairs
    (j < N1, key_lower <= k < N2).  Requires N1 <= N2 - key_lower.
    """
    b, hq, d = q.shape
    n1, n2 = k1.shape[1], k2.shape[1]
    hk = k1.shape[2]
    length = n2 - key_lower
    if not 1 <= n1 <= length:
        raise ValueError("the short axis must not be longer than the long axis")
    dev = q.device
    # caches [2, rows, 1, HK, D]: block index = row index
    long_cache = torch.stack((k2, v2)).reshape(2, b * n2, 1, hk, d)
    short_cache = torch.stack((k1, v1)).reshape(2, b * n1, 1, hk, d)
    pos = length - 1  # query position; long rows key_lower.. sit at positions 0..length-1
    p = torch.arange(length, device=dev, dtype=torch.int64)
    rows = torch.arange(b, device=dev, dtype=torch.int64)[:, None]
    long_table = (rows * n2 + key_lower + p[None, :]).to(torch.int32)
    short_row = (p - (length - n1)).clamp_min(0)  # positions before the short window map to row 0 (unused)
    short_table = (rows * n1 + short_row[None, :]).to(torch.int32)
    token_seq = torch.arange(b, device=dev, dtype=torch.int32)
    token_pos = torch.full((b,), pos, device=dev, dtype=torch.int32)
    return simplicial_paged_attention(q, short_cache, long_cache, short_table, token_seq, token_pos,
                                      short_window=n1, long_window=length, scale=scale,
                                      long_block_table=long_table, kernel=kernel)
