"""Write the small fp64 golden fixtures under tests/golden/.

The expected outputs are NOT produced by the oracle under test: they come from
a brute-force formulation (all (i, j, k) scores as one 5-D einsum, an explicit
window mask, one softmax over the flattened (j, k) pairs), the form the
reference's own CPU test uses to pin its oracle
(tests/test_simplicial_attention.py:37-46 in the reference).  The reference
repository ships no numeric golden vectors for this path, so these files pin
the CPU oracle against an independent evaluation and give the GPU tests a
fixed, committed target.

Run:  python tests/golden/make_golden.py   (writes simplicial_golden.npz)
"""

from __future__ import annotations

import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))

# (name, batch, seqlen, heads_q, heads_kv, dim, short_window, long_window, seed)
CASES = [
    ("gqa_tiny", 1, 9, 4, 2, 4, 2, 3, 42),
    ("mha_small", 2, 17, 2, 2, 8, 3, 8, 7),
    ("mqa_unaligned", 1, 40, 3, 1, 16, 5, 33, 11),
    ("single_pair", 1, 6, 2, 2, 4, 1, 1, 5),
    ("equal_windows", 1, 12, 2, 1, 8, 4, 4, 9),
    ("global_long", 1, 21, 2, 2, 8, 3, 10_000, 13),
    # head dims the GPU kernels accept (16..512)
    ("gqa_d32", 1, 24, 4, 2, 32, 4, 9, 17),
    ("mha_d16_long", 2, 19, 2, 2, 16, 2, 10_000, 19),
]


def brute_force(q, k1, k2, v1, v2, short_window, long_window, scale):
    """All-pairs evaluation with an explicit mask; returns O [B,N,H,D], LSE [B,N,H]."""
    groups = q.shape[2] // k1.shape[2]
    k1, k2, v1, v2 = (x.repeat_interleave(groups, dim=2) for x in (k1, k2, v1, v2))
    n = q.shape[1]
    scores = torch.einsum("bihd,bjhd,bkhd->bhijk", q, k1, k2) * scale
    i, j, k = torch.meshgrid(*(torch.arange(n) for _ in range(3)), indexing="ij")
    mask = (j <= i) & (k <= i) & (j > i - short_window) & (k > i - long_window)
    masked = scores.masked_fill(~mask, -float("inf"))
    flat = masked.flatten(-2)
    p = flat.softmax(-1).reshape_as(scores)
    out = torch.einsum("bhijk,bjhd,bkhd->bihd", p, v1, v2)
    lse = torch.logsumexp(flat, -1).permute(0, 2, 1)
    return out, lse


def make():
    arrays = {}
    for name, b, n, hq, hk, d, ws, wl, seed in CASES:
        g = torch.Generator().manual_seed(seed)
        q = torch.randn(b, n, hq, d, generator=g, dtype=torch.float64)
        k1, k2, v1, v2 = (torch.randn(b, n, hk, d, generator=g, dtype=torch.float64) for _ in range(4))
        scale = d ** -0.5
        out, lse = brute_force(q, k1, k2, v1, v2, ws, wl, scale)
        for key, val in (("q", q), ("k1", k1), ("k2", k2), ("v1", v1), ("v2", v2), ("out", out), ("lse", lse)):
            arrays[f"{name}/{key}"] = val.numpy()
        arrays[f"{name}/meta"] = np.array([b, n, hq, hk, d, ws, wl, seed], dtype=np.int64)
    path = os.path.join(HERE, "simplicial_golden.npz")
    np.savez_compressed(path, **arrays)
    return path


if __name__ == "__main__":
    print(make())
