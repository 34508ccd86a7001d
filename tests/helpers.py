"""Shared builders and tolerance checks for the parity tests."""

from __future__ import annotations

import math

import torch

# Tolerances stated by the benchmark contract: bf16 output max-abs <= 2e-2,
# LSE relative <= 1e-3; fp32 <= 1e-4.
#  - The LSE "relative" error is taken against max(|lse|, 1): the LSE is a log,
#    an absolute error e in it is a relative error ~e in the partition sum,
#    and |lse| -> 0 (one or two pairs) would make a pure ratio meaningless.
#  - bf16 outputs additionally get half a bf16 ulp of the reference value
#    (2^-8 |ref|): a bf16 result cannot be closer than its own rounding, which
#    matters only where |O| > 1 (windows of one or two pairs).
BF16_OUT_ATOL = 2e-2
BF16_OUT_RTOL = 2.0 ** -8
BF16_LSE_RTOL = 1e-3
FP32_TOL = 1e-4


def rand_inputs(b, n, hq, hk, d, dv=None, seed=0, dtype=torch.bfloat16, sigma=1.0, device="cpu"):
    """(q, k1, k2, v1, v2): fp32 N(0, sigma^2) draws, q scaled by 1/sqrt(d), cast to dtype."""
    dv = d if dv is None else dv
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(b, n, hq, d, generator=g) * sigma / math.sqrt(d)
    k1, k2 = (torch.randn(b, n, hk, d, generator=g) * sigma for _ in range(2))
    v1, v2 = (torch.randn(b, n, hk, dv, generator=g) * sigma for _ in range(2))
    return [x.to(dtype).to(device) for x in (q, k1, k2, v1, v2)]


def assert_out_close(actual, expected, dtype, atol=None, rtol=None):
    """max |a - e| - rtol*|e| <= atol; returns the plain max-abs error."""
    actual = actual.float().cpu()
    expected = expected.float().cpu()
    assert torch.isfinite(actual).all(), "non-finite output"
    if atol is None:
        atol = BF16_OUT_ATOL if dtype == torch.bfloat16 else FP32_TOL
    if rtol is None:
        rtol = BF16_OUT_RTOL if dtype == torch.bfloat16 else 0.0
    diff = (actual - expected).abs()
    excess = (diff - rtol * expected.abs()).max().item()
    err = diff.max().item()
    where = divmod(int(diff.argmax()), expected.shape[-1]) if expected.ndim else 0
    assert excess <= atol, f"max-abs error {err:.3e} (excess {excess:.3e} > {atol:.1e}) at {where}"
    return err


def assert_lse_close(actual, expected, dtype, rtol=None):
    """max |a - e| / max(|e|, 1) <= rtol; returns that relative error."""
    actual = actual.float().cpu()
    expected = expected.float().cpu()
    assert torch.isfinite(actual).all(), "non-finite lse"
    if rtol is None:
        rtol = BF16_LSE_RTOL if dtype == torch.bfloat16 else FP32_TOL
    rel = ((actual - expected).abs() / expected.abs().clamp_min(1.0)).max().item()
    assert rel <= rtol, f"lse relative error {rel:.3e} > {rtol:.1e}"
    return rel


def paged_batch(lengths, kv_heads, dim, block_size, dtype, hnd=False, seed=0, device="cuda"):
    """Contiguous per-sequence K/V plus the same rows scattered into shuffled pages.

    Block 0 is the null block.  Returns ([short, long] caches, int32 table,
    list of per-sequence (k1, k2, v1, v2) [1, n, HK, D]).
    """
    g = torch.Generator().manual_seed(seed)
    per = [math.ceil(n / block_size) for n in lengths]
    total = 1 + sum(per)
    perm = (torch.randperm(total - 1, generator=g) + 1).tolist()
    table = torch.zeros(len(lengths), max(per), dtype=torch.int32)
    shape = (2, total, kv_heads, block_size, dim) if hnd else (2, total, block_size, kv_heads, dim)
    caches = [torch.zeros(shape, dtype=dtype) for _ in range(2)]
    dense = []
    for s, n in enumerate(lengths):
        table[s, :per[s]] = torch.tensor(perm[:per[s]], dtype=torch.int32)
        perm = perm[per[s]:]
        k1, k2, v1, v2 = (torch.randn(1, n, kv_heads, dim, generator=g).to(dtype) for _ in range(4))
        dense.append((k1, k2, v1, v2))
        idx = torch.arange(n)
        blocks = table[s].long()[idx // block_size]
        offs = idx % block_size
        for cache, (k, v) in zip(caches, ((k1, v1), (k2, v2))):
            view = cache.transpose(2, 3) if hnd else cache
            view[0, blocks, offs] = k[0]
            view[1, blocks, offs] = v[0]
    if hnd:
        caches = [c.transpose(2, 3) for c in caches]
    return [c.to(device) for c in caches], table.to(device), dense
