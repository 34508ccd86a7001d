"""Seeded synthetic inputs for the benchmark configurations.

One generation rule for every configuration (recorded in every report):
``g = torch.Generator("cpu").manual_seed(seed)``; draw fp32 tensors in the
order Q, K, V, K', V' as [B, S, H, D] (Q with HQ heads, the others with HKV
heads); multiply by sigma; multiply Q by 1/sqrt(D); cast to the compute dtype.
The op is then called with ``scale=1.0`` and the mapping
``q=Q, k1=K', k2=K, v1=V', v2=V, short_window=w2, long_window=w1`` -- the
benchmark's long axis (K, V, w1) is the reference's (k2, v2, long_window)
and its short axis (K', V', w2) is (k1, v1, short_window).
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch

from . import cost


@dataclass(frozen=True)
class PrefillConfig:
    name: str
    batch: int
    seqlen: int
    heads_q: int
    heads_kv: int
    dim: int
    w1: int  # long window (K, V)
    w2: int  # short window (K', V')
    dtype: torch.dtype = torch.bfloat16
    sigma: float = 1.0
    seed: int = 0
    varlen_seqs: int = 0  # > 0: packed variable-length with this many sequences
    varlen_seed: int = 1
    lengths: tuple = field(default=())

    @property
    def tokens(self) -> int:
        return self.batch * self.seqlen


@dataclass(frozen=True)
class PagedConfig:
    name: str
    batch: int
    heads_q: int
    heads_kv: int
    dim: int
    w1: int
    w2: int
    page: int
    ctx_lo: int
    ctx_hi: int
    seed: int = 2
    dtype: torch.dtype = torch.bfloat16


C1 = PrefillConfig("C1-cpu-fp32", 1, 512, 4, 4, 64, 32, 16, torch.float32)
C2 = PrefillConfig("C2-bf16-prefill", 2, 4096, 16, 16, 128, 512, 32)
NS = PrefillConfig("NS-bf16-prefill-S8192", 2, 8192, 16, 16, 128, 512, 32)
C3 = PrefillConfig("C3-bf16-varlen-gqa", 1, 32768, 32, 8, 128, 512, 32, varlen_seqs=12)
C4 = PrefillConfig("C4-bf16-d256", 1, 16384, 8, 8, 256, 256, 64, sigma=0.5)
C5 = PagedConfig("C5-bf16-paged-decode", 64, 32, 8, 128, 512, 32, 64, 1024, 32768)
# The reference's DeepSeek-V4.1 adapter geometry (recipes/deepseek_v41/proposals.yaml:57-59,
# short window 32, long window 512), whose core runs in fp32 for training
# (deepseek_v41_adapter.py:136-144); two sequences of 8192 tokens.
DSV41 = PrefillConfig("DSV41-fp32-adapter", 2, 8192, 8, 2, 128, 512, 32, torch.float32)


def varlen_lengths(total: int, nseq: int, seed: int, lo: int = 256, hi: int = 6000) -> list[int]:
    """Lengths uniform in [lo, hi] from ``seed``, clipped to sum to ``total``.

    The running sum is truncated at ``total`` (later sequences dropped or cut);
    if the draws fall short, the last sequence is extended.
    """
    g = torch.Generator("cpu").manual_seed(seed)
    draws = torch.randint(lo, hi + 1, (nseq,), generator=g).tolist()
    out, acc = [], 0
    for n in draws:
        if acc >= total:
            break
        n = min(n, total - acc)
        out.append(n)
        acc += n
    if acc < total:
        out[-1] += total - acc
    return out


def cu_from_lengths(lengths) -> torch.Tensor:
    cu = [0]
    for n in lengths:
        cu.append(cu[-1] + n)
    return torch.tensor(cu, dtype=torch.int32)


def prefill_inputs(cfg: PrefillConfig, device="cpu", generator_device="cpu"):
    """(q, k1, k2, v1, v2, cu_seqlens or None) in the reference argument order.

    Dense configs return [B,S,H,D]; varlen configs return packed [T,H,D] plus
    int32 cu_seqlens.  Values are drawn fp32 on the CPU, then cast.
    """
    g = torch.Generator(generator_device).manual_seed(cfg.seed)
    shape_q = (cfg.batch, cfg.seqlen, cfg.heads_q, cfg.dim)
    shape_kv = (cfg.batch, cfg.seqlen, cfg.heads_kv, cfg.dim)
    Q = torch.randn(shape_q, generator=g, device=generator_device)
    K, V, Kp, Vp = (torch.randn(shape_kv, generator=g, device=generator_device) for _ in range(4))
    if cfg.sigma != 1.0:
        Q, K, V, Kp, Vp = (x * cfg.sigma for x in (Q, K, V, Kp, Vp))
    Q = Q * (1.0 / math.sqrt(cfg.dim))
    q, k1, k2, v1, v2 = (x.to(cfg.dtype).to(device) for x in (Q, Kp, K, Vp, V))
    cu = None
    if cfg.varlen_seqs:
        lengths = cfg.lengths or tuple(varlen_lengths(cfg.tokens, cfg.varlen_seqs, cfg.varlen_seed))
        cu = cu_from_lengths(lengths).to(device)
        q, k1, k2, v1, v2 = (x.reshape(cfg.tokens, x.shape[2], x.shape[3]) for x in (q, k1, k2, v1, v2))
    return q, k1, k2, v1, v2, cu


def paged_inputs(cfg: PagedConfig, device="cpu", pool_pages=None, null_block=True):
    """Paged decode batch: one new token per sequence at position ctx - 1.

    Returns dict with q [B,HQ,D], short/long caches [2, 1+pages, page, HKV, D],
    block_table [B, max_pages] int32 (a random permutation of the physical
    pages, block 0 = null page, shared by both axes), token_seq, token_pos
    int32, and the per-sequence context lengths.
    """
    g = torch.Generator("cpu").manual_seed(cfg.seed)
    ctx = torch.randint(cfg.ctx_lo, cfg.ctx_hi + 1, (cfg.batch,), generator=g)
    width = -(-cfg.ctx_hi // cfg.page)
    pages = cfg.batch * width if pool_pages is None else pool_pages
    table = (torch.randperm(pages, generator=g) + (1 if null_block else 0))[: cfg.batch * width]
    table = table.reshape(cfg.batch, width).to(torch.int32)
    nblocks = pages + (1 if null_block else 0)
    shape = (2, nblocks, cfg.page, cfg.heads_kv, cfg.dim)
    q = torch.randn((cfg.batch, cfg.heads_q, cfg.dim), generator=g) * (1.0 / math.sqrt(cfg.dim))
    out = {
        "q": q.to(cfg.dtype).to(device),
        "block_table": table.to(device),
        "token_seq": torch.arange(cfg.batch, dtype=torch.int32).to(device),
        "token_pos": (ctx - 1).to(torch.int32).to(device),
        "ctx": ctx,
    }
    # caches are large (C5: 2 x 8.6 GB); fill on the target device
    cg = torch.Generator(device).manual_seed(cfg.seed + 1000)
    out["short_cache"] = _randn_chunked(shape, cg, device, cfg.dtype)
    out["long_cache"] = _randn_chunked(shape, cg, device, cfg.dtype)
    return out


def _randn_chunked(shape, generator, device, dtype):
    """N(0,1) fill of a large tensor without an fp32 copy of the whole thing."""
    t = torch.empty(shape, device=device, dtype=dtype)
    flat = t.view(shape[0] * shape[1], -1)
    step = max(1, (1 << 26) // flat.shape[1])
    for i in range(0, flat.shape[0], step):
        n = min(step, flat.shape[0] - i)
        flat[i:i + n] = torch.randn((n, flat.shape[1]), generator=generator, device=device).to(dtype)
    return t


def prefill_flops(cfg: PrefillConfig) -> float:
    """Nominal FLOPs 4 * B * H * S * w1 * w2 * D (full windows)."""
    return 4.0 * cfg.batch * cfg.heads_q * cfg.seqlen * cfg.w1 * cfg.w2 * cfg.dim


def sequence_lengths(cfg: PrefillConfig) -> list[int]:
    """Lengths of the independent sequences of a prefill configuration."""
    if cfg.varlen_seqs:
        return list(cfg.lengths or varlen_lengths(cfg.tokens, cfg.varlen_seqs, cfg.varlen_seed))
    return [cfg.seqlen] * cfg.batch


def prefill_triples(cfg: PrefillConfig) -> int:
    """Scored (short key, long key) pairs summed over every query of the
    configuration (windows cut at each sequence start; limite_cost.py:38-45)."""
    return cost.sequence_triples(sequence_lengths(cfg), cfg.w2, cfg.w1)


def prefill_valid_flops(cfg: PrefillConfig) -> float:
    """Forward FLOPs of the valid pairs only: 4 * HQ * D per scored pair."""
    return cost.forward_flops(cfg.heads_q, cfg.dim, prefill_triples(cfg))


def prefill_bytes(cfg: PrefillConfig) -> float:
    """Algorithmic bytes: each input read once, O and LSE written once."""
    es = torch.finfo(cfg.dtype).bits // 8
    t = cfg.tokens
    inputs = t * cfg.heads_q * cfg.dim * es + 4 * t * cfg.heads_kv * cfg.dim * es
    return float(inputs + t * cfg.heads_q * cfg.dim * es + t * cfg.heads_q * 4)


def paged_bytes(cfg: PagedConfig, ctx: torch.Tensor, out_bytes: int = 4) -> float:
    """Algorithmic bytes of one decode step: the K/V windows actually visible
    to each token (min(ctx, w) rows per KV head and branch), Q, O and LSE."""
    es = torch.finfo(cfg.dtype).bits // 8
    row = cfg.heads_kv * cfg.dim * es
    long_rows = sum(min(int(c), cfg.w1) for c in ctx)
    short_rows = sum(min(int(c), cfg.w2) for c in ctx)
    kv = 2 * row * (long_rows + short_rows)
    q = cfg.batch * cfg.heads_q * cfg.dim * es
    o = cfg.batch * cfg.heads_q * cfg.dim * out_bytes
    return float(kv + q + o + cfg.batch * cfg.heads_q * 4)


def paged_flops(cfg: PagedConfig, ctx: torch.Tensor) -> float:
    return float(sum(4.0 * cfg.heads_q * min(int(c), cfg.w1) * min(int(c), cfg.w2) * cfg.dim for c in ctx))
