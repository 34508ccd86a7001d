"""CPU oracle for 2-simplicial (trilinear) sliding-window attention.

TEST INFRASTRUCTURE ONLY.  Nothing in the product package imports this file.
Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it, and only as the checker (or the timed CPU
baseline), never as the computation that is shipped.

It restates, in plain PyTorch on the CPU, what the reference computes:

* ``reference_simplicial`` follows
  ``src/archlab/architectures/simplicial_attention.py:49-74`` (per-query loop,
  two-window einsum, one joint softmax over the flattened pairs) and adds the
  natural-log LSE that the reference's kernels write
  (``src/archlab/architectures/simplicial_kernels.py:52``).  The reference
  oracle returns no LSE, so the LSE is the closed form
  ``logsumexp_{valid (j,k)} scale * score`` and is pinned by tests against an
  independent brute-force evaluation.
* ``varlen_reference`` applies the dense oracle per ``cu_seqlens`` slice: the
  "same-document" visibility of ``recipes/deepseek_v41/proposals.yaml:76``.
* ``paged_reference`` follows the gather addressing of
  ``src/archlab/architectures/simplicial_paged.py:38-52`` (block =
  table[seq, pos // block_size], offset = pos % block_size, one table per key
  axis) and evaluates each token with the dense math.
* ``token_layout`` follows ``src/archlab/training/serving.py:52-62``.
* ``causal_pairs`` / ``causal_triples`` follow
  ``src/archlab/architectures/limite_cost.py:31-45``.
* ``determinant_reference`` / ``reference_determinant_simplicial`` follow
  ``src/archlab/architectures/simplicial_attention.py:151-178`` (and the
  any-window form of ``tests/test_simplicial_determinant.py:173-189``): the
  score of (q, k1_j, k2_k) is the sum over 3-coordinate chunks of the signed
  3x3 determinant det([q; k1_j; k2_k]) (trailing dim % 3 coordinates take no
  part), evaluated with ``torch.linalg.det`` and independent of any operand
  expansion.

Argument names follow the reference: ``(k1, v1, short_window)`` is one key
axis and ``(k2, v2, long_window)`` the other.  Every check of this file lives
in ``tests/test_oracle.py``; each function's pinning is listed there.
"""

from __future__ import annotations

import math

import torch


def _score_scale(scale, dim):
    """simplicial_attention.py:41-46: None -> 1/sqrt(score_dim), else a finite real."""
    if scale is None:
        return 1.0 / math.sqrt(dim)
    if isinstance(scale, torch.Tensor) or not math.isfinite(float(scale)):
        raise ValueError("scale must be a finite real number")
    return float(scale)


def reference_simplicial(q, k1, k2, v1, v2, short_window, long_window, *,
                         query_positions=None, scale=None, return_lse=False):
    """Per-query joint-softmax oracle (simplicial_attention.py:49-74), plus LSE.

    q [B,N,HQ,D]; k1,k2 [B,N,HK,D]; v1,v2 [B,N,HK,DV].  Returns O
    [B,len(positions),HQ,DV] and, with ``return_lse``, the natural-log LSE
    [B,len(positions),HQ] in the dtype of the computation.
    """
    if q.ndim != 4 or any(x.ndim != 4 for x in (k1, k2, v1, v2)):
        raise ValueError("expected [batch, sequence, heads, head_dim]")
    if min(short_window, long_window) < 1 or short_window > long_window:
        raise ValueError("require 1 <= short_window <= long_window")
    scale = _score_scale(scale, q.shape[-1])
    groups = q.shape[2] // k1.shape[2]
    # GQA: query head h reads KV head h // groups (simplicial_attention.py:61-62).
    k1, k2, v1, v2 = [x.repeat_interleave(groups, dim=2) for x in (k1, k2, v1, v2)]
    outputs, lses = [], []
    positions = range(q.shape[1]) if query_positions is None else query_positions
    for i in positions:
        if not 0 <= i < q.shape[1]:
            raise ValueError("oracle query position outside sequence")
        j = slice(max(0, i - short_window + 1), i + 1)
        k = slice(max(0, i - long_window + 1), i + 1)
        scores = torch.einsum("bhd,bjhd,bkhd->bhjk", q[:, i], k1[:, j], k2[:, k]) * scale
        flat = scores.flatten(-2)
        probabilities = flat.softmax(-1).reshape_as(scores)
        outputs.append(torch.einsum("bhjk,bjhd,bkhd->bhd", probabilities, v1[:, j], v2[:, k]))
        if return_lse:
            lses.append(torch.logsumexp(flat, -1))
    out = torch.stack(outputs, dim=1)
    if return_lse:
        return out, torch.stack(lses, dim=1)
    return out


def kernel_rounding_reference(q, k1, k2, v1, v2, short_window, long_window, *, query_positions=None,
                              scale=None, round_to=torch.bfloat16):
    """The oracle with the reference KERNEL's rounding point applied.

    simplicial_kernels.py:35 forms ``a = (q * k1)`` in fp32 and rounds it to
    the input dtype before the score dot.  This evaluates the same math as
    ``reference_simplicial`` but with every a_j = round_to(q_i ⊙ k1_j), in
    float64 otherwise.  Returns (O, LSE).  With ``round_to=None`` it is
    ``reference_simplicial`` in float64.
    """
    scale = _score_scale(scale, q.shape[-1])
    groups = q.shape[2] // k1.shape[2]
    k1, k2, v1, v2 = [x.double().repeat_interleave(groups, dim=2) for x in (k1, k2, v1, v2)]
    q = q.double()
    outs, lses = [], []
    positions = range(q.shape[1]) if query_positions is None else query_positions
    for i in positions:
        j = slice(max(0, i - short_window + 1), i + 1)
        k = slice(max(0, i - long_window + 1), i + 1)
        a = q[:, i][:, None] * k1[:, j]  # [B, J, H, D]
        if round_to is not None:
            a = a.float().to(round_to).double()
        scores = torch.einsum("bjhd,bkhd->bhjk", a, k2[:, k]) * scale
        flat = scores.flatten(-2)
        p = flat.softmax(-1).reshape_as(scores)
        outs.append(torch.einsum("bhjk,bjhd,bkhd->bhd", p, v1[:, j], v2[:, k]))
        lses.append(torch.logsumexp(flat, -1))
    return torch.stack(outs, dim=1), torch.stack(lses, dim=1)


def varlen_reference(q, k1, k2, v1, v2, cu_seqlens, short_window, long_window, *,
                     scale=None, return_lse=False, query_positions=None):
    """Packed variable-length form: q [T,HQ,D], keys [T,HK,D], cu_seqlens [nseq+1].

    Each sequence is evaluated on its own (no key crosses a document boundary).
    ``query_positions`` (optional) is a list of global token indices.
    """
    cu = [int(x) for x in cu_seqlens]
    outs = torch.empty(q.shape[0], q.shape[1], v1.shape[-1], dtype=q.dtype)
    lses = torch.empty(q.shape[0], q.shape[1], dtype=q.dtype)
    wanted = None if query_positions is None else sorted(set(int(t) for t in query_positions))
    for s in range(len(cu) - 1):
        lo, hi = cu[s], cu[s + 1]
        if hi <= lo:
            continue
        if wanted is None:
            local = None
        else:
            local = [t - lo for t in wanted if lo <= t < hi]
            if not local:
                continue
        o, l = reference_simplicial(*(x[None, lo:hi] for x in (q, k1, k2, v1, v2)),
                                    short_window, long_window, scale=scale,
                                    query_positions=local, return_lse=True)
        idx = torch.arange(lo, hi) if local is None else torch.tensor(local) + lo
        outs[idx] = o[0]
        lses[idx] = l[0]
    if wanted is not None:
        outs, lses = outs[wanted], lses[wanted]
    return (outs, lses) if return_lse else outs


def paged_gather(cache, table, seq, positions):
    """Rows of a [2, blocks, block, HK, D] cache for one sequence's logical positions.

    simplicial_paged.py:41-44 / :49-52: block = table[seq, pos // block_size]
    (widened to int64 before the stride multiply), offset = pos % block_size.
    Returns (K, V), each [len(positions), HK, D].
    """
    block_size = cache.shape[2]
    pos = torch.as_tensor(positions, dtype=torch.int64)
    blocks = table[seq].to(torch.int64)[pos // block_size]
    offsets = pos % block_size
    return cache[0, blocks, offsets], cache[1, blocks, offsets]


def paged_reference(q, short_cache, long_cache, block_table, token_seq, token_pos, *,
                    short_window, long_window, scale, long_block_table=None, return_lse=False):
    """Paged serving form (simplicial_paged.py:68-128 semantics), one token at a time.

    q [T,HQ,D]; caches [2,blocks,block,HK,D]; tables [num_seqs, max_blocks].
    Output is computed in q's dtype promoted to at least float32 (the
    reference's paged API returns float32).
    """
    long_block_table = block_table if long_block_table is None else long_block_table
    work = torch.float64 if q.dtype == torch.float64 else torch.float32
    tokens, heads, dim = q.shape
    out = torch.empty(tokens, heads, long_cache.shape[-1], dtype=work)
    lse = torch.empty(tokens, heads, dtype=work)
    for t in range(tokens):
        s, p = int(token_seq[t]), int(token_pos[t])
        short_pos = list(range(max(0, p - short_window + 1), p + 1))
        long_pos = list(range(max(0, p - long_window + 1), p + 1))
        k1, v1 = paged_gather(short_cache, block_table, s, short_pos)
        k2, v2 = paged_gather(long_cache, long_block_table, s, long_pos)
        o, l = _single_query(q[t].to(work), k1.to(work), k2.to(work), v1.to(work), v2.to(work), scale)
        out[t], lse[t] = o, l
    return (out, lse) if return_lse else out


def _single_query(q, k1, k2, v1, v2, scale):
    """One query [HQ,D] against explicit windows k1/v1 [J,HK,D], k2/v2 [K,HK,D]."""
    groups = q.shape[0] // k1.shape[1]
    k1, k2, v1, v2 = [x.repeat_interleave(groups, dim=1) for x in (k1, k2, v1, v2)]
    scores = torch.einsum("hd,jhd,khd->hjk", q, k1, k2) * scale
    flat = scores.flatten(-2)
    p = flat.softmax(-1).reshape_as(scores)
    return torch.einsum("hjk,jhd,khd->hd", p, v1, v2), torch.logsumexp(flat, -1)


def token_layout(query_start_loc, seq_lens, tokens):
    """Per-token (sequence, absolute position) from packed metadata (serving.py:52-62).

    A packed step holds, for sequence s, the last (starts[s+1]-starts[s])
    tokens of a sequence of total length seq_lens[s].
    """
    starts = [int(x) for x in query_start_loc]
    lens = [int(x) for x in seq_lens]
    seq, pos = [], []
    for t in range(tokens):
        s = 0
        while s + 1 < len(starts) and starts[s + 1] <= t:
            s += 1
        s = min(s, len(lens) - 1)
        first = starts[s]
        seq.append(s)
        pos.append(lens[s] - (starts[s + 1] - first) + (t - first))
    return torch.tensor(seq, dtype=torch.int32), torch.tensor(pos, dtype=torch.int32)


def causal_pairs(length, span=None):
    """limite_cost.py:31-35: sum over queries of the causal window width."""
    if length < 1 or (span is not None and span < 1):
        raise ValueError("attention length/span must be positive")
    width = min(length, span) if span is not None else length
    return width * (width + 1) // 2 + (length - width) * width


def causal_triples(length, short_span, long_span):
    """limite_cost.py:38-45: closed-form count of valid (j,k) pairs over all queries."""
    causal_pairs(length, short_span)
    causal_pairs(length, long_span)
    a, b = sorted((min(length, short_span), min(length, long_span)))
    return (a * (a + 1) * (2 * a + 1) // 6
            + a * (b * (b + 1) - a * (a + 1)) // 2
            + (length - b) * a * b)


def determinant_reference(q, k1, k2, v1, v2, window_1, window_2, *, query_positions=None, scale=None):
    """Determinant-score attention with any positive windows (k1 within window_1, k2 within window_2).

    Follows simplicial_attention.py:151-178 (and the any-window oracle of
    tests/test_simplicial_determinant.py:173-189): per query i and chunk c of
    3 coordinates, score_c = det([q_i[c]; k1_j[c]; k2_k[c]]); the joint softmax
    runs over all (j, k) with i-window_1 < j <= i and i-window_2 < k <= i;
    O_i = sum P_ijk (v1_j * v2_k).  Default scale 1/sqrt(score_dim) of the
    unexpanded width.  Use float32/float64 (torch.linalg.det has no bf16).
    """
    if q.shape[-1] < 3:
        raise ValueError("determinant scores require at least 3 coordinates")
    if q.dtype not in (torch.float32, torch.float64):
        raise ValueError("determinant oracle requires float32/float64")
    if min(window_1, window_2) < 1:
        raise ValueError("windows must be positive")
    scale = _score_scale(scale, q.shape[-1])
    groups = q.shape[2] // k1.shape[2]
    k1, k2, v1, v2 = [x.repeat_interleave(groups, dim=2) for x in (k1, k2, v1, v2)]
    chunks = q.shape[-1] // 3
    qc, k1c, k2c = (x[..., :3 * chunks].reshape(*x.shape[:-1], chunks, 3) for x in (q, k1, k2))
    positions = range(q.shape[1]) if query_positions is None else query_positions
    outs = []
    for i in positions:
        if not 0 <= i < q.shape[1]:
            raise ValueError("oracle query position outside sequence")
        j0, k0 = max(0, i - window_1 + 1), max(0, i - window_2 + 1)
        a = qc[:, i]                      # [B,H,C,3]
        b = k1c[:, j0:i + 1]              # [B,J,H,C,3]
        c = k2c[:, k0:i + 1]              # [B,K,H,C,3]
        nj, nk = b.shape[1], c.shape[1]
        rows = torch.stack(torch.broadcast_tensors(a[:, None, None], b[:, :, None], c[:, None]), dim=-2)
        scores = torch.linalg.det(rows).sum(-1)            # [B,J,K,H]
        p = (scores * scale).permute(0, 3, 1, 2).reshape(q.shape[0], q.shape[2], nj * nk).softmax(-1)
        p = p.reshape(q.shape[0], q.shape[2], nj, nk)
        outs.append(torch.einsum("bhjk,bjhd,bkhd->bhd", p, v1[:, j0:i + 1], v2[:, k0:i + 1]))
    return torch.stack(outs, dim=1)


def reference_determinant_simplicial(q, k1, k2, v1, v2, short_window, long_window, *,
                                     query_positions=None, scale=None):
    """simplicial_attention.py:151-178: the determinant oracle with 1 <= short <= long."""
    if min(short_window, long_window) < 1 or short_window > long_window:
        raise ValueError("require 1 <= short_window <= long_window")
    return determinant_reference(q, k1, k2, v1, v2, short_window, long_window,
                                 query_positions=query_positions, scale=scale)
