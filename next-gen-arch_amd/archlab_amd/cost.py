"""Useful-work accounting of 2-simplicial attention: valid (key, key) pairs.

Mirrors ``causal_pairs`` / ``causal_triples`` of the reference's cost ledger
(archlab/architectures/limite_cost.py:31-45) and the FLOP charge it derives
from them (:69-73: 12 * H * D per valid pair for forward plus backward, i.e.
4 * H * D forward and 8 * H * D backward).  The nominal figure of the
benchmark, 4 * B * H * S * w1 * w2 * D, charges every query full windows;
the valid-pair figure charges only the pairs a query can see (windows cut by
the start of its sequence).

Query i (0-based) of a sequence sees min(i + 1, span) keys on an axis of
window ``span``, so the pair count of the two axes is
    sum_i min(i + 1, a) * min(i + 1, b)       (a <= b the two clipped windows)
which splits at i + 1 = a and i + 1 = b into a sum of squares, an
arithmetic series and a constant tail, each in closed form.
"""

from __future__ import annotations

from typing import Iterable, Optional


def causal_pairs(length: int, span: Optional[int] = None) -> int:
    """Valid causal (query, key) pairs of one sequence with keys within ``span``
    of the query (``None``: unbounded); limite_cost.py:31-35."""
    if length < 1 or (span is not None and span < 1):
        raise ValueError("attention length/span must be positive")
    w = length if span is None else min(length, span)
    ramp = w * (w + 1) // 2          # queries 0 .. w-1 see 1 .. w keys
    return ramp + (length - w) * w   # the rest see w keys each


def causal_triples(length: int, short_span: int, long_span: int) -> int:
    """Valid (query, short key, long key) triples of one sequence, i.e. the
    number of scored pairs summed over its queries; limite_cost.py:38-45."""
    causal_pairs(length, short_span)  # same argument checks
    causal_pairs(length, long_span)
    a, b = sorted((min(length, short_span), min(length, long_span)))
    squares = a * (a + 1) * (2 * a + 1) // 6            # i + 1 in 1..a: (i + 1)^2
    middle = a * ((b * (b + 1)) // 2 - (a * (a + 1)) // 2)  # i + 1 in a+1..b: a * (i + 1)
    tail = (length - b) * a * b                          # i + 1 > b: a * b
    return squares + middle + tail


def sequence_triples(lengths: Iterable[int], short_window: int, long_window: int) -> int:
    """Scored pairs of a batch of independent sequences (dense batch or packed
    variable-length), each sequence starting its windows afresh."""
    return sum(causal_triples(int(n), short_window, long_window) for n in lengths)


def forward_flops(heads_q: int, head_dim: int, triples: int) -> float:
    """Forward FLOPs of the scored pairs: 2 * D for the score and 2 * D for the
    value product per pair and query head (the forward third of the
    reference's 12 * H * D per pair, limite_cost.py:69-73)."""
    return 4.0 * heads_q * head_dim * triples


def backward_flops(heads_q: int, head_dim: int, triples: int) -> float:
    """Backward FLOPs of the scored pairs: twice the forward's (the
    reference's 12 * H * D per pair for forward + backward)."""
    return 8.0 * heads_q * head_dim * triples
