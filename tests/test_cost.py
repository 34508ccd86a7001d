"""CPU checks of the valid-pair accounting (archlab_amd.cost, the product's
restatement of the reference's limite_cost.py:31-45): brute-force counts of
the explicit masks, the reference test's known answer, and the configured
workloads' valid-pair fractions."""

import pytest

from archlab_amd import cost
from archlab_amd import workloads as W


@pytest.mark.parametrize("length,span", [(1, None), (9, None), (9, 3), (3, 9), (64, 1), (100, 37), (37, 100)])
def test_pairs_match_explicit_causal_mask(length, span):
    brute = sum(key <= query and (span is None or key > query - span)
                for query in range(length) for key in range(length))
    assert cost.causal_pairs(length, span) == brute


@pytest.mark.parametrize("length,short,long", [(1, 16, 32), (9, 3, 5), (19, 16, 19), (41, 16, 5), (70, 32, 64),
                                               (130, 7, 128), (5, 1, 1), (33, 33, 33)])
def test_triples_match_explicit_joint_mask(length, short, long):
    # every (query, short key, long key) with both keys causal and inside their windows
    brute = sum(1 for i in range(length) for j in range(length) for k in range(length)
                if j <= i and k <= i and j > i - short and k > i - long)
    assert cost.causal_triples(length, short, long) == brute
    # symmetric in the two windows
    assert cost.causal_triples(length, long, short) == brute


def test_known_answer_from_the_reference_tests():
    # tests/test_limite_performance.py:100 of the reference: a 2048-token
    # sequence with a 1025-key span has 1,574,400 causal pairs
    assert cost.causal_pairs(2048, 1025) == 1_574_400


def test_invalid_lengths_and_spans_raise():
    for bad in ((0, None), (5, 0), (-1, 3)):
        with pytest.raises(ValueError):
            cost.causal_pairs(*bad)
    with pytest.raises(ValueError):
        cost.causal_triples(4, 0, 2)


def test_flop_charges_split_the_reference_ledger():
    # limite_cost.py:69-73 charges 12 * H * D per valid pair for forward + backward
    h, d, t = 16, 128, 12345
    assert cost.forward_flops(h, d, t) + cost.backward_flops(h, d, t) == 12 * h * d * t


def test_workload_valid_pair_fractions():
    # full windows everywhere give the nominal 4 * B * H * S * w1 * w2 * D
    full = W.PrefillConfig("full", 2, 4096, 4, 4, 64, 16, 16)
    tail = cost.causal_triples(4096, 16, 16) - (4096 - 16) * 16 * 16
    assert W.prefill_valid_flops(full) == pytest.approx(W.prefill_flops(full) - 2 * 4 * 4 * 64 * (16 * 16 * 16 - tail))
    # BASELINE configurations: the windows cut at each sequence start
    expected = {"C1": 0.967, "C2": 0.9375, "NS": 0.969, "C4": 0.992}
    for name, frac in expected.items():
        cfg = getattr(W, name)
        assert W.prefill_valid_flops(cfg) / W.prefill_flops(cfg) == pytest.approx(frac, abs=5e-4)
    # packed varlen: the sum over its sequences, each starting afresh
    c3 = W.C3
    lengths = W.sequence_lengths(c3)
    assert sum(lengths) == c3.tokens and len(lengths) == 12
    per_seq = sum(cost.causal_triples(n, c3.w2, c3.w1) for n in lengths)
    assert W.prefill_valid_flops(c3) == 4.0 * c3.heads_q * c3.dim * per_seq
    assert W.prefill_valid_flops(c3) < W.prefill_flops(c3)
