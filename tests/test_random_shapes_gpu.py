"""Seeded random-shape sweep of the prefill forward and backward on the GPU
against the fp64 oracle (oracle/simplicial_oracle.py, the restatement of
reference_simplicial, archlab/architectures/simplicial_attention.py:49-74).

The paged (serving) forward gets the same treatment on drawn page sizes,
contexts, windows and layouts (restating the reference's paged test plan,
tests/test_simplicial_paged.py, over random geometries).

The shapes are drawn from a fixed seed so that every run checks the same
cases: batch 1-2 (or packed sequences), 1-180 tokens, KV heads 1-4, GQA
groups 1-4, score / value widths 64, 128 and 256 (equal or not where the
kernels take both), short windows 1-64 (one or two 32-row groups of short
keys), long windows from the short window up to 2.5x the sequence.  They reach
the matrix-core paths' less common branches together: dk2 / dv2 walk pieces
(few workgroups), dk1 partials of one or two row groups, the width-256
passes, partial last query blocks and sequence starts inside blocks.

Tolerances are the BASELINE parity gate's: bf16 output and gradients 2e-2 x
max(|ref|, 1), LSE 1e-3 relative where a query sees >= 64 (short, long) pairs
and 1e-2 where it sees fewer (there the reference's own bf16 rounding point of
q ⊙ k1 moves the LSE by more than 1e-3); fp32 1e-4 x max(|ref|, 1).
"""

import random

import pytest
import torch

from helpers import paged_batch, rand_inputs
from oracle import simplicial_oracle as O

pytestmark = pytest.mark.gpu

_WIDTHS = [(64, 64), (128, 128), (64, 128), (128, 64), (256, 256), (256, 128)]


def _draw(rng):
    d, dv = rng.choice(_WIDTHS)
    hk = rng.choice([1, 2, 3, 4])
    group = rng.choice([1, 2, 3, 4])
    if d == 256:  # keep the fp64 oracle quick at the widest heads
        hk, group = min(hk, 2), min(group, 2)
    b = rng.choice([1, 2])
    n = rng.randint(1, 180 // b)
    ws = rng.choice([1, 2, 7, 16, 31, 32, 33, 48, 63, 64])
    wl = max(ws, rng.choice([ws, ws + 1, 40, 96, 130, 200, 257, 450]))
    return b, n, hk * group, hk, d, dv, ws, wl


_CASES = [_draw(random.Random(1000 + i)) for i in range(48)]


def _oracle(x, ws, wl, dout, dl):
    xs = [t.double().requires_grad_(True) for t in x]
    o, lse = O.reference_simplicial(*xs, ws, wl, scale=None, return_lse=True)
    ((o * dout.double()).sum() + (lse * dl.double()).sum()).backward()
    return o.float(), lse.float(), [t.grad.float() for t in xs]


def _check(label, got, ref, rtol):
    got = got.float().cpu()
    assert torch.isfinite(got).all(), f"{label}: non-finite"
    err = (got - ref).abs().max().item()
    bound = rtol * max(ref.abs().max().item(), 1.0)
    assert err <= bound, f"{label}: max-abs {err:.3e} > {bound:.3e}"
    return err


@pytest.mark.parametrize("case", range(len(_CASES)))
def test_random_shape_forward_and_backward_bf16(cuda, case):
    """Forward (output, LSE) and the five gradients, with an LSE gradient, of
    a drawn shape in bf16 on the matrix cores."""
    from archlab_amd import simplicial_attention
    b, n, hq, hk, d, dv, ws, wl = _CASES[case]
    x = rand_inputs(b, n, hq, hk, d, dv=dv, seed=case, dtype=torch.bfloat16)
    g = torch.Generator().manual_seed(500 + case)
    dout = torch.randn(b, n, hq, dv, generator=g).bfloat16()
    dl = torch.randn(b, n, hq, generator=g)
    xd = [t.to(cuda).requires_grad_(True) for t in x]
    out, lse = simplicial_attention(*xd, ws, wl, return_lse=True)
    ((out.float() * dout.to(cuda).float()).sum() + (lse * dl.to(cuda)).sum()).backward()
    o_ref, l_ref, g_ref = _oracle([t.float() for t in x], ws, wl, dout.float(), dl)
    label = f"case {case}: b{b} n{n} h{hq}/{hk} d{d}/{dv} w{ws}x{wl}"
    errs = [_check(label + " out", out, o_ref, 2e-2)]
    # pairs each query sees (dense batches: positions from 0 in each sequence)
    pos = torch.arange(n, dtype=torch.float32)
    pairs = torch.clamp(pos + 1, max=ws) * torch.clamp(pos + 1, max=wl)
    bound = torch.where(pairs >= 64, 1e-3, 1e-2)[None, :, None]
    rel = (lse.cpu() - l_ref).abs() / l_ref.abs().clamp_min(1.0)
    lerr = rel.max().item()
    assert (rel <= bound).all(), f"{label} lse: {lerr:.3e}"
    for name, t, r in zip(("dq", "dk1", "dk2", "dv1", "dv2"), xd, g_ref):
        errs.append(_check(f"{label} {name}", t.grad, r, 2e-2))
    print(label + ": " + " ".join(f"{e:.1e}" for e in errs) + f" lse {lerr:.1e}", flush=True)


@pytest.mark.parametrize("case", [c for c in range(len(_CASES)) if _CASES[c][4] == _CASES[c][5] and _CASES[c][4] <= 128][:12])
def test_random_shape_backward_fp32(cuda, case):
    """The same shapes in fp32, short windows cut to 32 (equal widths up to
    128: the hi/lo matrix-core forward and backward)."""
    from archlab_amd import simplicial_attention
    b, n, hq, hk, d, dv, ws, wl = _CASES[case]
    ws = min(ws, 32)  # one 32-row group: the fp32 matrix-core passes
    x = rand_inputs(b, n, hq, hk, d, dv=dv, seed=case, dtype=torch.float32)
    g = torch.Generator().manual_seed(700 + case)
    dout = torch.randn(b, n, hq, dv, generator=g)
    dl = torch.randn(b, n, hq, generator=g)
    xd = [t.to(cuda).requires_grad_(True) for t in x]
    out, lse = simplicial_attention(*xd, ws, wl, return_lse=True)
    ((out * dout.to(cuda)).sum() + (lse * dl.to(cuda)).sum()).backward()
    o_ref, _, g_ref = _oracle(x, ws, wl, dout, dl)
    label = f"fp32 case {case}: b{b} n{n} h{hq}/{hk} d{d} w{ws}x{wl}"
    errs = [_check(label + " out", out, o_ref, 1e-4)]
    for name, t, r in zip(("dq", "dk1", "dk2", "dv1", "dv2"), xd, g_ref):
        errs.append(_check(f"{label} {name}", t.grad, r, 1e-4))
    print(label + ": " + " ".join(f"{e:.1e}" for e in errs), flush=True)


@pytest.mark.parametrize("case", range(12))
def test_random_packed_sequences_backward_bf16(cuda, case):
    """Packed variable-length sequences (random lengths, starts anywhere in a
    query block or key block) with GQA, against the per-sequence oracle."""
    from archlab_amd import simplicial_varlen_attention
    rng = random.Random(2000 + case)
    d, dv = rng.choice(_WIDTHS[:4])
    hk, group = rng.choice([1, 2]), rng.choice([1, 2, 4])
    ws = rng.choice([5, 32, 40, 64])
    wl = max(ws, rng.choice([64, 150, 300]))
    lengths = [rng.randint(1, 90) for _ in range(rng.randint(2, 5))]
    t = sum(lengths)
    cu = torch.tensor([0] + [sum(lengths[:i + 1]) for i in range(len(lengths))], dtype=torch.int32)
    x = [v[0] for v in rand_inputs(1, t, hk * group, hk, d, dv=dv, seed=3000 + case, dtype=torch.bfloat16)]
    g = torch.Generator().manual_seed(case)
    dout = torch.randn(t, hk * group, dv, generator=g).bfloat16()
    xd = [v.to(cuda).requires_grad_(True) for v in x]
    out = simplicial_varlen_attention(*xd, cu.to(cuda), ws, wl)
    (out.float() * dout.to(cuda).float()).sum().backward()
    xs = [v.double().requires_grad_(True) for v in x]
    o = O.varlen_reference(*xs, cu, ws, wl, scale=d ** -0.5)
    (o * dout.double()).sum().backward()
    label = f"packed case {case}: lengths {lengths} h{hk * group}/{hk} d{d}/{dv} w{ws}x{wl}"
    errs = [_check(label + " out", out, o.detach().float(), 2e-2)]
    for name, tg, r in zip(("dq", "dk1", "dk2", "dv1", "dv2"), xd, xs):
        errs.append(_check(f"{label} {name}", tg.grad, r.grad.float(), 2e-2))
    print(label + ": " + " ".join(f"{e:.1e}" for e in errs), flush=True)


def _draw_paged(rng):
    dim = rng.choice([64, 128, 128, 256])
    kv_heads = rng.choice([1, 2, 4])
    group = rng.choice([1, 2, 4, 8])
    block = rng.choice([16, 64])
    lengths = [rng.randint(1, 1500) for _ in range(rng.randint(1, 4))]
    ws = rng.choice([1, 4, 16, 32, 40, 64])
    wl = max(ws, rng.choice([ws, 64, 300, 1 << 30]))
    qdt = rng.choice([torch.bfloat16, torch.float32])
    hnd = rng.random() < 0.5
    return dim, kv_heads, group, block, lengths, ws, wl, qdt, hnd


_PAGED = [_draw_paged(random.Random(4000 + i)) for i in range(16)]


@pytest.mark.parametrize("case", range(len(_PAGED)))
def test_random_paged_decode_and_prefill_tokens(cuda, case):
    """Paged forward on drawn geometries (bf16 caches in NHD or HND layout,
    shuffled pages, a null block, bf16 or fp32 queries, windows up to global
    ones that clip to the block tables' reach) for each sequence's last token
    and two earlier positions, against the dense oracle on the same rows."""
    from archlab_amd import simplicial_paged_attention
    dim, kv_heads, group, block, lengths, ws, wl, qdt, hnd = _PAGED[case]
    heads = kv_heads * group
    (short, long), table, dense = paged_batch(lengths, kv_heads, dim, block, torch.bfloat16, hnd, seed=case,
                                              device=cuda)
    rng = random.Random(5000 + case)
    g = torch.Generator().manual_seed(6000 + case)
    seqs, positions, queries, expected = [], [], [], []
    for s, (n, (k1, k2, v1, v2)) in enumerate(zip(lengths, dense)):
        q = (torch.randn(1, n, heads, dim, generator=g) / dim ** 0.5).to(qdt)
        chosen = sorted({n - 1, rng.randrange(n), rng.randrange(n)})
        ref = O.reference_simplicial(q.double(), k1.double(), k2.double(), v1.double(), v2.double(), ws, wl,
                                     scale=1.0, query_positions=chosen)
        for i, position in enumerate(chosen):
            seqs.append(s)
            positions.append(position)
            queries.append(q[0, position])
            expected.append(ref[0, i])
    q = torch.stack(queries).to(cuda)
    seq = torch.tensor(seqs, dtype=torch.int32, device=cuda)
    pos = torch.tensor(positions, dtype=torch.int32, device=cuda)
    out = simplicial_paged_attention(q, short, long, table, seq, pos, short_window=ws, long_window=wl, scale=1.0)
    tol = 2e-4 if qdt == torch.float32 else 3e-2
    exp = torch.stack(expected).float()
    err = (out.cpu() - exp).abs().max().item()
    print(f"paged case {case}: d{dim} h{heads}/{kv_heads} block {block} lengths {lengths} w{ws}x{wl} "
          f"{qdt} hnd={hnd}: {err:.2e}", flush=True)
    torch.testing.assert_close(out.cpu(), exp, rtol=tol, atol=tol)
