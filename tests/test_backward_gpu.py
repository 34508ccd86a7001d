"""GPU parity of the backward (sa_prefill_bwd through torch.autograd) against
float64 autograd of the CPU oracle on the same values.

Tolerances (max-abs error over a gradient tensor, relative to that tensor's
largest reference magnitude g_max):
  * fp32 inputs: <= 1e-4 * max(g_max, 1);
  * bf16 inputs: <= 2e-2 * max(g_max, 1) -- the reference's backward rounds
    a = q ⊙ k1, dout ⊙ v1, dS and P (on the value paths) to bf16
    (simplicial_kernels.py:75-101), each a 2^-9 relative step, and the
    gradient is returned in bf16.
Also: the result is bitwise reproducible, the LSE output is differentiable,
and varlen gradients equal per-sequence ones.
"""

import pytest
import torch

from helpers import rand_inputs
from oracle import simplicial_oracle as O

pytestmark = pytest.mark.gpu


def _ref_grads(x, ws, wl, scale, dout, dlse=None):
    xs = [t.double().requires_grad_(True) for t in x]
    o, l = O.reference_simplicial(*xs, ws, wl, scale=scale, return_lse=True)
    loss = (o * dout.double()).sum()
    if dlse is not None:
        loss = loss + (l * dlse.double()).sum()
    loss.backward()
    return [t.grad.float() for t in xs]


def _assert_grads(got, ref, dtype, label):
    rtol = 1e-4 if dtype == torch.float32 else 2e-2
    names = ["dq", "dk1", "dk2", "dv1", "dv2"]
    msgs = []
    for n, g, r in zip(names, got, ref):
        g = g.float().cpu()
        assert torch.isfinite(g).all(), f"{label} {n}: non-finite"
        err = (g - r).abs().max().item()
        bound = rtol * max(r.abs().max().item(), 1.0)
        msgs.append(f"{n} {err:.2e}/{bound:.1e}")
        assert err <= bound, f"{label} {n}: max-abs {err:.3e} > {bound:.3e}"
    print(label + ": " + " ".join(msgs), flush=True)


def _run(cuda, b, n, hq, hk, d, ws, wl, dtype, dv=None, scale=None, seed=0, dlse=False):
    from archlab_amd import simplicial_attention
    x = rand_inputs(b, n, hq, hk, d, dv=dv, seed=seed, dtype=dtype)
    g = torch.Generator().manual_seed(seed + 100)
    dout = torch.randn(b, n, hq, x[3].shape[-1], generator=g).to(dtype)
    dl = torch.randn(b, n, hq, generator=g) if dlse else None
    xd = [t.to(cuda).requires_grad_(True) for t in x]
    out, lse = simplicial_attention(*xd, ws, wl, scale=scale, return_lse=True)
    loss = (out.float() * dout.to(cuda).float()).sum()
    if dlse:
        loss = loss + (lse * dl.to(cuda)).sum()
    loss.backward()
    got = [t.grad for t in xd]
    sc = d ** -0.5 if scale is None else scale
    ref = _ref_grads([t.float() for t in x], ws, wl, sc, dout.float(), dl)
    _assert_grads(got, ref, dtype, f"b{b} n{n} h{hq}/{hk} d{d} dv{dv or d} w{ws}x{wl} {dtype}")
    return xd, got


@pytest.mark.parametrize("hq,hk,d,ws,wl", [(4, 2, 32, 5, 12), (2, 2, 64, 1, 1), (6, 3, 16, 3, 40),
                                           (4, 4, 128, 8, 8)])
def test_backward_fp32(cuda, hq, hk, d, ws, wl):
    _run(cuda, 2, 37, hq, hk, d, ws, wl, torch.float32)


@pytest.mark.parametrize("hq,hk,d,ws,wl", [(4, 1, 64, 6, 20), (8, 2, 128, 32, 96)])
def test_backward_bf16(cuda, hq, hk, d, ws, wl):
    _run(cuda, 1, 70, hq, hk, d, ws, wl, torch.bfloat16)


def test_backward_value_dim_and_scale(cuda):
    _run(cuda, 1, 29, 4, 2, 32, 4, 9, torch.float32, dv=64, scale=0.3)


def test_backward_lse_gradient(cuda):
    _run(cuda, 1, 25, 2, 1, 32, 3, 7, torch.float32, dlse=True)


def test_backward_deterministic(cuda):
    from archlab_amd import simplicial_attention
    x = [t.to(cuda) for t in rand_inputs(1, 90, 8, 2, 128, seed=4, dtype=torch.bfloat16)]
    dout = torch.randn(1, 90, 8, 128, device=cuda).bfloat16()
    runs = []
    for _ in range(2):
        xd = [t.clone().requires_grad_(True) for t in x]
        simplicial_attention(*xd, 16, 64).backward(dout)
        runs.append([t.grad.clone() for t in xd])
    for a, b in zip(*runs):
        assert torch.equal(a, b)


def test_backward_varlen_equals_per_sequence(cuda):
    from archlab_amd import simplicial_attention, simplicial_varlen_attention
    lengths = [9, 1, 30, 17]
    t = sum(lengths)
    x = [v[0] for v in rand_inputs(1, t, 4, 2, 32, seed=8, dtype=torch.float32)]
    dout = torch.randn(t, 4, 32)
    cu = torch.tensor([0, 9, 10, 40, 57], dtype=torch.int32, device=cuda)
    xd = [v.to(cuda).requires_grad_(True) for v in x]
    simplicial_varlen_attention(*xd, cu, 4, 11).backward(dout.to(cuda))
    start = 0
    for n in lengths:
        xs = [v[start:start + n][None].to(cuda).requires_grad_(True) for v in x]
        simplicial_attention(*xs, 4, 11).backward(dout[start:start + n][None].to(cuda))
        for a, b in zip(xd, xs):
            torch.testing.assert_close(a.grad[start:start + n], b.grad[0], rtol=0, atol=0)
        start += n


# ---- the MFMA passes (bf16, D == DV in {64, 128}) ------------------------------

@pytest.mark.parametrize("hq,hk,d,ws,wl", [(4, 4, 128, 40, 130), (8, 2, 64, 32, 512), (4, 1, 128, 7, 33),
                                           (2, 2, 128, 1, 1)])
def test_backward_bf16_mfma_shapes(cuda, hq, hk, d, ws, wl):
    """Two short passes (ws 40), a long window wider than the sequence, GQA 4, single pairs."""
    _run(cuda, 1, 200, hq, hk, d, ws, wl, torch.bfloat16, seed=hq + ws)


def test_backward_bf16_negative_scale(cuda):
    _run(cuda, 1, 60, 4, 2, 128, 8, 40, torch.bfloat16, scale=-0.08)


def test_backward_bf16_varlen_with_lse_gradient(cuda):
    """Packed sequences (every sequence start is a single-pair query) and a gradient on the LSE."""
    from archlab_amd import simplicial_varlen_attention
    lengths = [1, 45, 3, 80]
    t = sum(lengths)
    x = [v[0] for v in rand_inputs(1, t, 8, 2, 128, seed=21, dtype=torch.bfloat16)]
    g = torch.Generator().manual_seed(5)
    dout = torch.randn(t, 8, 128, generator=g).bfloat16()
    dl = torch.randn(t, 8, generator=g)
    cu = torch.tensor([0, 1, 46, 49, 129], dtype=torch.int32)
    xd = [v.to(cuda).requires_grad_(True) for v in x]
    out, lse = simplicial_varlen_attention(*xd, cu.to(cuda), 12, 50, return_lse=True)
    ((out.float() * dout.to(cuda).float()).sum() + (lse * dl.to(cuda)).sum()).backward()
    xs = [v.double().requires_grad_(True) for v in x]
    o, l = O.varlen_reference(*xs, cu, 12, 50, scale=128 ** -0.5, return_lse=True)
    ((o * dout.double()).sum() + (l * dl.double()).sum()).backward()
    _assert_grads([v.grad for v in xd], [v.grad.float() for v in xs], torch.bfloat16, "varlen bf16 + dlse")


def test_backward_mfma_matches_portable(cuda):
    """The MFMA passes and the portable kernels agree to bf16 precision on the same inputs."""
    from archlab_amd import simplicial_attention
    x = [t.to(cuda) for t in rand_inputs(1, 150, 8, 2, 128, seed=12, dtype=torch.bfloat16)]
    dout = torch.randn(1, 150, 8, 128, device=cuda).bfloat16()
    grads = {}
    for kernel in ("auto", "generic"):
        xd = [t.clone().requires_grad_(True) for t in x]
        simplicial_attention(*xd, 32, 96, kernel=kernel).backward(dout)
        grads[kernel] = [t.grad.float() for t in xd]
    for name, a, b in zip(("dq", "dk1", "dk2", "dv1", "dv2"), grads["auto"], grads["generic"]):
        err = (a - b).abs().max().item()
        bound = 2e-2 * max(b.abs().max().item(), 1.0)
        print(f"mfma vs portable {name}: {err:.2e} / {bound:.1e}", flush=True)
        assert err <= bound, name


# ---- dk1 from the dq pass (bf16, short window <= 64): each dq workgroup
# writes, per 32-row group of short keys, a partial of Σ dA_{t,j} ⊙ q_{t,h}
# over its queries and heads that a fixed-order sum turns into dk1 ---------------

@pytest.mark.parametrize("b,n,hq,hk,d,ws,wl", [(1, 200, 4, 4, 128, 32, 96), (2, 37, 3, 3, 64, 20, 70),
                                               (1, 150, 6, 2, 128, 32, 200), (2, 61, 2, 2, 128, 5, 40),
                                               (1, 90, 3, 1, 64, 1, 1), (2, 77, 4, 2, 64, 32, 70),
                                               (1, 50, 8, 2, 128, 32, 100),
                                               (2, 75, 3, 1, 128, 64, 90), (1, 130, 6, 3, 64, 48, 70),
                                               (1, 99, 8, 2, 128, 33, 120)])
def test_backward_bf16_dk1_from_dq(cuda, b, n, hq, hk, d, ws, wl):
    """MHA, GQA groups of 3 (4 queries x 1 head per dq workgroup), 2 (2 x 2)
    and 4 (1 x 4) with one or two 32-row groups of short keys, token counts
    not a multiple of 4 (a partial last query block), batch boundaries inside
    a block, and single pairs."""
    _run(cuda, b, n, hq, hk, d, ws, wl, torch.bfloat16, seed=n + ws)


def test_backward_bf16_dk1_from_dq_varlen_lse(cuda):
    """Packed sequences (starts inside query blocks) and an LSE gradient on the fused path."""
    from archlab_amd import simplicial_varlen_attention
    lengths = [1, 45, 3, 80, 6]
    t = sum(lengths)
    x = [v[0] for v in rand_inputs(1, t, 4, 4, 128, seed=23, dtype=torch.bfloat16)]
    g = torch.Generator().manual_seed(6)
    dout = torch.randn(t, 4, 128, generator=g).bfloat16()
    dl = torch.randn(t, 4, generator=g)
    cu = torch.tensor([0, 1, 46, 49, 129, 135], dtype=torch.int32)
    xd = [v.to(cuda).requires_grad_(True) for v in x]
    out, lse = simplicial_varlen_attention(*xd, cu.to(cuda), 32, 50, return_lse=True)
    ((out.float() * dout.to(cuda).float()).sum() + (lse * dl.to(cuda)).sum()).backward()
    xs = [v.double().requires_grad_(True) for v in x]
    o, l = O.varlen_reference(*xs, cu, 32, 50, scale=128 ** -0.5, return_lse=True)
    ((o * dout.double()).sum() + (l * dl.double()).sum()).backward()
    _assert_grads([v.grad for v in xd], [v.grad.float() for v in xs], torch.bfloat16, "varlen MHA bf16 + dlse")


def test_backward_bf16_dk1_from_dq_deterministic(cuda):
    from archlab_amd import simplicial_attention
    x = [t.to(cuda) for t in rand_inputs(2, 70, 4, 4, 128, seed=9, dtype=torch.bfloat16)]
    dout = torch.randn(2, 70, 4, 128, device=cuda).bfloat16()
    runs = []
    for _ in range(2):
        xd = [t.clone().requires_grad_(True) for t in x]
        simplicial_attention(*xd, 32, 64).backward(dout)
        runs.append([t.grad.clone() for t in xd])
    for a, b in zip(*runs):
        assert torch.equal(a, b)


def test_backward_bf16_dk1_from_dq_matches_portable(cuda):
    """The fused dk1 and the portable kernels' dk1 agree to bf16 precision."""
    from archlab_amd import simplicial_attention
    x = [t.to(cuda) for t in rand_inputs(1, 150, 4, 4, 128, seed=13, dtype=torch.bfloat16)]
    dout = torch.randn(1, 150, 4, 128, device=cuda).bfloat16()
    grads = {}
    for kernel in ("auto", "generic"):
        xd = [t.clone().requires_grad_(True) for t in x]
        simplicial_attention(*xd, 32, 96, kernel=kernel).backward(dout)
        grads[kernel] = [t.grad.float() for t in xd]
    for name, a, b in zip(("dq", "dk1", "dk2", "dv1", "dv2"), grads["auto"], grads["generic"]):
        err = (a - b).abs().max().item()
        bound = 2e-2 * max(b.abs().max().item(), 1.0)
        print(f"fused mfma vs portable {name}: {err:.2e} / {bound:.1e}", flush=True)
        assert err <= bound, name


def test_backward_bf16_separate_dk1_when_partials_do_not_fit(cuda, monkeypatch):
    """When the workspace with the dq pass's dk1 partials cannot be allocated,
    the shim asks again with SA_FLAG_SEPARATE_DK1 (no partials) and dk1 comes
    from its own pass: gradients still match the fp64 oracle."""
    import archlab_amd.architectures.simplicial_attention as shim
    real_empty = torch.empty
    refused = []

    def empty(*size, **kw):
        n = size[0] if size and isinstance(size[0], int) else None
        if kw.get("dtype") is torch.uint8 and n is not None and n > (1 << 20):
            refused.append(n)
            raise torch.cuda.OutOfMemoryError("workspace refused by the test")
        return real_empty(*size, **kw)

    monkeypatch.setattr(shim.torch, "empty", empty)
    _run(cuda, 1, 200, 4, 4, 128, 32, 96, torch.bfloat16, seed=77)
    _run(cuda, 2, 61, 6, 2, 64, 20, 70, torch.bfloat16, seed=78)
    _run(cuda, 1, 200, 4, 4, 128, 64, 96, torch.bfloat16, seed=80)  # two row groups of short keys
    # fp32: the dk1 pass on the matrix cores (shape chosen so that the forward's
    # fp32 workspace stays under the refused size)
    _run(cuda, 1, 200, 4, 2, 128, 32, 96, torch.float32, seed=79)
    monkeypatch.undo()
    assert len(refused) == 4, refused  # one refused partials workspace per call, then the small one


# ---- fp32 inputs on the matrix cores: every operand as hi + lo bf16 terms,
# each product on three term pairs (D == DV in {64, 128}, short window <= 32;
# the reference's DeepSeek-V4.1 adapter sends fp32, deepseek_v41_adapter.py:136-144)

@pytest.mark.parametrize("b,n,hq,hk,d,ws,wl", [(1, 300, 8, 2, 128, 32, 256), (2, 70, 3, 1, 64, 20, 40),
                                               (1, 150, 4, 4, 128, 32, 96), (2, 61, 2, 2, 64, 5, 40),
                                               (1, 90, 3, 1, 64, 1, 1), (1, 77, 6, 2, 128, 7, 33)])
def test_backward_fp32_matrix_cores(cuda, b, n, hq, hk, d, ws, wl):
    _run(cuda, b, n, hq, hk, d, ws, wl, torch.float32, seed=n + ws)


def test_backward_fp32_matrix_cores_varlen_lse_and_repeatable(cuda):
    """Packed sequences and an LSE gradient at fp32 on the matrix cores; the
    result repeats bit for bit and differs from the portable kernels' (a
    different summation), both within 1e-4 of the fp64 oracle."""
    from archlab_amd import simplicial_varlen_attention
    lengths = [1, 45, 3, 80, 6]
    t = sum(lengths)
    x = [v[0] for v in rand_inputs(1, t, 8, 2, 128, seed=29, dtype=torch.float32)]
    g = torch.Generator().manual_seed(30)
    dout = torch.randn(t, 8, 128, generator=g)
    dl = torch.randn(t, 8, generator=g)
    cu = torch.tensor([0, 1, 46, 49, 129, 135], dtype=torch.int32)
    runs = {}
    for kernel in ("auto", "auto", "generic"):
        xd = [v.to(cuda).requires_grad_(True) for v in x]
        out, lse = simplicial_varlen_attention(*xd, cu.to(cuda), 32, 50, return_lse=True, kernel=kernel)
        ((out * dout.to(cuda)).sum() + (lse * dl.to(cuda)).sum()).backward()
        runs.setdefault(kernel, []).append([v.grad.clone() for v in xd])
    xs = [v.double().requires_grad_(True) for v in x]
    o, l = O.varlen_reference(*xs, cu, 32, 50, scale=128 ** -0.5, return_lse=True)
    ((o * dout.double()).sum() + (l * dl.double()).sum()).backward()
    ref = [v.grad.float() for v in xs]
    _assert_grads(runs["auto"][0], ref, torch.float32, "varlen fp32 matrix cores + dlse")
    _assert_grads(runs["generic"][0], ref, torch.float32, "varlen fp32 portable + dlse")
    assert all(torch.equal(a, b) for a, b in zip(*runs["auto"]))
    assert not all(torch.equal(a, b) for a, b in zip(runs["auto"][0], runs["generic"][0]))


@pytest.mark.parametrize("d,dv", [(16, 16), (32, 32), (32, 64)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_backward_narrow_widths_padded_onto_matrix_cores(cuda, d, dv, dtype):
    """Widths 16 and 32 zero-padded onto the matrix-core passes: the gradients
    of the unpadded tensors come back through the pad."""
    _run(cuda, 1, 90, 4, 2, d, 16, 48, dtype, dv=dv, seed=d + dv)


@pytest.mark.parametrize("hk", [16, 8])
def test_backward_bf16_dk2_workgroup_widths_match_portable(cuda, hk):
    """8192 tokens: 16 KV heads select 8-wave (256-key) dk2/dv2 workgroups,
    8 KV heads 4-wave (128-key) ones, as do the small shapes checked against
    the oracle above; gradients agree with the portable kernels."""
    from archlab_amd import simplicial_attention
    x = [t.to(cuda) for t in rand_inputs(1, 8192, hk, hk, 128, seed=hk, dtype=torch.bfloat16)]
    g = torch.Generator().manual_seed(hk + 1)
    dout = torch.randn(1, 8192, hk, 128, generator=g).bfloat16().to(cuda)
    grads = {}
    for kernel in ("auto", "generic"):
        xd = [t.clone().requires_grad_(True) for t in x]
        simplicial_attention(*xd, 32, 64, kernel=kernel).backward(dout)
        grads[kernel] = [t.grad.float() for t in xd]
    for name, a, b in zip(("dq", "dk1", "dk2", "dv1", "dv2"), grads["auto"], grads["generic"]):
        err = (a - b).abs().max().item()
        bound = 2e-2 * max(b.abs().max().item(), 1.0)
        print(f"hk {hk}: mfma vs portable {name}: {err:.2e} / {bound:.1e}", flush=True)
        assert err <= bound, name


# ---- dk2 / dv2 walk pieces: with few (key block, KV head) workgroups each
# walk over the queries is cut into up to 8 pieces whose fp32 sums are added
# in a fixed order; a last key block shorter than the piece count leaves some
# pieces empty (they write zero sums) ------------------------------------------

@pytest.mark.parametrize("b,n,hq,hk,d,ws,wl", [(1, 129, 2, 2, 128, 32, 512), (1, 130, 4, 2, 64, 20, 300),
                                               (2, 129, 2, 1, 128, 64, 400), (1, 700, 8, 1, 128, 32, 512)])
def test_backward_bf16_dk2_walk_pieces(cuda, b, n, hq, hk, d, ws, wl):
    _run(cuda, b, n, hq, hk, d, ws, wl, torch.bfloat16, seed=n + wl)


def test_backward_bf16_dk2_walk_pieces_varlen_repeatable(cuda):
    """Packed sequences across walk pieces, against the oracle, and bitwise repeatable."""
    from archlab_amd import simplicial_varlen_attention
    lengths = [1, 300, 7, 180, 2]
    t = sum(lengths)
    x = [v[0] for v in rand_inputs(1, t, 4, 1, 128, seed=41, dtype=torch.bfloat16)]
    g = torch.Generator().manual_seed(12)
    dout = torch.randn(t, 4, 128, generator=g).bfloat16()
    cu = torch.tensor([0, 1, 301, 308, 488, 490], dtype=torch.int32)
    runs = []
    for _ in range(2):
        xd = [v.to(cuda).requires_grad_(True) for v in x]
        out = simplicial_varlen_attention(*xd, cu.to(cuda), 32, 400)
        (out.float() * dout.to(cuda).float()).sum().backward()
        runs.append([v.grad for v in xd])
    for a, b in zip(*runs):
        assert torch.equal(a, b)
    xs = [v.double().requires_grad_(True) for v in x]
    o = O.varlen_reference(*xs, cu, 32, 400, scale=128 ** -0.5)
    (o * dout.double()).sum().backward()
    _assert_grads(runs[0], [v.grad.float() for v in xs], torch.bfloat16, "varlen bf16 walk pieces")


# ---- dk2 / dv2 on the matrix cores with short windows of 33-64 (two 32-row
# groups of short keys per step) ----------------------------------------------------

@pytest.mark.parametrize("b,n,hq,hk,d,ws,wl", [(1, 150, 4, 4, 128, 64, 100), (2, 70, 4, 2, 64, 33, 90),
                                               (1, 120, 8, 2, 128, 50, 200), (1, 90, 3, 3, 64, 64, 64)])
def test_backward_bf16_two_short_row_groups(cuda, b, n, hq, hk, d, ws, wl):
    _run(cuda, b, n, hq, hk, d, ws, wl, torch.bfloat16, seed=n + ws)


def test_backward_bf16_two_short_row_groups_varlen(cuda):
    """Packed sequences shorter and longer than the 64-key short window."""
    from archlab_amd import simplicial_varlen_attention
    lengths = [1, 70, 5, 60, 3]
    t = sum(lengths)
    x = [v[0] for v in rand_inputs(1, t, 4, 2, 128, seed=31, dtype=torch.bfloat16)]
    g = torch.Generator().manual_seed(8)
    dout = torch.randn(t, 4, 128, generator=g).bfloat16()
    cu = torch.tensor([0, 1, 71, 76, 136, 139], dtype=torch.int32)
    xd = [v.to(cuda).requires_grad_(True) for v in x]
    out = simplicial_varlen_attention(*xd, cu.to(cuda), 64, 80)
    (out.float() * dout.to(cuda).float()).sum().backward()
    xs = [v.double().requires_grad_(True) for v in x]
    o = O.varlen_reference(*xs, cu, 64, 80, scale=128 ** -0.5)
    (o * dout.double()).sum().backward()
    _assert_grads([v.grad for v in xd], [v.grad.float() for v in xs], torch.bfloat16, "varlen bf16 ws 64")


def test_backward_bf16_two_short_row_groups_match_portable(cuda):
    from archlab_amd import simplicial_attention
    x = [t.to(cuda) for t in rand_inputs(1, 160, 4, 4, 128, seed=17, dtype=torch.bfloat16)]
    dout = torch.randn(1, 160, 4, 128, device=cuda).bfloat16()
    grads = {}
    for kernel in ("auto", "generic"):
        xd = [t.clone().requires_grad_(True) for t in x]
        simplicial_attention(*xd, 64, 96, kernel=kernel).backward(dout)
        grads[kernel] = [t.grad.float() for t in xd]
    for name, a, b in zip(("dq", "dk1", "dk2", "dv1", "dv2"), grads["auto"], grads["generic"]):
        err = (a - b).abs().max().item()
        bound = 2e-2 * max(b.abs().max().item(), 1.0)
        print(f"ws 64 mfma vs portable {name}: {err:.2e} / {bound:.1e}", flush=True)
        assert err <= bound, name


# ---- score width DK != value width DV on the matrix cores (the determinant
# expansion's operands are DK = 128 over DV = 64 value heads) -----------------------

@pytest.mark.parametrize("b,n,hq,hk,d,dv,ws,wl", [
    (1, 150, 4, 4, 128, 64, 32, 96),  # MHA, dk1 from the dq pass
    (2, 61, 6, 3, 128, 64, 20, 70),   # GQA 2
    (1, 90, 8, 2, 128, 64, 64, 100),  # GQA 4, two short row groups (dk1 partials per row group)
    (1, 77, 3, 1, 64, 128, 32, 50),   # DV > DK, GQA 3
    (2, 40, 4, 2, 64, 128, 45, 60),   # DV > DK, two short row groups
    (1, 50, 2, 2, 128, 64, 1, 1),     # single pairs
])
def test_backward_bf16_value_width_differs(cuda, b, n, hq, hk, d, dv, ws, wl):
    _run(cuda, b, n, hq, hk, d, ws, wl, torch.bfloat16, dv=dv, seed=n + ws)


def test_backward_bf16_value_width_differs_varlen_lse(cuda):
    from archlab_amd import simplicial_varlen_attention
    lengths = [1, 45, 3, 80, 6]
    t = sum(lengths)
    x = [v[0] for v in rand_inputs(1, t, 8, 2, 128, dv=64, seed=27, dtype=torch.bfloat16)]
    g = torch.Generator().manual_seed(9)
    dout = torch.randn(t, 8, 64, generator=g).bfloat16()
    dl = torch.randn(t, 8, generator=g)
    cu = torch.tensor([0, 1, 46, 49, 129, 135], dtype=torch.int32)
    xd = [v.to(cuda).requires_grad_(True) for v in x]
    out, lse = simplicial_varlen_attention(*xd, cu.to(cuda), 32, 50, return_lse=True)
    ((out.float() * dout.to(cuda).float()).sum() + (lse * dl.to(cuda)).sum()).backward()
    xs = [v.double().requires_grad_(True) for v in x]
    o, l = O.varlen_reference(*xs, cu, 32, 50, scale=128 ** -0.5, return_lse=True)
    ((o * dout.double()).sum() + (l * dl.double()).sum()).backward()
    _assert_grads([v.grad for v in xd], [v.grad.float() for v in xs], torch.bfloat16, "varlen DK 128 DV 64 + dlse")


@pytest.mark.parametrize("d,dv,ws", [(128, 64, 32), (64, 128, 64)])
def test_backward_bf16_value_width_differs_matches_portable_and_repeats(cuda, d, dv, ws):
    """Against the portable kernels to bf16 precision; a second call is bitwise identical."""
    from archlab_amd import simplicial_attention
    x = [t.to(cuda) for t in rand_inputs(1, 130, 4, 2, d, dv=dv, seed=d + ws, dtype=torch.bfloat16)]
    dout = torch.randn(1, 130, 4, dv, device=cuda).bfloat16()
    runs = []
    for kernel in ("auto", "auto", "generic"):
        xd = [t.clone().requires_grad_(True) for t in x]
        simplicial_attention(*xd, ws, 96, kernel=kernel).backward(dout)
        runs.append([t.grad.float() for t in xd])
    for name, a, a2, b in zip(("dq", "dk1", "dk2", "dv1", "dv2"), *runs):
        assert torch.equal(a, a2), name
        err = (a - b).abs().max().item()
        bound = 2e-2 * max(b.abs().max().item(), 1.0)
        print(f"DK {d} DV {dv} ws {ws} mfma vs portable {name}: {err:.2e} / {bound:.1e}", flush=True)
        assert err <= bound, name


# ---- score width 256 (D = 256 heads, and DK 256 / DV 128 from the determinant
# expansion of 128-wide heads) on the matrix cores at one wave per SIMD; dk2 /
# dv2 with a short window of 33-64 run one launch per 32-row group ------------------

@pytest.mark.parametrize("b,n,hq,hk,d,dv,ws,wl", [
    (1, 90, 4, 2, 256, 256, 32, 96),   # GQA 2, dk1 from the dq pass
    (2, 37, 3, 3, 256, 256, 20, 40),   # MHA (4 queries per dq workgroup), partial last block
    (1, 70, 8, 2, 256, 128, 32, 64),   # GQA 4, DV 128
    (1, 60, 4, 4, 256, 256, 40, 60),   # two short row groups: dk1 from the dq pass, dk2 / dv2 in two launches
    (1, 80, 4, 2, 256, 128, 64, 100),  # a full 64-key short window, GQA 2, DV 128
    (1, 50, 2, 2, 256, 256, 70, 80),   # short window past 64: portable dk2 / dv2
    (1, 33, 2, 2, 256, 128, 1, 1),     # single pairs
])
def test_backward_bf16_score_width_256(cuda, b, n, hq, hk, d, dv, ws, wl):
    _run(cuda, b, n, hq, hk, d, ws, wl, torch.bfloat16, dv=dv, seed=n + ws)


def test_backward_bf16_score_width_256_varlen_lse_matches_portable_and_repeats(cuda):
    from archlab_amd import simplicial_varlen_attention
    cu = torch.tensor([0, 1, 30, 33, 90], dtype=torch.int32)
    x = [v[0] for v in rand_inputs(1, 90, 4, 2, 256, seed=41, dtype=torch.bfloat16)]
    g = torch.Generator().manual_seed(10)
    dout = torch.randn(90, 4, 256, generator=g).bfloat16()
    dl = torch.randn(90, 4, generator=g)
    runs = []
    for kernel in ("auto", "auto", "generic"):
        xd = [v.to(cuda).requires_grad_(True) for v in x]
        out, lse = simplicial_varlen_attention(*xd, cu.to(cuda), 32, 40, return_lse=True, kernel=kernel)
        ((out.float() * dout.to(cuda).float()).sum() + (lse * dl.to(cuda)).sum()).backward()
        runs.append([v.grad.float() for v in xd])
    xs = [v.double().requires_grad_(True) for v in x]
    o, l = O.varlen_reference(*xs, cu, 32, 40, scale=256 ** -0.5, return_lse=True)
    ((o * dout.double()).sum() + (l * dl.double()).sum()).backward()
    _assert_grads(runs[0], [v.grad.float() for v in xs], torch.bfloat16, "varlen D 256 + dlse")
    for name, a, a2, b in zip(("dq", "dk1", "dk2", "dv1", "dv2"), *runs):
        assert torch.equal(a, a2), name
        err = (a - b).abs().max().item()
        bound = 2e-2 * max(b.abs().max().item(), 1.0)
        print(f"D 256 mfma vs portable {name}: {err:.2e} / {bound:.1e}", flush=True)
        assert err <= bound, name


# ---- dk2 / dv2 on the matrix cores with short windows of 65-128 at widths
# <= 128: two launches of two 32-row groups, the second starting from the
# first's fp32 sums ------------------------------------------------------------------

@pytest.mark.parametrize("b,n,hq,hk,d,dv,ws,wl", [
    (1, 160, 4, 4, 128, 128, 100, 120),  # MHA
    (2, 90, 4, 2, 64, 64, 128, 130),     # the full 128-key window, GQA 2, batch of two
    (1, 120, 8, 2, 128, 64, 80, 100),    # GQA 4, DK 128 / DV 64
    (1, 70, 2, 2, 64, 128, 65, 70),      # one row past a single launch
])
def test_backward_bf16_short_windows_past_64(cuda, b, n, hq, hk, d, dv, ws, wl):
    _run(cuda, b, n, hq, hk, d, ws, wl, torch.bfloat16, dv=dv, seed=n + ws)


def test_backward_bf16_short_windows_past_64_varlen_matches_portable_and_repeats(cuda):
    from archlab_amd import simplicial_varlen_attention
    cu = torch.tensor([0, 3, 120, 121, 200], dtype=torch.int32)
    x = [v[0] for v in rand_inputs(1, 200, 4, 2, 128, seed=43, dtype=torch.bfloat16)]
    g = torch.Generator().manual_seed(11)
    dout = torch.randn(200, 4, 128, generator=g).bfloat16()
    runs = []
    for kernel in ("auto", "auto", "generic"):
        xd = [v.to(cuda).requires_grad_(True) for v in x]
        out = simplicial_varlen_attention(*xd, cu.to(cuda), 110, 120, kernel=kernel)
        (out.float() * dout.to(cuda).float()).sum().backward()
        runs.append([v.grad.float() for v in xd])
    xs = [v.double().requires_grad_(True) for v in x]
    o = O.varlen_reference(*xs, cu, 110, 120, scale=128 ** -0.5)
    (o * dout.double()).sum().backward()
    _assert_grads(runs[0], [v.grad.float() for v in xs], torch.bfloat16, "varlen ws 110")
    for name, a, a2, b in zip(("dq", "dk1", "dk2", "dv1", "dv2"), *runs):
        assert torch.equal(a, a2), name
        err = (a - b).abs().max().item()
        bound = 2e-2 * max(b.abs().max().item(), 1.0)
        print(f"ws 110 mfma vs portable {name}: {err:.2e} / {bound:.1e}", flush=True)
        assert err <= bound, name


def test_backward_c4_full_size_dk1_partials_match_separate_pass(cuda, monkeypatch):
    """C4 at its full size (S 16384, H 8, D 256, windows 256 x 64: two 32-row
    groups of short keys): dk1 from the dq pass's per-group partials agrees with
    the separate dk1 pass to bf16 precision, the other gradients come from the
    same kernels either way (bitwise equal), and a second call is bitwise
    identical."""
    import archlab_amd.architectures.simplicial_attention as shim
    from archlab_amd import simplicial_attention
    from archlab_amd import workloads as W
    cfg = W.C4
    q, k1, k2, v1, v2, _ = W.prefill_inputs(cfg, device=cuda)
    dout = torch.randn(q.shape[:-1] + (v1.shape[-1],), device=cuda).to(cfg.dtype)

    def grads():
        xd = [t.detach().clone().requires_grad_(True) for t in (q, k1, k2, v1, v2)]
        out = simplicial_attention(*xd, cfg.w2, cfg.w1, scale=1.0)  # q carries 1/sqrt(D)
        out.backward(dout)
        return [t.grad for t in xd]

    fused = grads()
    again = grads()
    for name, a, b in zip(("dq", "dk1", "dk2", "dv1", "dv2"), fused, again):
        assert torch.equal(a, b), name
    real_empty = torch.empty

    def empty(*size, **kw):  # refuse the workspace that holds the dk1 partials (2.3 GB at C4)
        n = size[0] if size and isinstance(size[0], int) else None
        if kw.get("dtype") is torch.uint8 and n is not None and n > (1 << 30):
            raise torch.cuda.OutOfMemoryError("workspace refused by the test")
        return real_empty(*size, **kw)

    monkeypatch.setattr(shim.torch, "empty", empty)
    separate = grads()
    monkeypatch.undo()
    for name, a, b in zip(("dq", "dk1", "dk2", "dv1", "dv2"), fused, separate):
        a, b = a.float(), b.float()
        err = (a - b).abs().max().item()
        bound = 1e-2 * max(b.abs().max().item(), 1.0)
        print(f"C4 fused vs separate dk1 {name}: {err:.2e} / {bound:.1e}", flush=True)
        if name in ("dk2", "dv1", "dv2"):
            assert torch.equal(a, b), name
        else:
            assert err <= bound, name


def test_backward_fp32_dv1_partials_match_separate_pass(cuda, monkeypatch):
    """The reference DeepSeek-V4.1 adapter shape in fp32 (B2 S8192, Hq 8 / Hkv 2,
    D 128, windows 32 x 512): dk1 and dv1 from the dq pass's partials agree
    with the separate dk1 / dv1 pass to fp32 precision (a different summation
    order), dk2 and dv2 come from the same kernel either way (bitwise equal),
    dq from the same arithmetic, and a second call is bitwise identical."""
    import archlab_amd.architectures.simplicial_attention as shim
    from archlab_amd import simplicial_attention
    from archlab_amd import workloads as W
    cfg = W.DSV41
    q, k1, k2, v1, v2, _ = W.prefill_inputs(cfg, device=cuda)
    g = torch.Generator("cpu").manual_seed(5)
    dout = torch.randn(q.shape[:-1] + (v1.shape[-1],), generator=g).to(cuda)

    def grads():
        xd = [t.detach().clone().requires_grad_(True) for t in (q, k1, k2, v1, v2)]
        out = simplicial_attention(*xd, cfg.w2, cfg.w1, scale=1.0)
        out.backward(dout)
        return [t.grad for t in xd]

    fused = grads()
    again = grads()
    for name, a, b in zip(("dq", "dk1", "dk2", "dv1", "dv2"), fused, again):
        assert torch.equal(a, b), name
    real_empty = torch.empty

    def empty(*size, **kw):  # refuse the workspace that holds the partials (1.1 GB here)
        n = size[0] if size and isinstance(size[0], int) else None
        if kw.get("dtype") is torch.uint8 and n is not None and n > (256 << 20):
            raise torch.cuda.OutOfMemoryError("workspace refused by the test")
        return real_empty(*size, **kw)

    monkeypatch.setattr(shim.torch, "empty", empty)
    separate = grads()
    monkeypatch.undo()
    for name, a, b in zip(("dq", "dk1", "dk2", "dv1", "dv2"), fused, separate):
        err = (a - b).abs().max().item()
        bound = 1e-5 * max(b.abs().max().item(), 1.0)
        print(f"DSV41 fp32 fused vs separate dk1 / dv1 {name}: {err:.2e} / {bound:.1e}", flush=True)
        if name in ("dk2", "dv2"):
            assert torch.equal(a, b), name
        else:
            assert err <= bound, name


@pytest.mark.parametrize("name", ["NS", "DSV41-bf16", "DSV41"])
def test_backward_full_size_matches_portable(cuda, name):
    """Full-size workloads, the matrix-core backward against the portable
    fp32-arithmetic kernels on the same inputs: NS (8-wave dk2 / dv2
    workgroups, dk1 from the dq pass), the reference DeepSeek-V4.1 adapter
    geometry (HQ 8 / HKV 2, windows 32 / 512, 2 x 8192 tokens) in bf16 (4-wave
    dk2 / dv2 workgroups whose walks over the queries are split into pieces)
    and in fp32 (hi/lo bf16 terms).  bf16 to 2e-2 x max|grad| (both paths round
    the same operands to bf16 and differ in fp32 summation order), fp32 to
    1e-4 x max|grad|."""
    import dataclasses
    from archlab_amd import simplicial_attention
    from archlab_amd import workloads as W
    cfg = {"NS": W.NS, "DSV41-bf16": dataclasses.replace(W.DSV41, dtype=torch.bfloat16), "DSV41": W.DSV41}[name]
    q, k1, k2, v1, v2, _ = W.prefill_inputs(cfg, device=cuda)
    g = torch.Generator().manual_seed(5)
    dout = torch.randn(q.shape[:-1] + (v1.shape[-1],), generator=g).to(cfg.dtype).to(cuda)
    grads = {}
    for kernel in ("auto", "generic"):
        xd = [t.detach().clone().requires_grad_(True) for t in (q, k1, k2, v1, v2)]
        simplicial_attention(*xd, cfg.w2, cfg.w1, scale=1.0, kernel=kernel).backward(dout)  # q carries 1/sqrt(D)
        grads[kernel] = [t.grad.float() for t in xd]
        del xd
    rtol = 1e-4 if cfg.dtype == torch.float32 else 2e-2
    for gname, a, b in zip(("dq", "dk1", "dk2", "dv1", "dv2"), grads["auto"], grads["generic"]):
        assert torch.isfinite(a).all(), gname
        err = (a - b).abs().max().item()
        bound = rtol * max(b.abs().max().item(), 1.0)
        print(f"{name} full size: mfma vs portable {gname}: {err:.2e} / {bound:.1e}", flush=True)
        assert err <= bound, gname
