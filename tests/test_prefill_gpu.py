"""GPU parity of the prefill kernels (dense and packed varlen) against the CPU oracle.

Inputs are seeded; the oracle receives exactly the values the kernel sees
(bf16 inputs upcast to fp32).  Tolerances: bf16 out max-abs <= 2e-2 and LSE
relative <= 1e-3; fp32 <= 1e-4.
"""

import os

import numpy as np
import pytest
import torch

from helpers import assert_lse_close, assert_out_close, rand_inputs
from oracle import simplicial_oracle as O

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "simplicial_golden.npz")


def _api():
    from archlab_amd.architectures.simplicial_attention import (
        prefill_kernel_name, simplicial_attention, simplicial_varlen_attention)
    return simplicial_attention, simplicial_varlen_attention, prefill_kernel_name


# (max relative LSE error against the fp32 oracle at positions with < 64
# pairs, case) of every bf16 check in this module, for the closing report
_FEW_PAIR_LSE = []


def _check(cuda, b, n, hq, hk, d, ws, wl, dtype, seed=0, positions=None, scale=1.0, sigma=1.0, kernel="auto",
           dv=None, mutate=None):
    """Kernel vs oracle on seeded inputs; returns (out, lse) at ``positions``.

    bf16 criteria (all printed before asserting):
      * out vs the fp32 oracle: max-abs <= 2e-2 (+ half a bf16 ulp of |ref|);
      * lse vs the fp32 oracle: rel <= 1e-3 at positions whose windows hold
        >= 64 (j, k) pairs, rel <= 1e-2 everywhere -- with a handful of pairs
        the LSE carries the bf16 rounding of a = q ⊙ k1 that the reference
        kernel applies (simplicial_kernels.py:35) undiluted;
      * vs the oracle with that same rounding point (kernel_rounding_reference):
        lse rel <= 1e-4 at every position, and out <= 4e-3 (+ one bf16 ulp)
        at positions with >= 64 pairs -- that oracle keeps P in float64,
        while the kernel (like the reference kernel, simplicial_kernels.py:48)
        rounds P to bf16 against its running max, an error a handful of
        pairs does not average out.
    """
    attn, _, name = _api()
    x = rand_inputs(b, n, hq, hk, d, dv=dv, seed=seed, dtype=dtype, sigma=sigma)
    if mutate is not None:
        x = mutate(x)
    out, lse = attn(*(t.to(cuda) for t in x), ws, wl, scale=scale, return_lse=True, kernel=kernel)
    torch.cuda.synchronize()
    pos = list(range(n)) if positions is None else list(positions)
    ref_o, ref_l = O.reference_simplicial(*(t.float() for t in x), ws, wl, scale=scale,
                                          query_positions=pos, return_lse=True)
    out, lse = out[:, pos].cpu(), lse[:, pos].cpu()
    label = f"[{name(x[0], x[1], x[3], kernel=kernel)}] b{b} n{n} h{hq}/{hk} d{d} w{ws}x{wl} {dtype}"
    if dtype != torch.bfloat16:
        e1 = assert_out_close(out, ref_o, dtype)
        e2 = assert_lse_close(lse, ref_l, dtype)
        print(f"{label}: out {e1:.2e} lse {e2:.2e}", flush=True)
        return out, lse
    full = [i for i, p in enumerate(pos) if min(p + 1, ws) * min(p + 1, wl) >= 64]
    few = [i for i, p in enumerate(pos) if min(p + 1, ws) * min(p + 1, wl) < 64]
    ro, rl = O.kernel_rounding_reference(*x, ws, wl, scale=scale, query_positions=pos)
    rel = lambda a, e: ((a.float() - e.float()).abs() / e.float().abs().clamp_min(1.0)).max().item()  # noqa: E731
    stats = {
        "out": (out.float() - ref_o).abs().max().item(),
        "lse_full": rel(lse[:, full], ref_l[:, full]) if full else 0.0,
        "lse_few": rel(lse[:, few], ref_l[:, few]) if few else 0.0,
        "lse_all": rel(lse, ref_l),
        "r_out": (out.float() - ro.float()).abs().max().item(),
        "r_lse": rel(lse, rl),
    }
    print(label + ": " + " ".join(f"{k} {v:.2e}" for k, v in stats.items()), flush=True)
    if few:
        _FEW_PAIR_LSE.append((stats["lse_few"], label))
    assert_out_close(out, ref_o, dtype)
    if full:
        assert_lse_close(lse[:, full], ref_l[:, full], dtype)
    assert_lse_close(lse, ref_l, dtype, rtol=1e-2)
    if full:
        assert_out_close(out[:, full], ro[:, full], dtype, atol=4e-3, rtol=2.0 ** -7)
    assert_lse_close(lse, rl, dtype, rtol=1e-4)
    return out, lse


def test_golden_fixtures_fp32(cuda):
    attn, _, _ = _api()
    data = np.load(GOLDEN)
    names = sorted({k.split("/")[0] for k in data.files})
    ran = 0
    for nm in names:
        b, n, hq, hk, d, ws, wl, seed = data[f"{nm}/meta"].tolist()
        if d < 16:  # the kernels accept score head dims 16..512 (reference contract)
            continue
        ran += 1
        x = [torch.from_numpy(data[f"{nm}/{k}"]).float().to(cuda) for k in ("q", "k1", "k2", "v1", "v2")]
        out, lse = attn(*x, ws, wl, return_lse=True)
        torch.testing.assert_close(out.cpu().double(), torch.from_numpy(data[f"{nm}/out"]), rtol=1e-4, atol=1e-4)
        torch.testing.assert_close(lse.cpu().double(), torch.from_numpy(data[f"{nm}/lse"]), rtol=1e-4, atol=1e-4)
    assert ran >= 3


def test_c1_fp32_full(cuda):
    """B1 H4 S512 D64, w1=32 (long), w2=16 (short), fp32, seed 0."""
    _check(cuda, 1, 512, 4, 4, 64, 16, 32, torch.float32, seed=0)


@pytest.mark.parametrize("d", [64, 128, 256])
@pytest.mark.parametrize("hq,hk", [(4, 4), (4, 2), (8, 2), (3, 1)])
def test_mfma_small_windows(cuda, d, hq, hk):
    _check(cuda, 2, 150, hq, hk, d, 16, 64, torch.bfloat16, seed=d + hq, kernel="mfma")


@pytest.mark.parametrize("ws,wl", [(1, 1), (5, 33), (32, 32), (33, 100), (64, 256), (100, 130), (32, 10_000)])
def test_mfma_window_edges(cuda, ws, wl):
    _check(cuda, 1, 300, 4, 2, 128, ws, wl, torch.bfloat16, seed=ws * 7 + wl, kernel="mfma")


@pytest.mark.parametrize("d,dv", [(128, 64), (256, 128), (512, 256)])
@pytest.mark.parametrize("hq,hk", [(4, 4), (8, 2), (3, 1)])
def test_mfma_score_and_value_widths_differ(cuda, d, dv, hq, hk):
    """Score width DK != value width DV (the determinant expansion's DK = 2 DV) on the MFMA kernel."""
    _check(cuda, 2, 150, hq, hk, d, 16, 64, torch.bfloat16, seed=d + dv + hq, kernel="mfma", dv=dv)


@pytest.mark.parametrize("ws,wl", [(1, 1), (33, 100), (5, 300)])
def test_mfma_score_and_value_widths_differ_windows(cuda, ws, wl):
    _check(cuda, 1, 320, 4, 2, 128, ws, wl, torch.bfloat16, seed=ws + wl, kernel="mfma", dv=64)
    _check(cuda, 1, 200, 8, 2, 256, ws, wl, torch.bfloat16, seed=ws + wl + 1, kernel="mfma", dv=128)
    # score width 512 (the determinant expansion of 256-wide heads), one wave per SIMD
    _check(cuda, 1, 160, 4, 2, 512, ws, wl, torch.bfloat16, seed=ws + wl + 2, kernel="mfma", dv=256)


def test_mfma_score_and_value_widths_differ_varlen(cuda):
    _, varlen, _ = _api()
    lengths = [3, 140, 61]
    cu = torch.tensor([0, 3, 143, 204], dtype=torch.int32)
    x = rand_inputs(1, sum(lengths), 8, 2, 256, dv=128, seed=31)
    out, lse = varlen(*(v[0].to(cuda) for v in x), cu.to(cuda), 40, 96, scale=1.0, return_lse=True,
                      kernel="mfma")
    ref_o, ref_l = O.varlen_reference(*(v[0].float() for v in x), cu, 40, 96, scale=1.0, return_lse=True)
    assert_out_close(out, ref_o, torch.bfloat16)
    assert_lse_close(lse, ref_l, torch.bfloat16, rtol=1e-2)


def test_mfma_production_windows(cuda):
    """Reference production geometry: short 32, long 512, GQA 4, positions across both edges."""
    pos = [0, 1, 30, 31, 32, 33, 100, 510, 511, 512, 513, 700, 1023, 1100, 1199]
    _check(cuda, 1, 1200, 8, 2, 128, 32, 512, torch.bfloat16, seed=5, positions=pos, kernel="mfma")


@pytest.mark.parametrize("boost", [8.0, 32.0])
def test_mfma_reference_max_moves_mid_window(cuda, boost):
    """A few long-axis keys whose scores stand far above the rest, met in a
    later chunk of the window.  At boost 8 the spike (~13 above the first
    chunks' maximum, in log2 units) stays under the 2^24 row-sum bound: its
    probabilities, up to ~2^13, are taken against the old reference max.  At
    boost 32 (~58 above) the bound is passed and the kernel moves the
    reference to the chunk maxima and recomputes that chunk.  q and k1 are put on grids
    whose products are exact in bf16 (4 significant bits each) and the spike
    is a power-of-two multiple of k2 rows, so that the reference's rounding of
    a = q ⊙ k1 does not turn the large scores into large errors and the
    fp32 oracle applies unchanged."""
    def spike(x):
        q, k1, k2, v1, v2 = (t.float() for t in x)
        q = (q * 64).round().clamp(-15, 15) / 8       # k/8, |k| <= 15
        k1 = (k1 * 4).round().clamp(-15, 15) / 4      # k/4, |k| <= 15
        k2 = k2.clone()
        k2[:, 300:304] *= boost
        return [t.to(x[0].dtype) for t in (q, k1, k2, v1, v2)]
    pos = [299, 300, 301, 310, 333, 400, 511, 600, 700, 811, 814, 815, 900]
    _check(cuda, 1, 960, 4, 4, 128, 32, 512, torch.bfloat16, seed=11, positions=pos, scale=0.05, kernel="mfma",
           mutate=spike)


def test_mfma_scale_variants(cuda):
    _check(cuda, 1, 200, 4, 4, 64, 8, 40, torch.bfloat16, seed=3, scale=None, kernel="mfma")
    _check(cuda, 1, 200, 4, 4, 64, 8, 40, torch.bfloat16, seed=3, scale=-0.7, kernel="mfma")
    _check(cuda, 1, 200, 4, 4, 64, 8, 40, torch.bfloat16, seed=3, scale=0.0, kernel="mfma")


def test_generic_bf16_and_fp32(cuda):
    _check(cuda, 1, 100, 4, 2, 128, 16, 40, torch.bfloat16, seed=1, kernel="generic")
    _check(cuda, 1, 100, 4, 2, 32, 16, 40, torch.float32, seed=2, kernel="generic")
    _check(cuda, 1, 70, 2, 1, 512, 8, 20, torch.float32, seed=4, dv=64)
    _check(cuda, 1, 70, 2, 2, 16, 3, 9, torch.bfloat16, seed=6)


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("hq,hk", [(4, 4), (8, 2), (3, 1)])
@pytest.mark.parametrize("ws,wl", [(1, 1), (16, 64), (33, 100), (32, 512)])
def test_fp32_inputs_on_matrix_cores(cuda, d, hq, hk, ws, wl):
    """fp32 inputs (the DeepSeek-V4.1 caller's core dtype, deepseek_v41_adapter.py:138-144)
    run on the MFMA kernel with hi/lo bf16 terms; parity at the fp32
    tolerance (1e-4) against the oracle, and against the portable kernel."""
    attn, _, name = _api()
    x = rand_inputs(1, 600, hq, hk, d, seed=d + hq + ws, dtype=torch.float32)
    assert name(x[0], x[1], x[3]) == "mfma"
    pos = sorted({0, 1, ws - 1, ws, wl - 1, wl, 299, 599} & set(range(600)))
    out, lse = _check(cuda, 1, 600, hq, hk, d, ws, wl, torch.float32, seed=d + hq + ws, positions=pos)
    xd = [t.to(cuda) for t in x]
    gen, gl = attn(*xd, ws, wl, scale=1.0, return_lse=True, kernel="generic")
    assert_out_close(out, gen[:, pos].cpu(), torch.float32)
    assert_lse_close(lse, gl[:, pos].cpu(), torch.float32)


def test_fp32_varlen_on_matrix_cores(cuda):
    _, varlen, _ = _api()
    lengths = [1, 37, 300, 5, 129]
    x = rand_inputs(1, sum(lengths), 8, 2, 128, seed=23, dtype=torch.float32)
    cu = torch.tensor([0] + list(np.cumsum(lengths)), dtype=torch.int32)
    out, lse = varlen(*(v[0].to(cuda) for v in x), cu.to(cuda), 16, 64, scale=1.0, return_lse=True, kernel="mfma")
    ref_o, ref_l = O.varlen_reference(*(v[0] for v in x), cu, 16, 64, scale=1.0, return_lse=True)
    assert_out_close(out, ref_o, torch.float32)
    assert_lse_close(lse, ref_l, torch.float32)


def test_value_dim_differs(cuda):
    attn, _, _ = _api()
    x = rand_inputs(1, 60, 4, 2, 64, dv=32, seed=8, dtype=torch.float32)
    out = attn(*(t.to(cuda) for t in x), 4, 20)
    ref = O.reference_simplicial(*x, 4, 20)
    assert_out_close(out, ref, torch.float32)


def test_mfma_matches_generic(cuda):
    attn, _, _ = _api()
    x = [t.to(cuda) for t in rand_inputs(2, 400, 8, 2, 128, seed=11)]
    a, la = attn(*x, 32, 128, scale=1.0, return_lse=True, kernel="mfma")
    b, lb = attn(*x, 32, 128, scale=1.0, return_lse=True, kernel="generic")
    assert_out_close(a, b, torch.bfloat16, atol=1e-2, rtol=2.0 ** -7)
    assert (la - lb).abs().max().item() < 1e-3


@pytest.mark.parametrize("seed", [0])
def test_c2_full_size_sampled(cuda, seed):
    """BASELINE config 2 at full size (B2 H16 S4096 D128, 512x32), window-edge positions."""
    pos = [0, 31, 32, 511, 512, 1000, 2047, 4095]
    _check(cuda, 2, 4096, 16, 16, 128, 32, 512, torch.bfloat16, seed=seed, positions=pos, kernel="mfma")


def test_ns_full_size_sampled(cuda):
    """The north-star shape (C2 at S=8192: B2 H16 D128, 512x32, the bench workload), window-edge positions."""
    pos = [0, 31, 32, 511, 512, 4095, 8191]
    _check(cuda, 2, 8192, 16, 16, 128, 32, 512, torch.bfloat16, seed=0, positions=pos, kernel="mfma")


def test_d256_config4_sampled_and_deterministic(cuda):
    """BASELINE config 4 shape family (D=256, w1=256, w2=64, sigma 0.5), shortened; bit-exact reruns."""
    attn, _, _ = _api()
    pos = [0, 63, 64, 255, 256, 1000, 2047]
    _check(cuda, 1, 2048, 8, 8, 256, 64, 256, torch.bfloat16, seed=4, sigma=0.5, positions=pos, kernel="mfma")
    x = [t.to(cuda) for t in rand_inputs(1, 2048, 8, 8, 256, seed=4, sigma=0.5)]
    runs = [attn(*x, 64, 256, scale=1.0, return_lse=True) for _ in range(3)]
    for o, l in runs[1:]:
        assert torch.equal(o, runs[0][0]) and torch.equal(l, runs[0][1])


def test_c4_full_workload_and_deterministic(cuda):
    """BASELINE config 4 at its real workload: B1 H8 S16384 D256, w1 (long) 256,
    w2 (short) 64, sigma 0.5, the bench generator.  Oracle parity at window-edge
    positions and three bit-identical full-size runs (deterministic mode on)."""
    from archlab_amd.workloads import C4, prefill_inputs
    attn, _, name = _api()
    x = prefill_inputs(C4)[:5]
    xd = [t.to(cuda) for t in x]
    prev = torch.are_deterministic_algorithms_enabled()
    torch.use_deterministic_algorithms(True)
    try:
        runs = [attn(*xd, C4.w2, C4.w1, scale=1.0, return_lse=True) for _ in range(3)]
    finally:
        torch.use_deterministic_algorithms(prev)
    torch.cuda.synchronize()
    for o, l in runs[1:]:
        assert torch.equal(o, runs[0][0]) and torch.equal(l, runs[0][1])
    assert name(x[0], x[1], x[3]) == "mfma"
    pos = [0, 63, 64, 255, 256, 8191, 16383]
    out, lse = runs[0][0][:, pos].cpu(), runs[0][1][:, pos].cpu()
    ref_o, ref_l = O.reference_simplicial(*(t.float() for t in x), C4.w2, C4.w1, scale=1.0, query_positions=pos,
                                          return_lse=True)
    ro, rl = O.kernel_rounding_reference(*x, C4.w2, C4.w1, scale=1.0, query_positions=pos)
    e1 = assert_out_close(out, ref_o, torch.bfloat16)
    e2 = assert_lse_close(lse[:, 1:], ref_l[:, 1:], torch.bfloat16)  # position 0 holds one pair
    assert_lse_close(lse, ref_l, torch.bfloat16, rtol=1e-2)
    assert_out_close(out, ro, torch.bfloat16, atol=4e-3, rtol=2.0 ** -7)
    assert_lse_close(lse, rl, torch.bfloat16, rtol=1e-4)
    print(f"C4 full: out {e1:.2e} lse {e2:.2e}", flush=True)


@pytest.mark.parametrize("dense", [True, False])
def test_windows_beyond_the_sequence_are_clipped_exactly(cuda, dense):
    """Windows >= the sequence length select every earlier key.  The library
    clips them by whole 32-key chunks, so a window that differs from another
    by a multiple of 32 gives bit-identical results; 2**32 + 100 (beyond int32)
    saturates to 2**31 - 1; every clipped window matches the oracle."""
    attn, varlen, _ = _api()
    x = [t.to(cuda) for t in rand_inputs(1, 300, 4, 2, 128, seed=13)]
    cu = torch.tensor([0, 120, 300], dtype=torch.int32, device=cuda)

    def run(ws, wl):
        if dense:
            return attn(*x, ws, wl, scale=1.0, return_lse=True)
        return varlen(*(t[0] for t in x), cu, ws, wl, scale=1.0, return_lse=True)
    base_o, base_l = run(32, 300)
    for wl in (300 + 32, 300 + 32 * 1000, 300 + 32 * (2 ** 25)):
        o, l = run(32, wl)
        assert torch.equal(o, base_o) and torch.equal(l, base_l), wl
    sat_o, sat_l = run(32, 2 ** 31 - 1)
    o, l = run(32, 2 ** 32 + 100)
    assert torch.equal(o, sat_o) and torch.equal(l, sat_l)
    full_o, full_l = run(2 ** 31 - 1, 2 ** 31 - 1)
    o, l = run(2 ** 32 + 100, 2 ** 32 + 100)
    assert torch.equal(o, full_o) and torch.equal(l, full_l)
    pos = [0, 150, 299] if dense else [0, 119, 120, 299]
    xs = [t.float().cpu() for t in x]
    if dense:
        ref_o, ref_l = O.reference_simplicial(*xs, 300, 300, scale=1.0, query_positions=pos, return_lse=True)
        got = [(full_o[0, pos], full_l[0, pos], ref_o[0], ref_l[0])]
        ref_s = O.reference_simplicial(*xs, 32, 300, scale=1.0, query_positions=pos)
        got_s = sat_o[0, pos]
    else:
        ref_o, ref_l = O.varlen_reference(*(t[0] for t in xs), cu.cpu(), 300, 300, scale=1.0,
                                          query_positions=pos, return_lse=True)
        got = [(full_o[pos], full_l[pos], ref_o, ref_l)]
        ref_s = O.varlen_reference(*(t[0] for t in xs), cu.cpu(), 32, 300, scale=1.0, query_positions=pos)
        got_s = sat_o[pos]
    for go, gl, ro, rl in got:
        assert_out_close(go, ro, torch.bfloat16)
        assert_lse_close(gl, rl, torch.bfloat16, rtol=1e-2)
    assert_out_close(got_s, ref_s, torch.bfloat16)


def test_deterministic_algorithms_allowed(cuda):
    attn, _, _ = _api()
    x = [t.to(cuda) for t in rand_inputs(1, 64, 2, 2, 64, seed=1)]
    prev = torch.are_deterministic_algorithms_enabled()
    torch.use_deterministic_algorithms(True)
    try:
        a = attn(*x, 4, 16)
        b = attn(*x, 4, 16)
    finally:
        torch.use_deterministic_algorithms(prev)
    assert torch.equal(a, b)


def test_noncontiguous_inputs(cuda):
    attn, _, _ = _api()
    x = [t.to(cuda) for t in rand_inputs(1, 96, 4, 2, 64, seed=9)]
    base = attn(*x, 8, 40)
    strided = [t.transpose(1, 2).contiguous().transpose(1, 2) for t in x]
    assert not strided[0].is_contiguous()
    assert torch.equal(attn(*strided, 8, 40), base)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_varlen_matches_per_sequence(cuda, dtype):
    attn, varlen, _ = _api()
    lengths = [1, 37, 300, 5, 129]
    t = sum(lengths)
    x = rand_inputs(1, t, 8, 2, 128 if dtype == torch.bfloat16 else 64, seed=21, dtype=dtype)
    packed = [v[0].to(cuda) for v in x]
    cu = torch.tensor([0] + list(np.cumsum(lengths)), dtype=torch.int32, device=cuda)
    out, lse = varlen(*packed, cu, 16, 64, scale=1.0, return_lse=True)
    start = 0
    for n in lengths:
        sl = slice(start, start + n)
        o, l = attn(*(p[None, sl] for p in packed), 16, 64, scale=1.0, return_lse=True)
        assert torch.equal(out[sl], o[0]), "varlen differs from the per-sequence dense call"
        assert torch.equal(lse[sl], l[0])
        start += n
    ref_o, ref_l = O.varlen_reference(*(v[0].float() for v in x), cu.cpu(), 16, 64, scale=1.0, return_lse=True)
    assert_out_close(out, ref_o, dtype)
    starts = np.repeat(np.cumsum([0] + lengths[:-1]), lengths)
    local = np.arange(t) - starts + 1
    full = torch.from_numpy(np.minimum(local, 16) * np.minimum(local, 64) >= 64)
    assert_lse_close(lse[full], ref_l[full], dtype)
    assert_lse_close(lse, ref_l, dtype, rtol=1e-2)


def test_c3_varlen_gqa_sampled(cuda):
    """BASELINE config 3 (T=32768 packed, 12 sequences, HQ32/HKV8, D128, 512x32) at sampled tokens."""
    from archlab_amd.workloads import C3, prefill_inputs
    _, varlen, _ = _api()
    q, k1, k2, v1, v2, cu = prefill_inputs(C3)
    out, lse = varlen(*(t.to(cuda) for t in (q, k1, k2, v1, v2)), cu.to(cuda), C3.w2, C3.w1, scale=1.0,
                      return_lse=True)
    cu_l = cu.tolist()
    pos = sorted({c for c in cu_l[:-1]} | {c + 31 for c in cu_l[:3]} | {c + 200 for c in cu_l[:4]} | {32767})
    ref_o, ref_l = O.varlen_reference(*(t.float() for t in (q, k1, k2, v1, v2)), cu, C3.w2, C3.w1, scale=1.0,
                                      query_positions=pos, return_lse=True)
    assert_out_close(out[pos], ref_o, torch.bfloat16)
    starts = {c for c in cu_l[:-1]}
    full = [i for i, p in enumerate(pos) if p not in starts]  # every sampled non-start token has >= 31 rows
    assert_lse_close(lse[pos][full], ref_l[full], torch.bfloat16)
    assert_lse_close(lse[pos], ref_l, torch.bfloat16, rtol=1e-2)


def test_contract_errors(cuda):
    attn, varlen, _ = _api()
    x = [t.to(cuda) for t in rand_inputs(1, 8, 4, 2, 64)]
    with pytest.raises(ValueError, match="short_window <= long_window"):
        attn(*x, 5, 4)
    with pytest.raises(ValueError, match="grouped-query"):
        attn(x[0][:, :, :3], *x[1:], 2, 4)
    with pytest.raises(ValueError, match="CUDA float32/bfloat16"):
        attn(*(t.half() for t in x), 2, 4)
    with pytest.raises(ValueError, match="finite real"):
        attn(*x, 2, 4, scale=float("nan"))
    # inputs that require grad take the autograd path (backward covered in test_backward_gpu)
    assert attn(x[0].float().requires_grad_(), *(t.float() for t in x[1:]), 2, 4).grad_fn is not None
    with pytest.raises(ValueError, match="MFMA kernel does not cover"):
        attn(*(t.float()[..., :32] for t in x), 2, 4, kernel="mfma")  # fp32 at D = 32


@pytest.mark.parametrize("d,dv", [(16, 16), (32, 32), (32, 64), (16, 128)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_narrow_widths_padded_onto_matrix_cores(cuda, d, dv, dtype):
    """Widths 16 and 32 run on the matrix cores zero-padded to 64 (or to the
    other width).  fp32: the oracle at 1e-4.  bf16: the oracle with the
    reference kernel's rounding point of a = bf16(q ⊙ k1) (simplicial_kernels.py:35)
    at LSE 1e-4 and out 4e-3 (+ one bf16 ulp), and the plain fp32 oracle at
    out 4e-2 / LSE 4e-3: with 16 or 32 terms per score that rounding moves
    the result further than at the BASELINE widths (64-256), the same for the
    reference kernel."""
    attn, varlen, name = _api()
    x = rand_inputs(1, 2, 4, 2, d, dv=dv, dtype=dtype)
    assert name(x[0], x[1], x[3]) == "mfma"
    if dtype == torch.float32:
        _check(cuda, 2, 120, 4, 2, d, 16, 48, dtype, seed=d + dv, dv=dv)
    else:
        x = rand_inputs(2, 120, 4, 2, d, dv=dv, seed=d + dv, dtype=dtype)
        out, lse = attn(*(t.to(cuda) for t in x), 16, 48, scale=1.0, return_lse=True)
        ro, rl = O.kernel_rounding_reference(*x, 16, 48, scale=1.0)
        fo, fl = O.reference_simplicial(*(t.float() for t in x), 16, 48, scale=1.0, return_lse=True)
        full = [p for p in range(120) if min(p + 1, 16) * min(p + 1, 48) >= 64]
        e1 = assert_out_close(out[:, full], ro[:, full], dtype, atol=4e-3, rtol=2.0 ** -7)
        e2 = assert_lse_close(lse, rl, dtype, rtol=1e-4)
        e3 = assert_out_close(out, fo, dtype, atol=4e-2)
        e4 = assert_lse_close(lse, fl, dtype, rtol=4e-3)
        print(f"[mfma padded] d{d} dv{dv} bf16: vs rounding oracle out {e1:.2e} lse {e2:.2e}; "
              f"vs fp32 oracle out {e3:.2e} lse {e4:.2e}", flush=True)
    lengths = [7, 60, 33]
    cu = torch.tensor([0, 7, 67, 100], dtype=torch.int32)
    xv = rand_inputs(1, sum(lengths), 4, 2, d, dv=dv, seed=d * dv, dtype=dtype)
    out, lse = varlen(*(v[0].to(cuda) for v in xv), cu.to(cuda), 8, 40, scale=1.0, return_lse=True)
    ref_o, ref_l = O.varlen_reference(*(v[0].float() for v in xv), cu, 8, 40, scale=1.0, return_lse=True)
    assert out.shape[-1] == dv
    assert_out_close(out, ref_o, dtype, atol=4e-2 if dtype == torch.bfloat16 else None)
    assert_lse_close(lse, ref_l, dtype, rtol=1e-2 if dtype == torch.bfloat16 else None)


def test_zz_report_few_pair_lse_error(cuda):
    """The measured maximum of the LSE error at positions whose windows hold
    fewer than 64 pairs (bound 1e-2 there, 1e-3 elsewhere), over every bf16
    check of this module that ran before this test."""
    if not _FEW_PAIR_LSE:
        pytest.skip("no bf16 check with few-pair positions ran in this session")
    worst, case = max(_FEW_PAIR_LSE)
    print(f"few-pair positions: max lse rel error {worst:.3e} (bound 1.0e-02) over {len(_FEW_PAIR_LSE)} checks; "
          f"worst in {case}", flush=True)
    assert worst <= 1e-2
