"""CPU checks of the host side: the C ABI library, its Python binding, the
reference-compatible argument contracts and the workload generators.  No
kernel is launched here."""

import ctypes
import os
import re
import subprocess

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "simplicial_mi355x.h")


def _declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(sa_[a-z_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    from archlab_amd import _native
    lib = _native.load()
    declared = _declared_functions()
    assert declared, "no declarations parsed"
    for name in declared:
        assert hasattr(lib, name), f"{name} declared in the header but not exported"
    assert set(declared) == set(_native.EXPORTS)
    out = subprocess.run(["nm", "-D", "--defined-only", _native.library_path()], capture_output=True, text=True)
    exported = {line.split()[-1] for line in out.stdout.splitlines() if " T " in line}
    # hidden visibility: the header's functions are the only exported code
    assert exported == set(declared), sorted(exported ^ set(declared))
    assert lib.sa_version().startswith(b"simplicial_mi355x")
    # the binding's struct layouts, the header and the library agree on the ABI version
    macro = int(re.search(r"#define SIMPLICIAL_MI355X_ABI_VERSION (\d+)", open(HEADER).read()).group(1))
    assert lib.sa_abi_version() == macro == _native.ABI_VERSION


def _c_layout(struct, fields):
    """sizeof / offsetof of a header struct, measured by the C compiler."""
    body = "\n".join(f'  printf("{f} %zu\\n", offsetof({struct}, {f}));' for f in fields)
    src = f"""#include <stdio.h>
#include <stddef.h>
#include "simplicial_mi355x.h"
int main(void) {{
  printf("sizeof %zu\\n", sizeof({struct}));
{body}
  return 0;
}}
"""
    import tempfile
    with tempfile.TemporaryDirectory() as tmp:
        c = os.path.join(tmp, "layout.c")
        exe = os.path.join(tmp, "layout")
        open(c, "w").write(src)
        subprocess.run(["gcc", "-std=c11", "-I", os.path.dirname(HEADER), c, "-o", exe], check=True)
        res = subprocess.run([exe], capture_output=True, text=True, check=True).stdout
    return {k: int(v) for k, v in (line.split() for line in res.splitlines())}


@pytest.mark.parametrize("cls,struct", [("PrefillArgs", "sa_prefill_args"), ("PagedArgs", "sa_paged_args"),
                                        ("PrefillBwdArgs", "sa_prefill_bwd_args")])
def test_python_binding_matches_c_struct_layout(cls, struct):
    from archlab_amd import _native
    py = getattr(_native, cls)
    fields = [f for f, _ in py._fields_]
    layout = _c_layout(struct, fields)
    assert layout["sizeof"] == ctypes.sizeof(py)
    for f in fields:
        assert layout[f] == getattr(py, f).offset, f


def test_c_abi_rejects_invalid_arguments_before_any_launch():
    from archlab_amd import _native
    lib = _native.load()
    args = _native.PrefillArgs(q=16, k1=16, k2=16, v1=16, v2=16, out=16, num_seqs=1, seqlen=4, total_tokens=4,
                               heads_q=4, heads_kv=2, head_dim=64, value_dim=64, short_window=5, long_window=4,
                               scale=1.0, dtype=_native.SA_DTYPE_BF16)
    assert lib.sa_prefill_fwd(ctypes.byref(args), None) == _native.SA_ERR_INVALID
    assert b"short_window" in lib.sa_last_error()
    args.short_window, args.heads_q = 2, 3
    assert lib.sa_prefill_fwd(ctypes.byref(args), None) == _native.SA_ERR_INVALID
    assert b"grouped-query" in lib.sa_last_error()
    args.heads_q, args.head_dim = 4, 48
    assert lib.sa_prefill_fwd(ctypes.byref(args), None) == _native.SA_ERR_INVALID
    assert lib.sa_prefill_kernel(ctypes.byref(args)) is None
    args.head_dim = 64
    assert lib.sa_prefill_kernel(ctypes.byref(args)) == b"mfma"
    args.dtype = _native.SA_DTYPE_F32
    assert lib.sa_prefill_kernel(ctypes.byref(args)) == b"generic"
    pargs = _native.PagedArgs(tokens=1, heads_q=4, heads_kv=3, head_dim=64, block_size=16, short_window=1,
                              long_window=2)
    assert lib.sa_paged_fwd(ctypes.byref(pargs), None, 0, None) == _native.SA_ERR_INVALID
    assert b"geometry" in lib.sa_last_error()


def _cpu_inputs(b=1, n=8, hq=4, hk=2, d=64):
    return [torch.zeros(b, n, h, d) for h in (hq, hk, hk, hk, hk)]


def test_prefill_contract_messages_match_reference():
    from archlab_amd import simplicial_attention
    x = _cpu_inputs()
    with pytest.raises(ValueError, match=r"expected \[batch, sequence, heads, head_dim\]"):
        simplicial_attention(x[0][0], *x[1:], 2, 4)
    with pytest.raises(ValueError, match="require 1 <= short_window <= long_window"):
        simplicial_attention(*x, 0, 4)
    with pytest.raises(ValueError, match="matching batch, sequence and heads"):
        simplicial_attention(x[0], x[1][:, :4], *x[2:], 2, 4)
    with pytest.raises(ValueError, match="incompatible grouped-query geometry"):
        simplicial_attention(x[0][:, :, :3], *x[1:], 2, 4)
    with pytest.raises(ValueError, match="same dtype and device"):
        simplicial_attention(x[0].double(), *x[1:], 2, 4)
    with pytest.raises(ValueError, match="finite real"):
        simplicial_attention(*x, 2, 4, scale=torch.tensor(1.0))
    with pytest.raises(ValueError, match="kernel supports CUDA float32/bfloat16"):
        simplicial_attention(*x, 2, 4)


def test_paged_contract_messages_match_reference():
    from archlab_amd import simplicial_paged_attention
    q = torch.zeros(3, 4, 64)
    cache = torch.zeros(2, 5, 16, 2, 64)
    table = torch.zeros(2, 3, dtype=torch.int32)
    seq = torch.zeros(3, dtype=torch.int32)
    kw = dict(short_window=2, long_window=4, scale=1.0)
    with pytest.raises(ValueError, match=r"expected q \[T,H,D\]"):
        simplicial_paged_attention(q[0], cache, cache, table, seq, seq, **kw)
    with pytest.raises(ValueError, match="incompatible paged simplicial geometry"):
        simplicial_paged_attention(q[:, :3], cache, cache, table, seq, seq, **kw)
    with pytest.raises(ValueError, match="require 1 <= short_window <= long_window"):
        simplicial_paged_attention(q, cache, cache, table, seq, seq, short_window=5, long_window=4, scale=1.0)
    with pytest.raises(ValueError, match="invalid paged simplicial inputs"):
        simplicial_paged_attention(q, cache, cache, table, seq, seq, **kw)  # CPU tensors


def test_token_layout_matches_oracle():
    from archlab_amd.serving import token_layout
    from oracle import simplicial_oracle as O
    starts = torch.tensor([0, 3, 4, 9, 9, 15], dtype=torch.int32)
    lens = torch.tensor([10, 1, 7, 5, 6], dtype=torch.int32)
    for tokens in (15, 9, 1):
        a = token_layout(starts, lens, tokens)
        b = O.token_layout(starts, lens, tokens)
        assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
        assert a[0].dtype == torch.int32 and a[1].dtype == torch.int32


def test_workload_definitions_match_baseline():
    from archlab_amd import workloads as W
    from oracle import simplicial_oracle as O
    assert W.prefill_flops(W.C2) == pytest.approx(1.0995e12, rel=1e-4)
    assert W.prefill_flops(W.NS) == pytest.approx(2.1990e12, rel=1e-4)
    assert W.prefill_flops(W.C4) == pytest.approx(2.1990e12, rel=1e-4)
    assert W.prefill_flops(W.C1) == pytest.approx(2.684e8, rel=1e-3)
    assert W.prefill_bytes(W.C2) == pytest.approx(201.9e6, rel=2e-3)
    lengths = W.varlen_lengths(32768, 12, 1)
    assert sum(lengths) == 32768 and len(lengths) <= 12
    cu = W.cu_from_lengths(lengths)
    assert cu.dtype == torch.int32 and int(cu[-1]) == 32768
    # the valid-pair fraction quoted for C2 (93.75%) follows from causal_triples
    full = W.C2.seqlen * W.C2.w1 * W.C2.w2
    assert O.causal_triples(W.C2.seqlen, W.C2.w2, W.C2.w1) / full == pytest.approx(0.9375, abs=2e-3)


def test_paged_workload_generator_small():
    from archlab_amd import workloads as W
    cfg = W.PagedConfig("tiny", 3, 4, 2, 64, 32, 8, 16, 20, 60, seed=3)
    inp = W.paged_inputs(cfg)
    t = inp["block_table"]
    assert t.dtype == torch.int32 and t.shape == (3, 4)
    assert int(t.min()) >= 1 and len(set(t.flatten().tolist())) == t.numel()  # distinct, null page unused
    assert inp["short_cache"].shape == (2, 13, 16, 2, 64)
    assert torch.equal(inp["token_pos"], (inp["ctx"] - 1).to(torch.int32))


def test_other_entry_point_contracts_on_cpu_tensors():
    """Checks that fire before any device work keep the reference's messages."""
    from archlab_amd import (deterministic_simplicial_attention, packed_simplicial_attention,
                             packed_simplicial_decode, simplicial_decode_attention, tilelang_attention,
                             tilelang_decode)
    q = torch.zeros(1, 1, 4, 128)
    k = torch.zeros(1, 8, 2, 128)
    with pytest.raises(ValueError, match="native packed decode requires CUDA FP32"):
        packed_simplicial_decode(q, k, k, k, k)
    with pytest.raises(ValueError, match="simplicial decode requires CUDA FP32 projections"):
        simplicial_decode_attention(q, k, k, k, k)
    with pytest.raises(ValueError, match="TileLang attention requires CUDA BF16 inputs"):
        tilelang_attention(q, k, k, scaling=1.0, long_window=4)
    with pytest.raises(ValueError, match="TileLang attention requires CUDA BF16 inputs"):
        tilelang_decode(q, k, k, scaling=1.0)
    x = torch.zeros(1, 8, 2, 128)
    with pytest.raises(ValueError, match="packed kernel requires CUDA"):
        packed_simplicial_attention(x, x, x, x, x, 2, 4)
    with pytest.raises(ValueError, match="require 1 <= short_window <= long_window"):
        packed_simplicial_attention(x, x, x, x, x, 5, 4)
    with pytest.raises(ValueError, match="deterministic simplicial core requires supported CUDA FP32 head geometry"):
        deterministic_simplicial_attention(x, x, x, x, x, 2, 4)


@pytest.mark.parametrize("d,width", [(3, 16), (8, 16), (64, 128), (128, 256), (256, 512)])
def test_determinant_operands_expand_to_the_determinant_sum(d, width):
    """The product's Sarrus expansion (pure tensor indexing) against the oracle's linalg.det."""
    from archlab_amd import determinant_operands
    g = torch.Generator().manual_seed(d)
    q, k1, k2 = (torch.randn(3, 5, d, generator=g, dtype=torch.float64) for _ in range(3))
    a, b, c = determinant_operands(q, k1, k2)
    assert a.shape[-1] == b.shape[-1] == c.shape[-1] == width
    used = d - d % 3
    chunks = [x[..., :used].reshape(3, 5, used // 3, 3) for x in (q, k1, k2)]
    expected = torch.linalg.det(torch.stack(chunks, dim=-2)).sum(-1)
    torch.testing.assert_close((a * b * c).sum(-1), expected, atol=1e-10, rtol=1e-10)
    assert not a[..., 2 * used:].count_nonzero() and not b[..., 2 * used:].count_nonzero()


def test_determinant_expansion_through_the_trilinear_oracle():
    """Expanded operands + the trilinear oracle == the determinant oracle (two independent paths)."""
    from archlab_amd import determinant_operands
    from oracle import simplicial_oracle as O
    g = torch.Generator().manual_seed(3)
    q = torch.randn(1, 6, 4, 8, generator=g, dtype=torch.float64)
    k1, k2 = (torch.randn(1, 6, 2, 8, generator=g, dtype=torch.float64) for _ in range(2))
    v1, v2 = (torch.randn(1, 6, 2, 5, generator=g, dtype=torch.float64) for _ in range(2))
    qs, k1s, k2s = determinant_operands(q, k1, k2)
    got = O.reference_simplicial(qs, k1s, k2s, v1, v2, 2, 4, scale=8 ** -0.5)
    torch.testing.assert_close(got, O.reference_determinant_simplicial(q, k1, k2, v1, v2, 2, 4),
                               atol=1e-12, rtol=1e-10)


def test_determinant_entry_point_contracts_on_cpu_tensors():
    from archlab_amd import (determinant_operands, determinant_simplicial_attention,
                             oriented_determinant_simplicial_attention)
    x = torch.zeros(1, 4, 2, 8)
    with pytest.raises(ValueError, match="at least 3 coordinates"):
        determinant_operands(x[..., :2], x[..., :2], x[..., :2])
    with pytest.raises(ValueError, match="matching score widths"):
        determinant_operands(x, x[..., :6], x)
    with pytest.raises(ValueError, match="positive integers"):
        oriented_determinant_simplicial_attention(x, x, x, x, x, 0, 2)
    with pytest.raises(ValueError, match="backend must be kernel or reference"):
        oriented_determinant_simplicial_attention(x, x, x, x, x, 1, 2, backend="triton")
    with pytest.raises(ValueError, match="not shipped"):
        oriented_determinant_simplicial_attention(x, x, x, x, x, 1, 2, backend="reference")
    with pytest.raises(ValueError, match="kernel supports CUDA"):
        determinant_simplicial_attention(x, x, x, x, x, 1, 2)


def _c5_plan_args(short_window, long_window, tokens=64, splits=0, table_width=512):
    """PagedArgs at BASELINE C5 geometry (HQ32/HKV8, D128, page 64) with aligned dummy pointers."""
    from archlab_amd import _native
    hk, d, bs, blocks = 8, 128, 64, 32769
    st = (blocks * bs * hk * d, bs * hk * d, hk * d, d)
    return _native.PagedArgs(
        q=256, q_stride_t=32 * d, q_stride_h=d, short_cache=256, sc_stride=(ctypes.c_int64 * 4)(*st),
        long_cache=256, lc_stride=(ctypes.c_int64 * 4)(*st), short_table=256, st_stride=table_width,
        long_table=256, lt_stride=table_width, token_seq=256, token_pos=256, out=256, o_stride_t=32 * d,
        o_stride_h=d, tokens=tokens, heads_q=32, heads_kv=hk, head_dim=d, block_size=bs, num_seqs=64,
        short_table_width=table_width, long_table_width=table_width, short_blocks=blocks, long_blocks=blocks,
        short_window=_native.window(short_window), long_window=_native.window(long_window), splits=splits,
        scale=1.0, q_dtype=_native.SA_DTYPE_BF16, cache_dtype=_native.SA_DTYPE_BF16,
        long_cache_dtype=_native.SA_DTYPE_BF16)


@pytest.mark.parametrize("long_window", [1 << 30, 2 ** 31 - 1, 2 ** 32 + 100])
@pytest.mark.parametrize("tokens", [1, 64, 2048])
def test_paged_plan_is_bounded_by_table_capacity_for_global_windows(long_window, tokens):
    """A global layer passes long_window = 1 << 30 (training/serving.py:49,80 in the
    reference).  The plan must depend on what the tables can address
    (512 pages x 64 = 32768 positions), never on the raw window: a few splits
    and a workspace of at most tens of MB."""
    from archlab_amd import _native
    lib = _native.load()
    args = _c5_plan_args(32, long_window, tokens=tokens)
    splits = lib.sa_paged_splits(ctypes.byref(args))
    ws = lib.sa_paged_workspace_bytes(ctypes.byref(args))
    cap_chunks = 512 * 64 // 32
    # grid of (token, KV group, split) workgroups: at most eight per CU (256 CUs
    # assumed without a GPU), or one split per 64 chunks of the capacity
    assert 1 <= splits <= max(8 * 256 // (tokens * 8), 1), splits
    assert splits <= cap_chunks // 2
    # partials: splits x tokens x 32 heads x (128 + 2) fp32
    assert ws <= splits * tokens * 32 * 130 * 4 + 3 * 256, ws
    assert ws <= 64 << 20, ws
    # a window of the capacity plus whole 32-key chunks plans the same launch
    same = _c5_plan_args(32, 512 * 64 + _native.window(long_window) % 32, tokens=tokens)
    assert lib.sa_paged_splits(ctypes.byref(same)) == splits
    assert lib.sa_paged_workspace_bytes(ctypes.byref(same)) == ws


def test_paged_plan_at_c5_is_one_direct_split():
    from archlab_amd import _native
    lib = _native.load()
    args = _c5_plan_args(32, 512)
    assert lib.sa_paged_splits(ctypes.byref(args)) == 1
    assert lib.sa_paged_workspace_bytes(ctypes.byref(args)) == 0
    assert lib.sa_paged_kernel(ctypes.byref(args)) == b"mfma"


def test_paged_plan_bounds_a_global_short_window():
    """Short windows are clipped the same way (row groups of 32 keys: one per
    pass, never ~33 million)."""
    from archlab_amd import _native
    lib = _native.load()
    args = _c5_plan_args(1 << 30, 1 << 30, tokens=4, table_width=8)  # 8 pages x 64 = 512 positions
    ws = lib.sa_paged_workspace_bytes(ctypes.byref(args))
    splits = lib.sa_paged_splits(ctypes.byref(args))
    assert splits >= 1
    # 512 positions -> 16 row groups per split at most
    assert ws <= splits * 16 * 4 * 32 * 130 * 4 + 3 * 256, ws


def test_window_lengths_beyond_int32_saturate():
    from archlab_amd import _native
    assert _native.window(2 ** 32 + 100) == 2 ** 31 - 1
    assert _native.window(1 << 30) == 1 << 30
    assert _native.window(7) == 7


def test_paged_accepts_the_reference_mixed_index_dtypes_before_launch():
    """The reference accepts int32/int64 tables and token arrays independently
    (simplicial_paged.py:88-94); only the device check may fail on CPU tensors."""
    from archlab_amd import simplicial_paged_attention
    q = torch.zeros(3, 4, 64)
    cache = torch.zeros(2, 5, 16, 2, 64)
    t32 = torch.zeros(2, 3, dtype=torch.int32)
    with pytest.raises(ValueError, match="invalid paged simplicial inputs"):  # CPU device, not the dtype mix
        simplicial_paged_attention(q, cache, cache.bfloat16(), t32, torch.zeros(3, dtype=torch.int32),
                                   torch.zeros(3, dtype=torch.int64), short_window=2, long_window=4, scale=1.0,
                                   long_block_table=t32.long())


@pytest.mark.parametrize("dtype,hq,hk,d,dv,ws,fused", [
    ("bf16", 4, 4, 128, 128, 32, True), ("bf16", 6, 2, 64, 64, 20, True), ("bf16", 8, 2, 128, 128, 32, True),
    ("bf16", 4, 2, 64, 64, 32, True), ("bf16", 4, 4, 128, 64, 32, True), ("bf16", 6, 2, 64, 128, 8, True),
    ("bf16", 4, 4, 128, 128, 40, True), ("f32", 4, 4, 64, 64, 32, True), ("f32", 6, 2, 128, 128, 20, True), ("bf16", 4, 4, 256, 128, 32, True),
    ("bf16", 8, 2, 256, 256, 16, True), ("bf16", 4, 4, 256, 64, 32, False), ("bf16", 4, 4, 256, 256, 40, True),
    ("bf16", 4, 2, 256, 128, 64, True), ("bf16", 4, 4, 256, 256, 65, False), ("bf16", 4, 2, 128, 64, 100, False),
    ("bf16", 4, 4, 64, 64, 128, False), ("bf16", 4, 4, 64, 64, 129, False), ("f32", 4, 4, 128, 128, 100, False),
    ("f32", 4, 4, 128, 128, 40, False), ("bf16", 3, 1, 64, 128, 64, True)])
def test_backward_workspace_reserves_dk1_partials_for_fused_shapes(dtype, hq, hk, d, dv, ws, fused):
    """The backward workspace holds delta and dlse rows ([tokens, hq] fp32 each,
    256-byte rounded) and, where dk1 comes from the dq pass (bf16, score width
    D and value width each 64 or 128, or D = 256 over values of 128 or 256,
    short window <= 64; fp32 with equal widths of 64 or 128, short window
    <= 32), the partials: 31 + NQ fp32 rows of D per dq workgroup of NQ
    queries x 4 / NQ heads (NQ = 4, 2, 1 for GQA groups that are odd, even,
    multiples of 4) and per 32-row group of short keys; fp32 calls the dv1
    partials as well (the same rows at the value width), while the two
    together stay within 8 GiB."""
    from archlab_amd import _native
    lib = _native.load()
    tokens = 1001
    fake = 1 << 20  # a 256-byte aligned non-null address: the size query reads no tensor
    fwd = _native.PrefillArgs(q=fake, k1=fake, k2=fake, v1=fake, v2=fake, out=fake, lse=fake,
                              q_stride_t=hq * d, q_stride_h=d, k_stride_t=hk * d, k_stride_h=d,
                              v_stride_t=hk * dv, v_stride_h=dv, o_stride_t=hq * dv, o_stride_h=dv, lse_stride_t=hq,
                              num_seqs=1, seqlen=tokens, total_tokens=tokens, heads_q=hq, heads_kv=hk,
                              head_dim=d, value_dim=dv, short_window=ws, long_window=512, scale=0.1,
                              dtype=_native.dtype_code(torch.bfloat16 if dtype == "bf16" else torch.float32))
    args = _native.PrefillBwdArgs(fwd=fwd)
    group = hq // hk
    nq = 1 if group % 4 == 0 else 2 if group % 2 == 0 else 4
    nr = -(-ws // 32)
    per_query = hq // (4 // nq) * nr * (31 + nq) * d * 4 / nq  # partial bytes per query
    rows = (tokens * hq * 4 + 255) // 256 * 256
    part = (-(-tokens // nq) * (hq // (4 // nq)) * nr * (31 + nq) * d * 4 + 255) // 256 * 256 if fused else 0
    # short windows of 65-128 at widths <= 128 (33-64 at score width 256): the
    # fp32 dk2 / dv2 sums of the first of two launches
    one = 32 if d == 256 else 64
    widths = (d in (64, 128) and dv in (64, 128)) or (d == 256 and dv in (128, 256))
    phased = dtype == "bf16" and widths and one < ws <= 2 * one
    dkv2 = (tokens * hk * (d + dv) * 4 + 255) // 256 * 256 if phased else 0
    # fp32 on the matrix cores (equal widths of 64 or 128, short window <= 32):
    # k2 and v2 as hi/lo bf16 rows, [tokens][hk][2 d] each
    f32_mfma = dtype == "f32" and d == dv and d in (64, 128) and ws <= 32
    split = 2 * ((tokens * hk * d * 4 + 255) // 256 * 256) if f32_mfma else 0
    walk = _walk_split_bytes(dtype, tokens, hk, d, dv, ws, 512)
    vpart = part // d * dv if fused and dtype == "f32" else 0  # dv1 partials (fp32)
    assert lib.sa_prefill_bwd_workspace_bytes(ctypes.byref(args)) == 2 * rows + part + dkv2 + split + walk + vpart
    if fused and dtype == "f32":
        # dk1 partials of ~6 GiB: both together would pass 8 GiB, so only dk1's are reserved
        mid = int((6 << 30) / per_query) // 4 * 4
        args.fwd.total_tokens = args.fwd.seqlen = mid
        rows_m = (mid * hq * 4 + 255) // 256 * 256
        part_m = (-(-mid // nq) * (hq // (4 // nq)) * nr * (31 + nq) * d * 4 + 255) // 256 * 256
        split_m = 2 * ((mid * hk * d * 4 + 255) // 256 * 256)
        assert lib.sa_prefill_bwd_workspace_bytes(ctypes.byref(args)) == 2 * rows_m + part_m + split_m
    if fused:
        # past 8 GiB of partials the separate dk1 pass runs: no partials reserved
        big = int((8 << 30) / per_query) // 4 * 4 + 8
        args.fwd.total_tokens = args.fwd.seqlen = big
        rows = (big * hq * 4 + 255) // 256 * 256
        split = 2 * ((big * hk * d * 4 + 255) // 256 * 256) if f32_mfma else 0
        dkv2_big = (big * hk * (d + dv) * 4 + 255) // 256 * 256 if phased else 0
        walk = _walk_split_bytes(dtype, big, hk, d, dv, ws, 512)
        assert lib.sa_prefill_bwd_workspace_bytes(ctypes.byref(args)) == 2 * rows + dkv2_big + split + walk
    # a caller short of memory selects the separate dk1 pass: no partials reserved
    args.fwd.total_tokens = args.fwd.seqlen = tokens
    args.fwd.flags = _native.SA_FLAG_SEPARATE_DK1
    rows = (tokens * hq * 4 + 255) // 256 * 256
    split = 2 * ((tokens * hk * d * 4 + 255) // 256 * 256) if f32_mfma else 0
    walk = _walk_split_bytes(dtype, tokens, hk, d, dv, ws, 512)
    assert lib.sa_prefill_bwd_workspace_bytes(ctypes.byref(args)) == 2 * rows + dkv2 + split + walk


def _dkv2_lds(d, dv, nr, nwk):
    rsa, rsb, rkv = 2 * d + 32, 2 * dv + 32, 2 * (d + dv)
    return 2 * nr * 32 * (rsa + rsb) + 64 * nr * rkv + 3 * -(-2 * rkv // 1024) * 1024 + nwk * 64 * 16


def _walk_split_bytes(dtype, tokens, hk, d, dv, ws, wl, cus=256):
    """Workspace of the dk2 / dv2 walk splits (bf16, widths 64 / 128, short
    window <= 64): when the (key block, KV head) workgroups -- 256 keys (8 waves)
    if both widths are 128 and they make at least 2 (one group of 32 short rows)
    or 1 (two groups) per CU, else 128 keys (4 waves) -- number fewer than the
    CUs' resident slots (two waves per SIMD, or what 160 KB of LDS holds), each
    walk over the queries is cut into pieces (up to 8, >= 128 queries each),
    whose fp32 sums take [splits][tokens][hk][max(d, dv)].  Without a GPU the
    library counts 256 CUs."""
    if dtype != "bf16" or d not in (64, 128) or dv not in (64, 128) or ws > 64:
        return 0
    nr = 1 if ws <= 32 else 2
    if d == dv == 128 and -(-tokens // 256) * hk >= (2 if nr == 1 else 1) * cus:
        return 0
    blocks = -(-tokens // 128) * hk
    per_cu = max(1, min(160 * 1024 // _dkv2_lds(d, dv, nr, 4), 2))
    splits = min(-(-cus * per_cu // blocks), 8, (128 + wl - 1) // 128)
    if splits <= 1:
        return 0
    return (splits * tokens * hk * max(d, dv) * 4 + 255) // 256 * 256
