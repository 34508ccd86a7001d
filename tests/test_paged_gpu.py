"""GPU parity of the paged (serving) kernels; restates the reference's paged
test plan (tests/test_simplicial_paged.py in the reference) plus the
BASELINE decode configuration.  Page-table handling is checked bit-exactly
(rtol = atol = 0) through invariants; values against the CPU oracle.
"""

import pytest
import torch

from helpers import assert_lse_close, assert_out_close, paged_batch
from oracle import simplicial_oracle as O

pytestmark = pytest.mark.gpu


def _paged():
    from archlab_amd.architectures.simplicial_paged import paged_plan, simplicial_paged_attention
    return simplicial_paged_attention, paged_plan


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 2e-4), (torch.bfloat16, 3e-2)])
@pytest.mark.parametrize("heads,kv_heads", [(4, 2), (10, 2), (8, 1)])
@pytest.mark.parametrize("short_window,long_window", [(16, 64), (16, 10_000), (4, 4)])
@pytest.mark.parametrize("hnd", [False, True])
def test_matches_oracle_for_prefill_and_decode_tokens(cuda, dtype, tol, heads, kv_heads, short_window,
                                                      long_window, hnd):
    paged, plan = _paged()
    dim, block_size, lengths = 64, 16, [1, 23, 140]
    (short, long), table, contiguous = paged_batch(lengths, kv_heads, dim, block_size, dtype, hnd, device=cuda)
    g = torch.Generator().manual_seed(1)
    seqs, positions, queries, expected = [], [], [], []
    for s, (n, (k1, k2, v1, v2)) in enumerate(zip(lengths, contiguous)):
        q = torch.randn(1, n, heads, dim, generator=g).to(dtype)
        oracle = O.reference_simplicial(q.double(), k1.double(), k2.double(), v1.double(), v2.double(),
                                        short_window, long_window)
        chosen = range(n) if s != 1 else [n - 1]  # sequence 1 is a decode step; others are prefills
        for position in chosen:
            seqs.append(s)
            positions.append(position)
            queries.append(q[0, position])
            expected.append(oracle[0, position])
    q = torch.stack(queries).to(cuda)
    seq = torch.tensor(seqs, dtype=torch.int32, device=cuda)
    pos = torch.tensor(positions, dtype=torch.int32, device=cuda)
    out = paged(q, short, long, table, seq, pos, short_window=short_window, long_window=long_window,
                scale=dim ** -0.5)
    torch.testing.assert_close(out.cpu(), torch.stack(expected).float(), rtol=tol, atol=tol)
    name = plan(q, short, long, table, seq, pos, short_window=short_window, long_window=long_window)[0]
    print(f"[{name}] {dtype} h{heads}/{kv_heads} w{short_window}x{long_window} hnd={hnd}", flush=True)


@pytest.mark.parametrize("dim", [128, 256])
@pytest.mark.parametrize("heads,kv_heads", [(4, 1), (4, 2), (4, 4)])
def test_head_dims_128_and_256(cuda, dim, heads, kv_heads):
    """bf16 MFMA paged kernels at the larger head dims (tasks of 1, 2 and 4 waves), prefill and decode tokens."""
    paged, plan = _paged()
    block_size, lengths, ws, wl = 16, [37, 90], 16, 48
    (short, long), table, contiguous = paged_batch(lengths, kv_heads, dim, block_size, torch.bfloat16, seed=5,
                                                   device=cuda)
    g = torch.Generator().manual_seed(6)
    seqs, positions, queries, expected = [], [], [], []
    for s, (n, (k1, k2, v1, v2)) in enumerate(zip(lengths, contiguous)):
        q = torch.randn(1, n, heads, dim, generator=g).to(torch.bfloat16)
        oracle = O.reference_simplicial(q.double(), k1.double(), k2.double(), v1.double(), v2.double(), ws, wl)
        for position in (range(n) if s == 0 else [n - 1]):
            seqs.append(s)
            positions.append(position)
            queries.append(q[0, position])
            expected.append(oracle[0, position])
    q = torch.stack(queries).to(cuda)
    seq = torch.tensor(seqs, dtype=torch.int32, device=cuda)
    pos = torch.tensor(positions, dtype=torch.int32, device=cuda)
    out = paged(q, short, long, table, seq, pos, short_window=ws, long_window=wl, scale=dim ** -0.5)
    name = plan(q, short, long, table, seq, pos, short_window=ws, long_window=wl)[0]
    err = (out.cpu() - torch.stack(expected).float()).abs().max().item()
    print(f"[{name}] bf16 d{dim} h{heads}/{kv_heads}: max-abs {err:.2e}", flush=True)
    assert name == "mfma"
    torch.testing.assert_close(out.cpu(), torch.stack(expected).float(), rtol=3e-2, atol=3e-2)


def test_token_order_and_batch_composition_do_not_change_results(cuda):
    paged, _ = _paged()
    dim, heads, kv_heads = 64, 4, 2
    for dtype in (torch.float32, torch.bfloat16):
        (short, long), table, _ = paged_batch([50, 70], kv_heads, dim, 16, dtype, seed=3, device=cuda)
        g = torch.Generator().manual_seed(4)
        q = torch.randn(120, heads, dim, generator=g).to(dtype).to(cuda)
        seq = torch.tensor([0] * 50 + [1] * 70, dtype=torch.int32, device=cuda)
        pos = torch.tensor(list(range(50)) + list(range(70)), dtype=torch.int32, device=cuda)
        kwargs = dict(short_window=16, long_window=33, scale=dim ** -0.5, splits=3)
        full = paged(q, short, long, table, seq, pos, **kwargs)
        order = torch.randperm(120, generator=g).to(cuda)
        shuffled = paged(q[order], short, long, table, seq[order], pos[order], **kwargs)
        torch.testing.assert_close(shuffled, full[order], rtol=0, atol=0)
        single = paged(q[60:61], short, long, table, seq[60:61], pos[60:61], **kwargs)
        torch.testing.assert_close(single, full[60:61], rtol=0, atol=0)


def test_graph_replay_matches_eager(cuda):
    paged, _ = _paged()
    dim, heads, kv_heads = 64, 4, 2
    (short, long), table, _ = paged_batch([40, 90], kv_heads, dim, 16, torch.bfloat16, seed=5, device=cuda)
    g = torch.Generator().manual_seed(6)
    q = torch.randn(2, heads, dim, generator=g).to(torch.bfloat16).to(cuda)
    seq = torch.tensor([0, 1], dtype=torch.int32, device=cuda)
    pos = torch.tensor([39, 89], dtype=torch.int32, device=cuda)
    kwargs = dict(short_window=16, long_window=64, scale=dim ** -0.5, splits=2)
    eager = paged(q, short, long, table, seq, pos, **kwargs)
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        paged(q, short, long, table, seq, pos, **kwargs)
    torch.cuda.current_stream().wait_stream(stream)
    with torch.cuda.graph(graph):
        captured = paged(q, short, long, table, seq, pos, **kwargs)
    torch.cuda.synchronize()
    for new_pos in ([20, 60], [39, 89], [5, 10]):
        pos.copy_(torch.tensor(new_pos, dtype=torch.int32, device=cuda))
        graph.replay()
        torch.cuda.synchronize()
        expected = paged(q, short, long, table, seq, pos, **kwargs)
        torch.cuda.synchronize()
        torch.testing.assert_close(captured, expected, rtol=0, atol=0)
    pos.copy_(torch.tensor([39, 89], dtype=torch.int32, device=cuda))
    graph.replay()
    torch.cuda.synchronize()
    torch.testing.assert_close(captured, eager, rtol=0, atol=0)


def test_separate_short_and_long_block_tables(cuda):
    paged, _ = _paged()
    dim, heads, kv_heads, lengths = 64, 4, 2, [30, 75]
    for dtype in (torch.float32, torch.bfloat16):
        (short, long), table, _ = paged_batch(lengths, kv_heads, dim, 16, dtype, seed=7, device=cuda)
        gen = torch.Generator().manual_seed(11)
        order = torch.randperm(long.shape[1] - 1, generator=gen) + 1
        remap = torch.zeros(long.shape[1], dtype=torch.long)
        remap[1:] = order
        moved = torch.zeros_like(long)
        moved[:, remap.to(cuda)] = long
        moved_table = remap.to(cuda)[table.long()].to(torch.int32)
        q = torch.randn(sum(lengths), heads, dim, generator=gen).to(dtype).to(cuda)
        seq = torch.tensor(sum(([s] * n for s, n in enumerate(lengths)), []), dtype=torch.int32, device=cuda)
        pos = torch.tensor(sum((list(range(n)) for n in lengths), []), dtype=torch.int32, device=cuda)
        kwargs = dict(short_window=16, long_window=40, scale=dim ** -0.5)
        shared = paged(q, short, long, table, seq, pos, **kwargs)
        separate = paged(q, short, moved, table, seq, pos, long_block_table=moved_table, **kwargs)
        torch.testing.assert_close(separate, shared, rtol=0, atol=0)


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 2e-5), (torch.bfloat16, 2e-2)])
def test_long_axis_splits_agree(cuda, dtype, tol):
    paged, _ = _paged()
    dim, heads, kv_heads, lengths = 64, 8, 2, [300, 37]
    (short, long), table, _ = paged_batch(lengths, kv_heads, dim, 16, dtype, seed=13, device=cuda)
    g = torch.Generator().manual_seed(14)
    q = torch.randn(2, heads, dim, generator=g).to(dtype).to(cuda)
    seq = torch.tensor([0, 1], dtype=torch.int32, device=cuda)
    pos = torch.tensor([299, 36], dtype=torch.int32, device=cuda)
    kwargs = dict(short_window=16, long_window=10_000, scale=dim ** -0.5)
    one = paged(q, short, long, table, seq, pos, splits=1, **kwargs)
    for splits in (2, 7, 19, None):
        many = paged(q, short, long, table, seq, pos, splits=splits, **kwargs)
        torch.testing.assert_close(many, one, rtol=tol, atol=tol)


def test_block_offsets_beyond_int32_elements(cuda):
    """Caches larger than 2**31 elements: block * block_stride must not overflow."""
    paged, _ = _paged()
    dim, heads, kv_heads, block_size, lengths = 64, 4, 1, 16, [40, 70]
    (short, long), table, _ = paged_batch(lengths, kv_heads, dim, block_size, torch.bfloat16, seed=3, device=cuda)
    g = torch.Generator().manual_seed(15)
    q = torch.randn(sum(lengths), heads, dim, generator=g).to(torch.bfloat16).to(cuda)
    seq = torch.tensor(sum(([s] * n for s, n in enumerate(lengths)), []), dtype=torch.int32, device=cuda)
    pos = torch.tensor(sum((list(range(n)) for n in lengths), []), dtype=torch.int32, device=cuda)
    kwargs = dict(short_window=16, long_window=60, scale=dim ** -0.5)
    expected = paged(q, short, long, table, seq, pos, **kwargs)
    shift = 2 ** 31 // (block_size * kv_heads * dim) + 7  # first moved block's offset exceeds int32
    big = []
    for cache in (short, long):
        moved = torch.zeros((2, shift + cache.shape[1], block_size, kv_heads, dim), dtype=cache.dtype, device=cuda)
        moved[:, shift:] = cache
        big.append(moved)
    moved_table = torch.where(table > 0, table + shift, table)
    out = paged(q, big[0], big[1], moved_table, seq, pos, **kwargs)
    torch.testing.assert_close(out, expected, rtol=0, atol=0)
    del big


def test_int64_metadata_and_lse(cuda):
    paged, _ = _paged()
    dim, heads, kv_heads, lengths = 128, 8, 2, [100, 33]
    (short, long), table, dense = paged_batch(lengths, kv_heads, dim, 16, torch.bfloat16, seed=17, device=cuda)
    g = torch.Generator().manual_seed(18)
    q = (torch.randn(2, heads, dim, generator=g) / dim ** 0.5).to(torch.bfloat16)
    seq = torch.tensor([0, 1], dtype=torch.int32)
    pos = torch.tensor([99, 32], dtype=torch.int32)
    kwargs = dict(short_window=32, long_window=64, scale=1.0)
    a, la = paged(q.to(cuda), short, long, table, seq.to(cuda), pos.to(cuda), return_lse=True, **kwargs)
    b, lb = paged(q.to(cuda), short, long, table.long(), seq.long().to(cuda), pos.long().to(cuda),
                  return_lse=True, **kwargs)
    torch.testing.assert_close(a, b, rtol=0, atol=0)
    torch.testing.assert_close(la, lb, rtol=0, atol=0)
    for t, (s, p) in enumerate(zip(seq.tolist(), pos.tolist())):
        k1, k2, v1, v2 = (x.float() for x in dense[s])
        qq = torch.zeros(1, p + 1, heads, dim)
        qq[0, p] = q[t].float()
        ro, rl = O.reference_simplicial(qq, k1[:, :p + 1], k2[:, :p + 1], v1[:, :p + 1], v2[:, :p + 1], 32, 64,
                                        scale=1.0, query_positions=[p], return_lse=True)
        assert_out_close(a[t], ro[0, 0], torch.bfloat16)
        assert_lse_close(la[t], rl[0, 0], torch.bfloat16)


def test_c5_decode_config(cuda):
    """64 sequences, HQ32/HKV8, D128, w1=512 (long) w2=32 (short), page 64.

    Every one of the 64 tokens is checked against the paged oracle; two calls
    with the same split count are bit-identical."""
    from archlab_amd.workloads import C5, paged_inputs
    paged, plan = _paged()
    inp = paged_inputs(C5, device=cuda)
    args = (inp["q"], inp["short_cache"], inp["long_cache"], inp["block_table"], inp["token_seq"], inp["token_pos"])
    kw = dict(short_window=C5.w2, long_window=C5.w1, scale=1.0)
    out, lse = paged(*args, return_lse=True, **kw)
    again, lse2 = paged(*args, return_lse=True, **kw)
    assert torch.equal(out, again) and torch.equal(lse, lse2)
    name, splits, _ = plan(*args, **kw)
    assert name == "mfma"
    sub = [inp[k] for k in ("short_cache", "long_cache")]
    ref_o, ref_l = O.paged_reference(inp["q"].cpu(), _gather_only(sub[0]), _gather_only(sub[1]),
                                     inp["block_table"].cpu(), inp["token_seq"].cpu(), inp["token_pos"].cpu(),
                                     short_window=C5.w2, long_window=C5.w1, scale=1.0, return_lse=True)
    err = assert_out_close(out, ref_o, torch.bfloat16)
    rel = assert_lse_close(lse, ref_l, torch.bfloat16)
    print(f"[{name}] C5 splits={splits}: all 64 tokens, out max-abs {err:.2e}, lse rel {rel:.2e}", flush=True)


def test_physical_page_placement_is_bit_exact(cuda):
    """Page-table handling is bit-exact: the same logical rows placed in
    contiguous pages (identity table) or scattered over a shuffled pool give
    identical bits, on both kernels, with one table or a table per axis."""
    paged, plan = _paged()
    dim, heads, kv_heads, bs, lengths = 128, 8, 2, 16, [70, 129, 33]
    for qdtype, cdtype in ((torch.bfloat16, torch.bfloat16), (torch.float32, torch.bfloat16),
                           (torch.float32, torch.float32)):
        (short, long), table, _ = paged_batch(lengths, kv_heads, dim, bs, cdtype, seed=31, device=cuda)
        # the same logical rows in identity order: page i of sequence s at 1 + sum(pages before s) + i
        ident = torch.zeros_like(table)
        nxt = 1
        for s, n in enumerate(lengths):
            pages = -(-n // bs)
            ident[s, :pages] = torch.arange(nxt, nxt + pages, dtype=table.dtype, device=cuda)
            nxt += pages
        flat_short, flat_long = torch.zeros_like(short), torch.zeros_like(long)
        for s, n in enumerate(lengths):
            pages = -(-n // bs)
            for src, dst in ((short, flat_short), (long, flat_long)):
                dst[:, ident[s, :pages].long()] = src[:, table[s, :pages].long()]
        g = torch.Generator().manual_seed(32)
        tokens = [(0, 69), (1, 128), (2, 32), (1, 5), (0, 0)]
        q = torch.randn(len(tokens), heads, dim, generator=g).to(qdtype).to(cuda)
        seq = torch.tensor([t[0] for t in tokens], dtype=torch.int32, device=cuda)
        pos = torch.tensor([t[1] for t in tokens], dtype=torch.int32, device=cuda)
        kw = dict(short_window=24, long_window=100, scale=dim ** -0.5, return_lse=True)
        o1, l1 = paged(q, short, long, table, seq, pos, **kw)
        o2, l2 = paged(q, flat_short, flat_long, ident, seq, pos, **kw)
        o3, l3 = paged(q, flat_short, long, ident, seq, pos, long_block_table=table, **kw)
        assert torch.equal(o1, o2) and torch.equal(l1, l2)
        assert torch.equal(o1, o3) and torch.equal(l1, l3)
        name = plan(q, short, long, table, seq, pos, short_window=24, long_window=100)[0]
        print(f"[{name}] q {qdtype} caches {cdtype}: placement-invariant", flush=True)


class _gather_only:
    """Lazy CPU view of a device cache: paged_gather indexes [kv, blocks, offsets]."""

    def __init__(self, cache):
        self.cache = cache
        self.shape = cache.shape

    def __getitem__(self, idx):
        kv, blocks, offs = idx
        return self.cache[kv, blocks.to(self.cache.device), offs.to(self.cache.device)].cpu()


def test_contract_errors(cuda):
    paged, _ = _paged()
    (short, long), table, _ = paged_batch([20], 2, 64, 16, torch.float32, seed=1, device=cuda)
    q = torch.randn(1, 4, 64, device=cuda)
    seq = torch.zeros(1, dtype=torch.int32, device=cuda)
    pos = torch.zeros(1, dtype=torch.int32, device=cuda)
    with pytest.raises(ValueError, match="short_window <= long_window"):
        paged(q, short, long, table, seq, pos, short_window=8, long_window=4, scale=1.0)
    with pytest.raises(ValueError, match="geometry"):
        paged(q[:, :3], short, long, table, seq, pos, short_window=2, long_window=4, scale=1.0)
    with pytest.raises(ValueError, match="invalid paged"):
        paged(q, short, long, table.float(), seq, pos, short_window=2, long_window=4, scale=1.0)
    with pytest.raises(ValueError, match="contiguous"):
        paged(q.transpose(1, 2).contiguous().transpose(1, 2), short, long, table, seq, pos, short_window=2,
              long_window=4, scale=1.0)
    empty = paged(q[:0], short, long, table, seq[:0], pos[:0], short_window=2, long_window=4, scale=1.0)
    assert empty.shape == (0, 4, 64) and empty.dtype == torch.float32


def test_global_window_at_c5_geometry(cuda):
    """The reference serves global layers with long_window = 1 << 30
    (training/serving.py:49,80).  At C5 geometry (contexts up to 32768) the
    plan stays bounded, the result equals the one for a window of exactly the
    table capacity bit for bit (every window beyond it selects the same keys),
    and matches the oracle on sampled tokens."""
    from archlab_amd.workloads import C5, paged_inputs
    paged, plan = _paged()
    inp = paged_inputs(C5, device=cuda)
    args = (inp["q"], inp["short_cache"], inp["long_cache"], inp["block_table"], inp["token_seq"], inp["token_pos"])
    capacity = inp["block_table"].shape[1] * C5.page
    kw = dict(short_window=C5.w2, scale=1.0)
    name, splits, ws = plan(*args, long_window=1 << 30, **kw)
    print(f"[{name}] global window: splits={splits} workspace={ws} B", flush=True)
    assert name == "mfma" and ws <= 64 << 20
    out, lse = paged(*args, long_window=1 << 30, return_lse=True, **kw)
    o2, l2 = paged(*args, long_window=capacity, return_lse=True, **kw)  # same window mod 32: same chunks
    assert torch.equal(o2, out) and torch.equal(l2, lse)
    sat, sat_l = paged(*args, long_window=2 ** 31 - 1, return_lse=True, **kw)
    o3, l3 = paged(*args, long_window=2 ** 32 + 100, return_lse=True, **kw)  # saturates to 2**31 - 1
    assert torch.equal(o3, sat) and torch.equal(l3, sat_l)
    assert_out_close(sat, out, torch.bfloat16)
    pick = [int(torch.argmin(inp["ctx"])), 5, int(torch.argmax(inp["ctx"]))]
    sub = [inp[k] for k in ("short_cache", "long_cache")]
    ref_o, ref_l = O.paged_reference(inp["q"][pick].cpu(), _gather_only(sub[0]), _gather_only(sub[1]),
                                     inp["block_table"].cpu(), inp["token_seq"][pick].cpu(),
                                     inp["token_pos"][pick].cpu(), short_window=C5.w2, long_window=capacity,
                                     scale=1.0, return_lse=True)
    assert_out_close(out[pick], ref_o, torch.bfloat16)
    assert_lse_close(lse[pick], ref_l, torch.bfloat16)


@pytest.mark.parametrize("heads,kv_heads", [(8, 2), (2, 2)])
@pytest.mark.parametrize("splits", [1, 3, None])
def test_split_longer_than_one_offset_segment(cuda, heads, kv_heads, splits):
    """A split whose long window spans more than 1024 positions walks its chunks
    in segments of cached row offsets (4 and 1 waves per workgroup)."""
    paged, plan = _paged()
    dim, lengths, ws, wl = 128, [2600, 1500], 32, 2400
    (short, long), table, dense = paged_batch(lengths, kv_heads, dim, 16, torch.bfloat16, seed=21, device=cuda)
    g = torch.Generator().manual_seed(22)
    q = (torch.randn(4, heads, dim, generator=g) / dim ** 0.5).to(torch.bfloat16)
    seq = torch.tensor([0, 0, 1, 1], dtype=torch.int32)
    pos = torch.tensor([2599, 1100, 1499, 40], dtype=torch.int32)
    out, lse = paged(q.to(cuda), short, long, table, seq.to(cuda), pos.to(cuda), short_window=ws, long_window=wl,
                     scale=1.0, splits=splits, return_lse=True)
    name, used, _ = plan(q.to(cuda), short, long, table, seq.to(cuda), pos.to(cuda), short_window=ws,
                         long_window=wl, splits=splits)
    assert name == "mfma"
    print(f"h{heads}/{kv_heads} splits={used}", flush=True)
    for t, (s, p) in enumerate(zip(seq.tolist(), pos.tolist())):
        k1, k2, v1, v2 = (x.float() for x in dense[s])
        qq = torch.zeros(1, p + 1, heads, dim)
        qq[0, p] = q[t].float()
        ro, rl = O.reference_simplicial(qq, k1[:, :p + 1], k2[:, :p + 1], v1[:, :p + 1], v2[:, :p + 1], ws, wl,
                                        scale=1.0, query_positions=[p], return_lse=True)
        assert_out_close(out[t], ro[0, 0], torch.bfloat16)
        assert_lse_close(lse[t], rl[0, 0], torch.bfloat16)


def test_mixed_index_and_cache_dtypes(cuda):
    """int32 and int64 tables / token arrays mix freely, as the reference
    accepts them (simplicial_paged.py:88-94); fp32 and bf16 caches mix on the
    portable kernel.  Index handling is bit-exact."""
    paged, plan = _paged()
    dim, heads, kv_heads, lengths = 64, 4, 2, [60, 33]
    (short, long), table, _ = paged_batch(lengths, kv_heads, dim, 16, torch.bfloat16, seed=23, device=cuda)
    g = torch.Generator().manual_seed(24)
    q = torch.randn(3, heads, dim, generator=g).to(torch.bfloat16).to(cuda)
    seq = torch.tensor([0, 1, 0], dtype=torch.int32, device=cuda)
    pos = torch.tensor([59, 32, 7], dtype=torch.int32, device=cuda)
    kw = dict(short_window=8, long_window=40, scale=dim ** -0.5)
    base = paged(q, short, long, table, seq, pos, **kw)
    for lt, sq, ps in ((table.long(), seq, pos), (table, seq.long(), pos), (table, seq, pos.long()),
                       (table.long(), seq.long(), pos)):
        mixed = paged(q, short, long, table, sq, ps, long_block_table=lt, **kw)
        torch.testing.assert_close(mixed, base, rtol=0, atol=0)
    # mixed cache dtypes: the generic kernel against its own all-fp32 result on the same values
    ref = paged(q.float(), short.float(), long.float(), table, seq, pos, **kw)
    mix = paged(q.float(), short, long.float(), table, seq, pos, **kw)
    torch.testing.assert_close(mix, ref, rtol=0, atol=0)
    assert plan(q.float(), short, long.float(), table, seq, pos, **kw)[0] == "generic"


@pytest.mark.parametrize("qdtype,tol", [(torch.bfloat16, 3e-2), (torch.float32, 2e-4)])
@pytest.mark.parametrize("short_dtype,long_dtype", [(torch.float16, torch.float16), (torch.float16, torch.bfloat16),
                                                    (torch.bfloat16, torch.float16), (torch.float32, torch.float16)])
def test_fp16_caches(cuda, qdtype, tol, short_dtype, long_dtype):
    """fp16 short and long caches, alone or mixed with bf16 / fp32 ones, as the
    reference's paged loads accept them (simplicial_paged.py:42-52): against
    the paged oracle on the cache values (bf16 query: the reference rounds
    q ⊙ k1, k2 and v2 to bf16, within the bf16 tolerance; fp32 query: 2e-4)."""
    paged, plan = _paged()
    dim, heads, kv_heads, bs, lengths = 64, 8, 2, 16, [23, 70]
    (short, long), table, _ = paged_batch(lengths, kv_heads, dim, bs, torch.float32, seed=41, device="cpu")
    short, long = short.to(short_dtype), long.to(long_dtype)
    g = torch.Generator().manual_seed(42)
    tokens = [(0, 22), (1, 69), (1, 40), (0, 3), (1, 0)]
    q = (torch.randn(len(tokens), heads, dim, generator=g) * dim ** -0.5).to(qdtype)
    seq = torch.tensor([t[0] for t in tokens], dtype=torch.int32)
    pos = torch.tensor([t[1] for t in tokens], dtype=torch.int32)
    kw = dict(short_window=8, long_window=40, scale=1.0)
    out, lse = paged(q.to(cuda), short.to(cuda), long.to(cuda), table.to(cuda), seq.to(cuda), pos.to(cuda),
                     return_lse=True, **kw)
    ref_o, ref_l = O.paged_reference(q.float(), short.float(), long.float(), table, seq, pos, return_lse=True, **kw)
    err = (out.cpu() - ref_o).abs().max().item()
    torch.testing.assert_close(out.cpu(), ref_o, rtol=tol, atol=tol)
    torch.testing.assert_close(lse.cpu(), ref_l, rtol=tol, atol=tol)
    name = plan(q.to(cuda), short.to(cuda), long.to(cuda), table.to(cuda), seq.to(cuda), pos.to(cuda),
                short_window=8, long_window=40)[0]
    print(f"[{name}] q {qdtype} short {short_dtype} long {long_dtype}: max-abs {err:.2e}", flush=True)
    assert name == "generic"


@pytest.mark.parametrize("dim", [64, 128])
@pytest.mark.parametrize("heads,kv_heads", [(4, 2), (10, 2), (8, 1), (32, 8)])
@pytest.mark.parametrize("short_window,long_window", [(16, 64), (16, 10_000), (32, 512), (4, 4)])
def test_fp32_query_over_bf16_caches_on_matrix_cores(cuda, dim, heads, kv_heads, short_window, long_window):
    """The reference's serving caller passes an fp32 query with bf16 caches
    (serving.py:83) and its kernel keeps a = q ⊙ k1 and P in fp32
    (simplicial_paged.py:45, :60).  The MFMA kernel carries both as hi/lo
    bf16 terms; parity at the reference's fp32 tolerance (2e-4,
    tests/test_simplicial_paged.py:37) against the float64 oracle."""
    paged, plan = _paged()
    block_size, lengths = 16, [1, 23, 140, 700]
    (short, long), table, contiguous = paged_batch(lengths, kv_heads, dim, block_size, torch.bfloat16, seed=dim,
                                                   device=cuda)
    g = torch.Generator().manual_seed(heads)
    seqs, positions, queries, expected = [], [], [], []
    for s, (n, (k1, k2, v1, v2)) in enumerate(zip(lengths, contiguous)):
        q = torch.randn(1, n, heads, dim, generator=g)  # fp32, not bf16-representable
        chosen = list(range(n)) if n < 200 else [0, 31, 32, 511, 512, n - 1]
        oracle = O.reference_simplicial(q.double(), k1.double(), k2.double(), v1.double(), v2.double(),
                                        short_window, long_window, query_positions=chosen, scale=dim ** -0.5)
        for i, position in enumerate(chosen):
            seqs.append(s)
            positions.append(position)
            queries.append(q[0, position])
            expected.append(oracle[0, i])
    q = torch.stack(queries).to(cuda)
    seq = torch.tensor(seqs, dtype=torch.int32, device=cuda)
    pos = torch.tensor(positions, dtype=torch.int32, device=cuda)
    kw = dict(short_window=short_window, long_window=long_window, scale=dim ** -0.5)
    name = plan(q, short, long, table, seq, pos, **kw)[0]
    assert name == "mfma"
    out = paged(q, short, long, table, seq, pos, **kw)
    ref = torch.stack(expected).float()
    err = (out.cpu() - ref).abs().max().item()
    gen = paged(q, short, long, table, seq, pos, kernel="generic", **kw)
    print(f"[{name}] fp32 q d{dim} h{heads}/{kv_heads} w{short_window}x{long_window}: max-abs {err:.2e} "
          f"(generic {(gen.cpu() - ref).abs().max().item():.2e})", flush=True)
    torch.testing.assert_close(out.cpu(), ref, rtol=2e-4, atol=2e-4)


def test_fp32_query_c5_decode(cuda):
    """C5 with the fp32 query the serving caller sends, on the MFMA kernel, at
    the fp32 tolerance against the float64 oracle on sampled tokens."""
    from archlab_amd.workloads import C5, paged_inputs
    paged, plan = _paged()
    inp = paged_inputs(C5, device=cuda)
    g = torch.Generator().manual_seed(3)
    qf = (torch.randn(inp["q"].shape, generator=g) / C5.dim ** 0.5).to(cuda)
    args = (qf, inp["short_cache"], inp["long_cache"], inp["block_table"], inp["token_seq"], inp["token_pos"])
    kw = dict(short_window=C5.w2, long_window=C5.w1, scale=1.0)
    assert plan(*args, **kw)[0] == "mfma"
    out, lse = paged(*args, return_lse=True, **kw)
    again, lse2 = paged(*args, return_lse=True, **kw)
    assert torch.equal(out, again) and torch.equal(lse, lse2)
    pick = [0, 9, 33, 63]
    sub = [inp[k] for k in ("short_cache", "long_cache")]
    ref_o, ref_l = O.paged_reference(qf[pick].cpu().double(), _gather_only(sub[0]), _gather_only(sub[1]),
                                     inp["block_table"].cpu(), inp["token_seq"][pick].cpu(),
                                     inp["token_pos"][pick].cpu(), short_window=C5.w2, long_window=C5.w1,
                                     scale=1.0, return_lse=True)
    torch.testing.assert_close(out[pick].cpu(), ref_o.float(), rtol=2e-4, atol=2e-4)
    torch.testing.assert_close(lse[pick].cpu(), ref_l.float(), rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("dim,ws,qdtype", [(128, 48, torch.bfloat16), (64, 80, torch.bfloat16),
                                           (128, 48, torch.float32)])
@pytest.mark.parametrize("heads,kv_heads", [(4, 1), (8, 2)])
def test_short_windows_of_several_row_groups(cuda, dim, ws, qdtype, heads, kv_heads):
    """Short windows beyond 32 keys (two or three 32-row groups per token: the
    workgroup's waves hold different groups, each loading its own short rows),
    prefill and decode tokens, bf16 caches with a bf16 or fp32 query."""
    paged, plan = _paged()
    block_size, lengths, wl = 16, [70, 130], 100
    (short, long), table, contiguous = paged_batch(lengths, kv_heads, dim, block_size, torch.bfloat16, seed=9,
                                                   device=cuda)
    g = torch.Generator().manual_seed(10)
    seqs, positions, queries, expected = [], [], [], []
    for s, (n, (k1, k2, v1, v2)) in enumerate(zip(lengths, contiguous)):
        q = torch.randn(1, n, heads, dim, generator=g).to(qdtype)
        oracle = O.reference_simplicial(q.double(), k1.double(), k2.double(), v1.double(), v2.double(), ws, wl)
        for position in (range(n) if s == 0 else [n - 1]):
            seqs.append(s)
            positions.append(position)
            queries.append(q[0, position])
            expected.append(oracle[0, position])
    q = torch.stack(queries).to(cuda)
    seq = torch.tensor(seqs, dtype=torch.int32, device=cuda)
    pos = torch.tensor(positions, dtype=torch.int32, device=cuda)
    out = paged(q, short, long, table, seq, pos, short_window=ws, long_window=wl, scale=dim ** -0.5)
    name = plan(q, short, long, table, seq, pos, short_window=ws, long_window=wl)[0]
    err = (out.cpu() - torch.stack(expected).float()).abs().max().item()
    print(f"[{name}] {qdtype} d{dim} h{heads}/{kv_heads} w{ws}x{wl}: max-abs {err:.2e}", flush=True)
    assert name == "mfma"
    tol = 3e-2 if qdtype == torch.bfloat16 else 2e-4
    torch.testing.assert_close(out.cpu(), torch.stack(expected).float(), rtol=tol, atol=tol)
