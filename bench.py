#!/usr/bin/env python3
"""Benchmark of the 2-simplicial attention hot path on one MI355X.

Prints ONE JSON line.  Headline (``value``): bf16 2-simplicial prefill
forward throughput in TFLOP/s on the north-star shape (B=2, H=16, S=8192,
D=128, long window w1=512, short window w2=32), effective FLOPs
4*B*H*S*w1*w2*D, with inputs resident in HBM.  The same line carries:
  * ``configs``: the other BASELINE prefill configurations C2, C3 (packed
    varlen + GQA) and C4 (D=256), each with its roofline and CPU baseline;
  * ``decode``: the paged decode of BASELINE config C5 (tok/s, HBM GB/s);
  * ``fp32``: the fp32 inputs the reference's callers send -- paged decode
    with an fp32 query over bf16 caches (serving.py:83) at C5, fp32 prefill
    at C2 geometry (deepseek_v41_adapter.py:138-144), and C1 in full;
  * ``backward``: forward + backward through autograd on the headline shape
    (and on the ``--bwd-configs`` workloads, C3 and C4 by default, in
    ``"backward_configs"``);
  * ``roofline`` of the dominant kernel and ``cpu_baseline`` (the oracle
    timed on this host's cores on a bounded sample of the same workload);
  * beside every nominal prefill figure, ``valid_pair_flops`` and
    ``valid_pair_tflops``: the FLOPs of the (short key, long key) pairs the
    queries can actually see (windows cut at sequence starts), counted in
    closed form as the reference's cost ledger does (limite_cost.py:31-45, :69-73);
  * ``copy_calibration``: a 1 GiB device copy, this GPU's achievable HBM
    rate, also set beside the decode rate (``decode.achievable_copy_gbs``).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
                       [--legs prefill,configs,decode,global,fp32,backward,det,copy,cpu]
"""

from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "next-gen-arch_amd"))

PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0      # MI355X HBM3E


def _args():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--decode-steps", type=int, default=200)
    ap.add_argument("--bwd-steps", type=int, default=10)
    ap.add_argument("--bwd-configs", default="C3,C4", help="further workloads of the backward leg")
    ap.add_argument("--legs", default="prefill,configs,decode,global,fp32,backward,det,copy,cpu")
    ap.add_argument("--configs", default="C2,C3,C4", help="prefill configurations of the configs leg")
    ap.add_argument("--workload", default="NS", help="prefill workload: NS, C2, C3, C4")
    ap.add_argument("--cpu-positions", type=int, default=256)
    ap.add_argument("--cpu-decode-tokens", type=int, default=64)
    ap.add_argument("--fp32-steps", type=int, default=5)
    ap.add_argument("--global-steps", type=int, default=20)
    return ap.parse_args()


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "hbm_traffic.txt")


def measured_traffic(kernel, workload):
    """HBM bytes per dispatch of `kernel` on `workload` from the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE table (KiB per dispatch, each scaled by
    the factor its counter reads for a copy of known size), or None."""
    try:
        with open(TRAFFIC_FILE) as f:
            for line in f:
                parts = line.split()
                if len(parts) == 6 and not line.startswith("#") and parts[0] == kernel and parts[1] == workload:
                    fetch, write, ff, wf = (float(x) for x in parts[2:])
                    return 1024.0 * (fetch * ff + write * wf)
    except OSError:
        pass
    return None


def _time_kernel(fn, steps, warmup, flush=None):
    """Average device time per call (HIP events on the launch stream) plus wall time."""
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    times = []
    wall0 = time.perf_counter()
    if flush is None:
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for _ in range(steps):
            fn()
        end.record(stream)
        torch.cuda.synchronize()
        times = [start.elapsed_time(end) / steps] * steps
    else:
        evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
        for s, e in evs:
            flush()
            s.record(stream)
            fn()
            e.record(stream)
        torch.cuda.synchronize()
        times = [s.elapsed_time(e) for s, e in evs]
    wall = time.perf_counter() - wall0
    return statistics.fmean(times), statistics.median(times), wall


PREFILL_CFGS = ("NS", "C2", "C3", "C4")


def prefill_leg(args, name=None, steps=None):
    """One bf16 prefill configuration, inputs resident in HBM, HIP events on the launch stream."""
    import torch
    from archlab_amd import simplicial_attention, simplicial_varlen_attention
    from archlab_amd import workloads as W
    name = name or args.workload
    cfg = getattr(W, name)
    dev = torch.device("cuda:0")
    q, k1, k2, v1, v2, cu = W.prefill_inputs(cfg, device=dev)
    if cu is None:
        def fn():
            return simplicial_attention(q, k1, k2, v1, v2, cfg.w2, cfg.w1, scale=1.0, return_lse=True,
                                        kernel="mfma")
    else:
        def fn():
            return simplicial_varlen_attention(q, k1, k2, v1, v2, cu, cfg.w2, cfg.w1, scale=1.0,
                                               return_lse=True, kernel="mfma")
    mean_ms, med_ms, _ = _time_kernel(fn, steps or args.steps, args.warmup)
    flops = W.prefill_flops(cfg)
    tflops = flops / (mean_ms * 1e-3) / 1e12
    valid = W.prefill_valid_flops(cfg)
    del q, k1, k2, v1, v2, cu
    torch.cuda.empty_cache()
    return {
        "name": name, "cfg": cfg, "ms": mean_ms, "median_ms": med_ms, "tflops": tflops, "flops": flops,
        "bytes": W.prefill_bytes(cfg), "valid_pair_flops": valid,
        "valid_pair_tflops": valid / (mean_ms * 1e-3) / 1e12,
    }


def _prefill_roofline(pre):
    return {
        "bound": "mfma", "achieved": round(pre["tflops"], 2), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
        "frac": round(pre["tflops"] / PEAK_BF16_TFLOPS, 4),
        "traffic": measured_traffic("prefill_mfma_kernel", pre["name"]),
        "algorithmic_bytes": pre["bytes"],
    }


def _workload_label(cfg):
    return (f"{cfg.name}: bf16 prefill B={cfg.batch} H={cfg.heads_q}/{cfg.heads_kv} S={cfg.seqlen} D={cfg.dim} "
            f"w1(long)={cfg.w1} w2(short)={cfg.w2}" + (f" varlen {cfg.varlen_seqs} seqs" if cfg.varlen_seqs else "")
            + (f" sigma={cfg.sigma}" if cfg.sigma != 1.0 else ""))


def configs_leg(args):
    """The other BASELINE prefill configurations, each with its own roofline and CPU baseline."""
    out = {}
    for name in [c for c in args.configs.split(",") if c]:
        pre = prefill_leg(args, name)
        res = {"workload": _workload_label(pre["cfg"]), "ms_per_step": round(pre["ms"], 4),
               "tflops": round(pre["tflops"], 2), "flops_per_step": pre["flops"],
               "valid_pair_flops": pre["valid_pair_flops"], "valid_pair_tflops": round(pre["valid_pair_tflops"], 2),
               "kernel": "prefill_mfma_kernel", "roofline": _prefill_roofline(pre)}
        if "cpu" in set(args.legs.split(",")):
            res["cpu_baseline"] = cpu_leg(args, pre["cfg"])
        out[name] = res
    return out


def decode_leg(args):
    import torch
    from archlab_amd import simplicial_paged_attention
    from archlab_amd import workloads as W
    from archlab_amd.architectures.simplicial_paged import paged_plan
    cfg = W.C5
    dev = torch.device("cuda:0")
    inp = W.paged_inputs(cfg, device=dev)
    a = (inp["q"], inp["short_cache"], inp["long_cache"], inp["block_table"], inp["token_seq"], inp["token_pos"])
    kw = dict(short_window=cfg.w2, long_window=cfg.w1, scale=1.0)
    name, splits, ws_bytes = paged_plan(*a, **kw)
    # 1 GiB read between steps: evicts the windows from L2 and the 256 MB MALL,
    # and runs long enough that the host has queued the next call before the
    # GPU reaches it (the events then bracket the kernel alone).  A read, not a
    # fill: a fill leaves up to 256 MB of dirty lines whose write-back would
    # run inside the timed kernel and be charged to it.
    flush_buf = torch.ones(256 * 1024 * 1024, dtype=torch.int32, device=dev)

    def flush():
        flush_buf.max()

    def fn():
        return simplicial_paged_attention(*a, return_lse=True, **kw)
    mean_ms, med_ms, _ = _time_kernel(fn, args.decode_steps, max(args.warmup, 10), flush=flush)
    fp32_q = None
    if "fp32" in set(args.legs.split(",")):
        # the reference's serving caller sends an fp32 query over bf16 caches
        # (serving.py:83: q.float() * (scaling * sqrt(D)))
        qf = inp["q"].float()
        af = (qf,) + a[1:]
        fname, fsplits, _ = paged_plan(*af, **kw)
        fmean, fmed, _ = _time_kernel(lambda: simplicial_paged_attention(*af, return_lse=True, **kw),
                                      args.decode_steps, max(args.warmup, 10), flush=flush)
        fbytes = W.paged_bytes(cfg, inp["ctx"], out_bytes=4) + qf.numel() * 2  # q in 4 bytes instead of 2
        fp32_q = {"workload": f"{cfg.name} with an fp32 query (bf16 caches)", "us_per_step": round(fmed * 1e3, 3),
                  "tok_per_s": round(cfg.batch / (fmed * 1e-3), 1), "algorithmic_bytes_per_step": fbytes,
                  "achieved_gbs": round(fbytes / (fmed * 1e-3) / 1e9, 1),
                  "hbm_frac": round(fbytes / (fmed * 1e-3) / 1e9 / PEAK_HBM_GBS, 4), "kernel": fname,
                  "splits": fsplits}
    # the same with a write flush (a fill of the buffer), for comparison only
    _, wmed_ms, _ = _time_kernel(fn, args.decode_steps, 2, flush=lambda: flush_buf.fill_(1))
    # Back to back, as the layers of one serving step make their calls: four
    # calls, each over pages of its own (the block table rolled by 16 columns
    # per call: no two calls share a page, and 4 x 144 MB exceed the 256 MB
    # MALL), captured in one graph (no host gap between the launches) and
    # timed from one event before the first to one after the last, after the
    # same flush.  The time per call then holds the launch-to-launch gap but
    # not the event-to-dispatch latency of an isolated launch.
    layers = 4
    tables = [torch.roll(inp["block_table"], shifts=-16 * L, dims=1).contiguous() for L in range(layers)]

    def run_layers():
        for tab in tables:
            simplicial_paged_attention(a[0], a[1], a[2], tab, a[4], a[5], return_lse=True, **kw)
    run_layers()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run_layers()
    _, lmed_ms, _ = _time_kernel(graph.replay, max(args.decode_steps // layers, 10), 3, flush=flush)
    del graph, tables
    nbytes = W.paged_bytes(cfg, inp["ctx"], out_bytes=4)
    gbs = nbytes / (med_ms * 1e-3) / 1e9
    res = {
        "workload": cfg.name, "tokens_per_step": cfg.batch, "us_per_step": med_ms * 1e3,
        "mean_us_per_step": mean_ms * 1e3, "tok_per_s": cfg.batch / (med_ms * 1e-3),
        "algorithmic_bytes_per_step": nbytes, "achieved_gbs": gbs, "hbm_frac": gbs / PEAK_HBM_GBS,
        "kernel": name, "splits": splits, "flops_per_step": W.paged_flops(cfg, inp["ctx"]),
        "l2_flushed": True, "flush": "1 GiB read between steps",
        "us_per_step_after_write_flush": wmed_ms * 1e3,
        "us_per_step_back_to_back": lmed_ms * 1e3 / layers,
        "hbm_frac_back_to_back": nbytes / (lmed_ms * 1e-3 / layers) / 1e9 / PEAK_HBM_GBS,
    }
    if "global" in set(args.legs.split(",")):
        res["global_layer"] = global_layer_leg(args, cfg, inp, flush)
    traffic = measured_traffic("paged_mfma_kernel", "C5")
    res["roofline"] = {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                       "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": traffic}
    if "cpu" in set(args.legs.split(",")):
        res["cpu_baseline"] = decode_cpu_leg(args, cfg, inp)
    del inp, flush_buf
    torch.cuda.empty_cache()
    return res, fp32_q


def global_layer_leg(args, cfg, inp, flush):
    """The reference's serving call on a global layer (serving.py:49, :80-83):
    fp32 query, long_window = 1 << 30 (every key of the context), bf16 caches
    at the C5 contexts and block table; GQA group 4 (C5's 32 / 8 heads) and
    group 1 (8 / 8 heads over the same caches)."""
    import dataclasses
    import torch
    from archlab_amd import simplicial_paged_attention
    from archlab_amd import workloads as W
    from archlab_amd.architectures.simplicial_paged import paged_plan
    out = {}
    capacity = inp["block_table"].shape[1] * cfg.page
    for name, hq in (("G4_fp32_q", cfg.heads_q), ("G1_fp32_q", cfg.heads_kv)):
        q = inp["q"][:, :hq].float().contiguous()
        a = (q, inp["short_cache"], inp["long_cache"], inp["block_table"], inp["token_seq"], inp["token_pos"])
        kw = dict(short_window=cfg.w2, long_window=1 << 30, scale=1.0)
        kname, splits, ws = paged_plan(*a, **kw)
        mean_ms, med_ms, _ = _time_kernel(lambda: simplicial_paged_attention(*a, return_lse=True, **kw),
                                          args.global_steps, 3, flush=flush)
        g = dataclasses.replace(cfg, heads_q=hq, w1=capacity)
        nbytes = W.paged_bytes(g, inp["ctx"], out_bytes=4) + q.numel() * 2  # fp32 q: 4 bytes, not 2
        out[name] = {"workload": f"{cfg.name} global layer: HQ {hq} / HKV {cfg.heads_kv}, fp32 query, "
                                 f"long_window 2^30 (contexts {int(inp['ctx'].min())}-{int(inp['ctx'].max())})",
                     "us_per_step": round(med_ms * 1e3, 2), "tok_per_s": round(cfg.batch / (med_ms * 1e-3), 1),
                     "algorithmic_bytes_per_step": nbytes,
                     "achieved_gbs": round(nbytes / (med_ms * 1e-3) / 1e9, 1),
                     "hbm_frac": round(nbytes / (med_ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                     "kernel": kname, "splits": splits, "workspace_bytes": ws}
        _progress(f"global layer {name}: {med_ms * 1e3:.1f} us/step, splits {splits}")
    return out


def decode_cpu_leg(args, cfg, inp):
    """Oracle (fp32 restatement of the dense math) on the first tokens of C5:
    their windows are gathered through the block table on the GPU, copied to
    the host, and only the CPU evaluation is timed."""
    import torch
    from oracle import simplicial_oracle as O
    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    n = max(1, min(args.cpu_decode_tokens, cfg.batch))
    table = inp["block_table"].to(torch.int64)

    def gather(cache, s, lo, hi):
        pos = torch.arange(lo, hi + 1, device=cache.device)
        blocks = table[s][pos // cfg.page]
        return cache[0, blocks, pos % cfg.page], cache[1, blocks, pos % cfg.page]

    work = []
    for t in range(n):
        s, p = int(inp["token_seq"][t]), int(inp["token_pos"][t])
        k1, v1 = gather(inp["short_cache"], s, max(0, p - cfg.w2 + 1), p)
        k2, v2 = gather(inp["long_cache"], s, max(0, p - cfg.w1 + 1), p)
        work.append([x.float().cpu() for x in (inp["q"][t], k1, k2, v1, v2)])
    O._single_query(*work[0], 1.0)  # warm-up
    runs = []
    for _ in range(3):
        t0 = time.perf_counter()
        for w in work:
            O._single_query(*w, 1.0)
        runs.append(time.perf_counter() - t0)
    med = statistics.median(runs)
    which = "all" if n == cfg.batch else f"the first {n} of"
    return {
        "value": n / med, "unit": "tok/s", "cores": threads, "kind": "port",
        "sample": (f"oracle._single_query fp32 on {which} {cfg.batch} C5 tokens (windows gathered "
                   f"through the block table, all {cfg.heads_q} heads), median of 3; "
                   f"{med / n * 1e3:.2f} ms/token"),
    }


def backward_leg(args, fwd_ms, workload=None, cfg=None):
    """Forward + backward (torch.autograd through the library's backward) on the
    prefill workload; nominal backward FLOPs = 2x the forward's (the reference
    counts 12*H*D*triples for forward + backward, limite_cost.py:69-73)."""
    import torch
    from archlab_amd import simplicial_attention, simplicial_varlen_attention
    from archlab_amd import workloads as W
    cfg = cfg or getattr(W, workload or args.workload)
    dev = torch.device("cuda:0")
    q, k1, k2, v1, v2, cu = W.prefill_inputs(cfg, device=dev)
    xs = [t.detach().requires_grad_(True) for t in (q, k1, k2, v1, v2)]
    g = torch.Generator("cpu").manual_seed(7)
    dy = torch.randn(q.shape[:-1] + (v1.shape[-1],), generator=g).to(cfg.dtype).to(dev)

    def fwd():
        if cu is None:
            return simplicial_attention(*xs, cfg.w2, cfg.w1, scale=1.0)
        return simplicial_varlen_attention(*xs, cu, cfg.w2, cfg.w1, scale=1.0)

    def step():
        return torch.autograd.grad(fwd(), xs, dy)
    mean_ms, med_ms, _ = _time_kernel(step, args.bwd_steps, 3)
    if fwd_ms is None:
        with torch.no_grad():
            fwd_ms, _, _ = _time_kernel(fwd, args.bwd_steps, 3)
    bwd_ms = mean_ms - fwd_ms
    flops = 2.0 * W.prefill_flops(cfg)
    valid = 2.0 * W.prefill_valid_flops(cfg)
    del xs, dy, q, k1, k2, v1, v2
    torch.cuda.empty_cache()
    return {
        "workload": cfg.name, "fwd_bwd_ms": mean_ms, "fwd_ms": fwd_ms, "bwd_ms": bwd_ms,
        "bwd_flops": flops, "bwd_tflops": flops / (bwd_ms * 1e-3) / 1e12,
        "bwd_frac_of_peak": flops / (bwd_ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS,
        "bwd_valid_pair_flops": valid, "bwd_valid_pair_tflops": valid / (bwd_ms * 1e-3) / 1e12,
        "dtype": str(cfg.dtype).replace("torch.", ""),
        "kernels": ("bwd_dq_mfma_kernel (dq, dk1 and dv1 partials), bwd_dk1_sum_kernel, bwd_dkv2_mfma_kernel "
                    "(dk2 and dv2 in one launch) (+ split_hilo_kernel, bwd_delta_kernel)"
                    if cfg.dtype == torch.float32 else
                    "bwd_dq_mfma_kernel, bwd_dkv1_mfma_kernel, bwd_dkv2_mfma_kernel (+ bwd_delta_kernel)"),
    }


def determinant_leg(args):
    """Score width 512 over value width 256 (the determinant expansion of
    256-wide heads, simplicial_attention.py:111-148) at C4 geometry, bf16
    forward on the matrix cores; FLOPs 2 * (DS + DV) per pair and head."""
    import dataclasses
    import torch
    from archlab_amd import simplicial_attention
    from archlab_amd import workloads as W
    cfg = dataclasses.replace(W.C4, name="C4-DS512-DV256")
    dev = torch.device("cuda:0")
    g = torch.Generator("cpu").manual_seed(cfg.seed)
    shp = lambda h, d: (cfg.batch, cfg.seqlen, h, d)  # noqa: E731
    q = (torch.randn(shp(cfg.heads_q, 512), generator=g) * 0.5 / math.sqrt(512)).to(torch.bfloat16).to(dev)
    k1, k2 = ((torch.randn(shp(cfg.heads_kv, 512), generator=g) * 0.5).to(torch.bfloat16).to(dev) for _ in range(2))
    v1, v2 = ((torch.randn(shp(cfg.heads_kv, 256), generator=g) * 0.5).to(torch.bfloat16).to(dev) for _ in range(2))
    fn = lambda: simplicial_attention(q, k1, k2, v1, v2, cfg.w2, cfg.w1, scale=1.0, return_lse=True,  # noqa: E731
                                      kernel="mfma")
    mean_ms, _, _ = _time_kernel(fn, max(5, args.steps // 5), 2)
    flops = 2.0 * cfg.batch * cfg.heads_q * cfg.seqlen * cfg.w1 * cfg.w2 * (512 + 256)
    del q, k1, k2, v1, v2
    torch.cuda.empty_cache()
    return {"workload": f"{cfg.name}: bf16 prefill B={cfg.batch} H={cfg.heads_q} S={cfg.seqlen} DS=512 DV=256 "
                        f"w1(long)={cfg.w1} w2(short)={cfg.w2}", "ms_per_step": round(mean_ms, 4),
            "flops_per_step": flops, "tflops": round(flops / (mean_ms * 1e-3) / 1e12, 2),
            "kernel": "prefill_mfma_kernel<512,256>"}


def copy_leg(args):
    """Plain device copy of a known byte count (1 GiB read + 1 GiB written per
    call): the calibration kernel for the FETCH_SIZE / WRITE_SIZE counters."""
    import torch
    n = 1 << 29  # bf16 elements = 1 GiB
    src = torch.ones(n, dtype=torch.bfloat16, device="cuda:0")
    dst = torch.empty_like(src)
    mean_ms, _, _ = _time_kernel(lambda: dst.copy_(src), max(2, args.steps // 4), 1)
    return {"bytes_read": 2 * n, "bytes_written": 2 * n, "ms": mean_ms,
            "gbs": 4 * n / (mean_ms * 1e-3) / 1e9}


def cpu_leg(args, cfg, full=False):
    """Oracle (fp32 restatement of reference_simplicial) on evenly spaced query
    positions (window edges and, for packed workloads, sequence starts
    included), or on every position with ``full``."""
    import torch
    from archlab_amd import workloads as W
    from oracle import simplicial_oracle as O
    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    q, k1, k2, v1, v2, cu = W.prefill_inputs(cfg, device="cpu")
    x = [t.float() for t in (q, k1, k2, v1, v2)]
    s = cfg.tokens if cu is not None else cfg.seqlen
    if full:
        pos = list(range(s))
    else:
        n = max(6, min(args.cpu_positions, s))
        edges = {0, cfg.w2 - 1, cfg.w2, cfg.w1 - 1, cfg.w1, s - 1}
        if cu is not None:
            edges |= {int(c) for c in cu[:-1]}
        pos = sorted(set(int(round(i * (s - 1) / (n - 1))) for i in range(n)) | {e for e in edges if 0 <= e < s})

    def run(positions):
        if cu is None:
            return O.reference_simplicial(*x, cfg.w2, cfg.w1, scale=1.0, query_positions=positions, return_lse=True)
        return O.varlen_reference(*x, cu, cfg.w2, cfg.w1, scale=1.0, query_positions=positions, return_lse=True)
    run(pos[:4])  # warm-up
    runs = []
    for _ in range(3):
        t0 = time.perf_counter()
        run(pos)
        runs.append(time.perf_counter() - t0)
    med = statistics.median(runs)
    if cu is None:
        # nominal FLOPs of the sampled queries (same 4*B*H*w1*w2*D per query as the GPU figure)
        flops = 4.0 * cfg.batch * cfg.heads_q * cfg.w1 * cfg.w2 * cfg.dim * len(pos)
        per_query = med / len(pos)
        total = cfg.seqlen
    else:
        flops = W.prefill_flops(cfg) * len(pos) / cfg.tokens
        per_query = med / len(pos)
        total = cfg.tokens
    kind = "all" if full else f"{len(pos)} evenly spaced"
    sample = (f"oracle.{'reference_simplicial' if cu is None else 'varlen_reference'} fp32 on {kind} query "
              f"positions{'' if full else ' (incl. window edges' + (' and sequence starts)' if cu is not None else ')')} "
              f"of {cfg.name}, all B*H rows, median of 3; {per_query * 1e3:.2f} ms/query")
    if not full:
        sample += f"; full {total}-query run extrapolated to {per_query * total:.1f} s"
    return {"value": flops / med / 1e12, "unit": "TFLOP/s", "cores": threads, "kind": "port", "sample": sample,
            "seconds": round(med, 3)}


def fp32_prefill_leg(args):
    """fp32 prefill at C2 geometry (what deepseek_v41_adapter.py:138-144 sends)
    and BASELINE config C1 in full (fp32) on the GPU, plus C1 on the CPU."""
    import dataclasses
    import torch
    from archlab_amd import simplicial_attention
    from archlab_amd import workloads as W
    from archlab_amd.architectures.simplicial_attention import prefill_kernel_name
    dev = torch.device("cuda:0")
    out = {}
    for cfg, steps in ((dataclasses.replace(W.C2, name="C2-fp32-prefill", dtype=torch.float32), args.fp32_steps),
                       (W.C1, max(args.fp32_steps, 20))):
        q, k1, k2, v1, v2, _ = W.prefill_inputs(cfg, device=dev)
        fn = lambda: simplicial_attention(q, k1, k2, v1, v2, cfg.w2, cfg.w1, scale=1.0, return_lse=True)  # noqa: E731
        mean_ms, _, _ = _time_kernel(fn, steps, 1)
        flops = W.prefill_flops(cfg)
        res = {"workload": _workload_label(cfg).replace("bf16", "fp32"), "ms_per_step": round(mean_ms, 4),
               "tflops": round(flops / (mean_ms * 1e-3) / 1e12, 3), "kernel": prefill_kernel_name(q, k1, v1)}
        del q, k1, k2, v1, v2
        if cfg is W.C1 and "cpu" in set(args.legs.split(",")):
            res["cpu_baseline"] = cpu_leg(args, cfg, full=True)
        out["C1" if cfg is W.C1 else "C2_fp32"] = res
    torch.cuda.empty_cache()
    return out


def _progress(msg):
    """Progress on stderr (stdout carries only the JSON line)."""
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def _rounded(d):
    return {k: (round(v, 4) if isinstance(v, float) else v) for k, v in d.items()}


def main():
    args = _args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; --gpus must be 1",
                          "n_gpus": args.gpus}))
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print(json.dumps({"error": "no ROCm GPU visible"}))
        sys.exit(1)
    legs = set(args.legs.split(","))
    from archlab_amd import workloads as W
    out = {
        "metric": "2-simplicial fwd TFLOP/s + % bf16 MFMA peak (S=8k,D=128); decode tok/s",
        "value": None, "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": None, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic (seeded N(0,1), Q scaled 1/sqrt(D), scale=1.0)",
    }
    t_start = time.perf_counter()
    pre = None
    if "prefill" in legs:
        pre = prefill_leg(args)
        cfg = pre["cfg"]
        out["value"] = round(pre["tflops"], 2)
        out["ms_per_step"] = round(pre["ms"], 4)
        out["config"] = {"workload": _workload_label(cfg), "flops_per_step": pre["flops"],
                         "valid_pair_flops": pre["valid_pair_flops"],
                         "valid_pair_tflops": round(pre["valid_pair_tflops"], 2),
                         "kernel": "prefill_mfma_kernel"}
        out["roofline"] = _prefill_roofline(pre)
        _progress(f"prefill {pre['name']}: {pre['ms']:.3f} ms, {pre['tflops']:.1f} TFLOP/s")
    if "configs" in legs:
        out["configs"] = configs_leg(args)
        _progress("configs: " + ", ".join(f"{k} {v['ms_per_step']} ms" for k, v in out["configs"].items()))
    fp32 = {}
    if "decode" in legs:
        dec, fp32_q = decode_leg(args)
        out["decode"] = _rounded(dec)
        if fp32_q is not None:
            fp32["C5_fp32_q"] = fp32_q
        if pre is None:
            out["value"] = round(dec["tok_per_s"], 1)
            out["unit"] = "tok/s"
            out["ms_per_step"] = round(dec["us_per_step"] / 1e3, 5)
            out["config"] = {"workload": dec["workload"]}
            out["roofline"] = dec["roofline"]
        _progress(f"decode C5: {dec['us_per_step']:.2f} us/step")
    if "fp32" in legs:
        fp32.update(fp32_prefill_leg(args))
        # the reference's fp32 training core at its adapter geometry, forward +
        # backward, next to the same shape in bf16
        import dataclasses
        f32b = backward_leg(args, None, cfg=W.DSV41)
        b16b = backward_leg(args, None, cfg=dataclasses.replace(W.DSV41, name="DSV41-bf16", dtype=torch.bfloat16))
        fp32["DSV41_fwd_bwd"] = _rounded(f32b)
        fp32["DSV41_fwd_bwd"]["bf16_same_shape"] = _rounded(b16b)
        fp32["DSV41_fwd_bwd"]["bwd_fp32_over_bf16"] = round(f32b["bwd_ms"] / b16b["bwd_ms"], 3)
        _progress(f"fp32 DSV41 fwd+bwd: {f32b['fwd_bwd_ms']:.2f} ms (bwd {f32b['bwd_ms']:.2f} ms, "
                  f"bf16 bwd {b16b['bwd_ms']:.2f} ms)")
        _progress("fp32: " + ", ".join(
            f"{k} {v.get('ms_per_step', v.get('us_per_step', v.get('fwd_bwd_ms')))}" for k, v in fp32.items()))
    if fp32:
        out["fp32"] = fp32
    if "backward" in legs:
        bwd = backward_leg(args, pre["ms"] if pre is not None else None)
        out["backward"] = _rounded(bwd)
        _progress(f"backward: {bwd['bwd_ms']:.2f} ms")
        extra = {}
        for name in [c for c in args.bwd_configs.split(",") if c and c != args.workload]:
            b = backward_leg(args, None, workload=name)
            extra[name] = _rounded(b)
            _progress(f"backward {name}: {b['bwd_ms']:.2f} ms")
        if extra:
            out["backward_configs"] = extra
    if "det" in legs:
        out["determinant_ds512"] = determinant_leg(args)
        _progress(f"DS 512 / DV 256: {out['determinant_ds512']['ms_per_step']} ms")
    if "copy" in legs:
        out["copy_calibration"] = copy = _rounded(copy_leg(args))
        if "decode" in out:
            # the decode rate next to the achievable copy rate of this GPU
            out["decode"]["achievable_copy_gbs"] = copy["gbs"]
            out["decode"]["frac_of_achievable_copy"] = round(out["decode"]["achieved_gbs"] / copy["gbs"], 4)
        _progress(f"copy: {copy['gbs']:.0f} GB/s")
    if "cpu" in legs:
        cfg = pre["cfg"] if pre is not None else W.NS
        out["cpu_baseline"] = cpu_leg(args, cfg)
        _progress("cpu baseline done")
    _progress(f"total {time.perf_counter() - t_start:.1f} s")
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
