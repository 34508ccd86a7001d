// Paged-KV forward (serving form: any mix of prefill and decode tokens) for the
// 2-simplicial attention library.  Replaces the reference's Triton _paged
// kernel and its torch split merge (archlab/architectures/simplicial_paged.py:19-65,
// :105-128) behind simplicial_paged_attention.
//
// Each query token carries (sequence, absolute position).  Its short window
// (k1, v1) and long window (k2, v2) are gathered through one block table per
// cache: block = table[seq, pos / block_size] (widened to int64 before the
// stride multiply), slot = pos % block_size.
//
// bf16 MFMA kernel: a workgroup owns (token, KV group, split, task block).
// A task is (query head in the group, 32-row group of the short window); NW
// waves take NW tasks.  The long window is cut into 32-key chunks that start
// at pos - long_window + 1; the split index partitions only the chunks that
// hold valid keys (not the table capacity), so no split scans empty pages.
// All waves of a workgroup consume the same chunk, double-buffered in LDS,
// gathered with 16-byte loads (a 64-element bf16 row is 8 lanes x 16 B).
// Every (split, row group) writes a partial (max, sum, unnormalised output);
// sa_paged_combine merges them in a fixed order, so results are
// run-to-run bit-identical.
#include "sa_generic.h"
#include "sa_mfma.h"
#include "sa_launch.h"

namespace sa {

struct PagedParams {
  const void* q;  // bf16, or fp32 (QF32 kernels)
  int64_t q_st, q_sh;
  const bf16* sc;
  const bf16* lc;
  int64_t sc_a, sc_b, sc_s, sc_h;
  int64_t lc_a, lc_b, lc_s, lc_h;
  const void* stable;
  const void* ltable;
  int64_t st_s, lt_s;
  const void* tseq;
  const void* tpos;
  int stab64, ltab64, seq64, pos64;  // index widths (int64 when set)
  int st_w, lt_w, num_seqs;
  int64_t s_blocks, l_blocks;
  int tokens, hq, hk, group, bs;
  int ws, wl, nc, nr;
  float sl2;
  int q_neg;
  int splits;
  int tasks;    // group * nr
  int tblocks;  // task blocks per (token, KV group)
  float* part_o;  // [P][tokens][hq][D], P = splits * nr
  float* part_m;  // [P][tokens][hq]
  float* part_z;
  int direct;     // splits * nr == 1: write out / lse directly, no partials
  float* out;
  int64_t o_st, o_sh;
  float* lse;
  const int32_t* caps;  // optional per-token window limits [tokens][2]
};

constexpr int kPosCache = 1024;            // long-window positions whose row offsets are kept in LDS
constexpr int kSegChunks = kPosCache / kChunk;  // chunks of one such segment

// MULTI: the split may span more than one segment of kSegChunks chunks (long
// windows); without it the segment loop below runs exactly once and folds
// away, which keeps the register allocation of the short-window kernel.
// QF32: fp32 query over bf16 caches (the reference's serving input,
// serving.py:83): a = q ⊙ k1 and P stay fp32-accurate through hi/lo bf16
// terms (RowBlock HL), twice the MFMA work of the bf16 kernel.
// Workgroups of one or two waves hold one wave per SIMD whatever their
// register count (two workgroups per CU), so they may use the whole register
// file; four-wave workgroups are bounded to two waves per SIMD.
template <int D, int NW, int P, bool MULTI, bool QF32>
__global__ __launch_bounds__(64 * NW, (D >= 256 || NW < 4 ? 1 : 2)) void paged_mfma_kernel(PagedParams p) {
  using G = FwdGeom<D, D, kChunk, NW>;
  using RB = RowBlock<D, D, QF32>;
  constexpr bool kPipelined = D <= 128 && P >= 2;  // second score tile fits the registers up to D = 128
  constexpr int kStepPF = 2;  // V fragments read ahead of the PV MFMAs (C5 42.0 -> 41.6 us)
  constexpr int SLOT = G::SLOT;
  constexpr int R = P + 1;
  constexpr int NI = G::NI;  // DMA instructions per wave per tile
  extern __shared__ __attribute__((aligned(16))) char lds[];
  const int tid = tid_x(), lane = tid & 63;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half = lane >> 5, n = lane & 31;

  int b = bid_x();
  const int tb = b % p.tblocks;
  b /= p.tblocks;
  const int split = b % p.splits;
  b /= p.splits;
  const int g = b % p.hk;
  const int token = b / p.hk;

  // per-token scalars, both index loads in one round trip (uniform: SGPRs)
  const int seq_raw = (int)clamp64(p.seq64 ? ((const int64_t*)p.tseq)[token] : ((const int32_t*)p.tseq)[token], 0,
                                   p.num_seqs - 1);
  const int pos_raw = (int)(p.pos64 ? ((const int64_t*)p.tpos)[token] : ((const int32_t*)p.tpos)[token]);
  // per-token window limits (the chunk grid stays the one of p.wl)
  int ws_t = p.ws, wl_t = p.wl;
  if (p.caps) {
    ws_t = max(1, min(ws_t, p.caps[2 * token]));
    wl_t = max(1, min(wl_t, p.caps[2 * token + 1]));
  }
  const int64_t seq = __builtin_amdgcn_readfirstlane(seq_raw);
  const int pos = __builtin_amdgcn_readfirstlane(pos_raw);
  const int task = tb * NW + wid;
  const bool task_ok = task < p.tasks;
  const int hi = task_ok ? task % p.group : 0;
  const int r = task_ok ? task / p.group : 0;
  const int h = g * p.group + hi;

  const int lo2 = max(0, pos - __builtin_amdgcn_readfirstlane(wl_t) + 1);
  const int lo1 = max(0, pos - __builtin_amdgcn_readfirstlane(ws_t) + 1);
  const int kstart = pos - p.wl + 1;  // chunk grid origin (position)
  const int cfirst = (lo2 - kstart) / kChunk;
  const int nvalid = p.nc - cfirst;
  const int per = (nvalid + p.splits - 1) / p.splits;
  const int cbeg = cfirst + split * per;
  const int cend = min(p.nc, cbeg + per);

  RB rb;
  const int j = pos - 32 * r - n;
  const bool row_ok = task_ok && j >= lo1 && cbeg < cend;

  // Row offsets (element offset of the K row of head g) of the long-window
  // positions of one segment (at most kSegChunks chunks = kPosCache
  // positions) are computed once and kept in LDS: a block-table load inside
  // the pipeline would be a vector load whose result feeds a DMA address, and
  // waiting for it would also wait for every older tile load (vector loads
  // complete in order).  A split longer than one segment (global layers)
  // walks its chunks segment by segment; the row state carries over.  All
  // block-table loads of a segment, including (first segment) this lane's
  // short-axis row, go out in one round trip.
  int64_t* roff = (int64_t*)(lds + R * SLOT);
  // With one row group (nr == 1: every wave's rows are j = pos - n), the
  // short rows (k1 at slot row n = pos - j, v1 in the V
  // region: the ring-slot geometry) and the q rows of the workgroup's tasks
  // are staged once per workgroup by DMA, ahead of the first tiles: the A
  // rows (and, for bf16 queries, the v1 registers) are read from LDS while
  // the tiles stream.
  // (Vector loads of the short rows would retire behind the tile DMAs and be
  // fetched by every wave.)  The short rows use the ring slot that the first
  // segment's third tile fills only after the key loop's first barrier.
  constexpr int QB = (QF32 ? 4 : 2) * D;         // bytes of one q row
  int64_t* const soffs = roff + kPosCache;       // [32] short-row offsets
  char* const qslot = (char*)(soffs + 32);       // [NW] q rows, QB bytes each (bf16 staged: then [NW] fp32 rows)
  constexpr bool kStage = D <= 128 && P >= 2 && P * NI < 64 && !MULTI;  // the wait below counts P tiles' DMAs
  const bool stage = kStage && p.nr == 1;        // uniform
  // Lookups are branch-free (clamped indices) so that every load of a batch
  // is in flight before the first result is used.
  constexpr int kBatch = 4;  // long-axis table loads in flight per lane
  constexpr int kStep = kBatch * 64 * NW;
  int64_t soff = 0;
  auto fill = [&](int seg_lo, int nseg, int i0, bool with_short) {
    int64_t raw[kBatch], sraw = 0;
    auto lookup = [&](auto tag) {
      using I = decltype(tag);
      const I* lt = (const I*)p.ltable + seq * p.lt_s;
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        const int ps = seg_lo + min(i0 + tid + u * 64 * NW, nseg - 1);
        raw[u] = (int64_t)lt[min(ps / p.bs, p.lt_w - 1)];
      }
    };
    if (with_short) {  // issued with the long-table loads (uniform branches)
      const int col = min(max(j, 0) / p.bs, p.st_w - 1);
      sraw = p.stab64 ? ((const int64_t*)p.stable)[seq * p.st_s + col]
                      : (int64_t)((const int32_t*)p.stable)[seq * p.st_s + col];
    }
    if (p.ltab64) lookup(int64_t{});
    else lookup(int32_t{});
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int i = i0 + tid + u * 64 * NW;
      if (i < nseg)
        roff[i] = clamp64(raw[u], 0, p.l_blocks - 1) * p.lc_b + (int64_t)((seg_lo + i) % p.bs) * p.lc_s +
                  (int64_t)g * p.lc_h;
    }
    if (with_short && row_ok)
      soff = clamp64(sraw, 0, p.s_blocks - 1) * p.sc_b + (int64_t)(j % p.bs) * p.sc_s + (int64_t)g * p.sc_h;
    if (with_short && stage && wid == 0 && lane < 32) soffs[lane] = soff;  // row n of the short slot
  };

  // this lane's tile row / segment / tensor for each of its DMA instructions:
  // kept in registers, or, with many instructions per wave (one-wave
  // workgroups at widths of 256: 3 x 34 values), decoded again at each use
  // from a fresh lane id
  constexpr bool kKeepSlots = NI <= 20;
  int drow[kKeepSlots ? NI : 1], dseg[kKeepSlots ? NI : 1], dv[kKeepSlots ? NI : 1];
  if constexpr (kKeepSlots) {
#pragma unroll
    for (int k = 0; k < NI; ++k) G::decode(wid, k, lane, dv[k], drow[k], dseg[k]);
  }
  auto slot_of = [&](int k, int& v_, int& row_, int& seg_) {
    if constexpr (kKeepSlots) {
      v_ = dv[k], row_ = drow[k], seg_ = dseg[k];
    } else {
      G::decode(wid, k, fresh_lane(), v_, row_, seg_);
    }
  };

  // tile rows outside [lo2, pos] re-read the nearest valid row (masked later);
  // every row offset is read from LDS before the first DMA is issued
  auto issue = [&](int c, int seg_lo) {
    const int k0 = kstart + kChunk * c;
    char* slot = lds + (c % R) * SLOT;
    constexpr int KG = NI < 8 ? NI : 8;  // offsets read per group of DMA instructions
    static_for<0, (NI + KG - 1) / KG>([&](auto kg) {
      constexpr int kb = decltype(kg)::value * KG;
      int64_t off[KG];
      int tv[KG], tseg[KG];
#pragma unroll
      for (int k = 0; k < KG; ++k)
        if (kb + k < NI) {
          int trow;
          slot_of(kb + k, tv[k], trow, tseg[k]);
          off[k] = roff[min(min(max(k0 + trow, lo2), pos) - seg_lo, kPosCache - 1)];
        }
#pragma unroll
      for (int k = 0; k < KG; ++k)
        if (kb + k < NI) dma16(p.lc + off[k] + (tv[k] ? p.lc_a : 0) + tseg[k] * 8, G::dst(slot, wid, kb + k));
    });
  };

  // v1 of this lane's short row, in the layout the epilogue consumes: held in
  // registers through the key loop (D <= 128; at D = 256 the registers are
  // needed by the accumulators and the epilogue loads it)
  constexpr bool kV1Regs = D <= 128 && (!QF32 || (!MULTI && NW == 4));
  bf16x4 v1r[kV1Regs ? D / 64 : 1][2][4];
  if (cbeg < cend) {
    for (int sb = cbeg; sb < cend; sb += kSegChunks) {
      const int se = MULTI ? min(cend, sb + kSegChunks) : cend;
      const int seg_lo = max(lo2, kstart + kChunk * sb);
      const int nseg = min(pos, kstart + kChunk * se - 1) - seg_lo + 1;  // 1 .. kPosCache
      const bool first = sb == cbeg;
      fill(seg_lo, nseg, 0, first);
      for (int i0 = kStep; i0 < nseg; i0 += kStep) fill(seg_lo, nseg, i0, false);
      __syncthreads();
      char* const sslot = lds + ((sb + 2) % R) * SLOT;  // free until tile sb+2 is issued
      if (first && stage) {
        // the short rows: NI DMA instructions per wave, ring-slot geometry
#pragma unroll
        for (int k = 0; k < NI; ++k) {
          int sv_, srow_, sseg_;
          slot_of(k, sv_, srow_, sseg_);
          dma16(p.sc + soffs[srow_] + (sv_ ? p.sc_a : 0) + sseg_ * 8, G::dst(sslot, wid, k));
        }
        // the q rows of the workgroup's tasks (wave 0): lane -> row, 16-byte segment
        if (wid == 0) {
          constexpr int kQI = (NW * QB + 1023) / 1024;
#pragma unroll
          for (int k = 0; k < kQI; ++k) {
            const int b = 1024 * k + 16 * lane;
            const int qr = min(b / QB, NW - 1), qs = (b % QB) / 16;
            const int tq = tb * NW + qr;
            const int hq = g * p.group + (tq < p.tasks ? tq % p.group : 0);
            const int64_t qe = (int64_t)token * p.q_st + (int64_t)hq * p.q_sh;  // elements
            const char* src = QF32 ? (const char*)((const float*)p.q + qe) : (const char*)((const bf16*)p.q + qe);
            dma16((const bf16*)(src + 16 * qs), qslot + b);
          }
        }
      }
#pragma unroll
      for (int e = 0; e < P; ++e)
        if (sb + e < se) issue(sb + e, seg_lo);
      if (first) {
        if (stage) {
          // the staged rows have landed (the tiles issued after them may not)
          if constexpr (kStage) wait_tiles<NI, P + 1>(min(P, se - sb));
          block_barrier();
          if constexpr (QF32)
            rb.form_a_f32((const float*)(qslot + wid * QB), (const bf16*)(sslot + n * G::RSK), row_ok, half,
                          p.q_neg != 0);
          else {
            // the wave's q row widened to fp32 (after the NW staged rows)
            char* const qf = qslot + NW * QB + wid * 4 * D;
            RB::widen_q(qslot + wid * QB, qf, fresh_lane(), p.q_neg != 0);
            rb.form_a_qf(sslot + n * G::RSK, qf, row_ok, half);
          }
          if constexpr (kV1Regs) {
            const char* v1s = sslot + G::VOFF + n * G::RSV;
#pragma unroll
            for (int sl = 0; sl < D / 64; ++sl)
#pragma unroll
              for (int dbl = 0; dbl < 2; ++dbl)
#pragma unroll
                for (int q4 = 0; q4 < 4; ++q4)
                  v1r[sl][dbl][q4] = *(const bf16x4*)(v1s + 2 * (64 * sl + 32 * dbl + 8 * q4 + 4 * half));
            // every read of the slot is complete before the barrier that
            // precedes the DMA of tile sb+2 into it
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
          }
        } else {
          if constexpr (kV1Regs) {
            const bf16* v1row = p.sc + soff + p.sc_a;
#pragma unroll
            for (int sl = 0; sl < D / 64; ++sl)
#pragma unroll
              for (int dbl = 0; dbl < 2; ++dbl)
#pragma unroll
                for (int q4 = 0; q4 < 4; ++q4)
                  v1r[sl][dbl][q4] = *(const bf16x4*)(v1row + 64 * sl + 32 * dbl + 8 * q4 + 4 * half);
          }
          const int64_t qoff = (int64_t)token * p.q_st + (int64_t)h * p.q_sh;
          if constexpr (QF32) rb.form_a_f32((const float*)p.q + qoff, p.sc + soff, row_ok, half, p.q_neg != 0);
          else rb.form_a((const bf16*)p.q + qoff, p.sc + soff, row_ok, half, p.q_neg != 0);
        }
        rb.reset(row_ok);
      }
      if constexpr (kPipelined) {
        // software-pipelined loop (see the prefill kernel): iteration c needs K
        // of chunk c+1 and V of chunk c
        wait_tiles<NI, P>(min(P - 1, se - 1 - sb));
        block_barrier();
        floatx16 s = rb.template qk<G::RSK>(lds + (sb % R) * SLOT, 0, lane);
        float cmax = RB::row_max(s) * p.sl2;
        auto begin_chunk = [&](int c) {
          block_barrier();
          if (c + P < se) issue(c + P, seg_lo);
          const int kfirst = kstart + kChunk * c;
          const int klo = task_ok ? max(lo2 - kfirst, 0) : kChunk;
          const int khi = task_ok ? min(pos - kfirst, kChunk - 1) : -1;
          if (klo > 0 || khi < kChunk - 1) {  // edge chunk (uniform branch)
            RB::mask(s, lane, klo, khi);
            cmax = RB::row_max(s) * p.sl2;
          }
          rb.rescale(cmax);
        };
        int c = sb;
        for (; c + 1 < se; ++c) {
          wait_tiles<NI, P>(min(P - 2, se - 2 - c));
          begin_chunk(c);
          const char* slot = lds + (c % R) * SLOT;
          rb.template step<G::RSK, G::RSV, true, kStepPF>(s, cmax, lds + ((c + 1) % R) * SLOT, slot + G::VOFF, 0,
                                                          lane, p.sl2);
        }
        begin_chunk(c);
        const char* slot = lds + (c % R) * SLOT;
        rb.template step<G::RSK, G::RSV, false, kStepPF>(s, cmax, slot, slot + G::VOFF, 0, lane, p.sl2);
      } else {
        for (int c = sb; c < se; ++c) {
          wait_tiles<NI, P>(min(P - 1, se - 1 - c));
          block_barrier();
          if (c + P < se) issue(c + P, seg_lo);
          // unconditional (see the prefill kernel): idle waves get an empty key range
          const int kfirst = kstart + kChunk * c;
          const char* slot = lds + (c % R) * SLOT;
          // the split's first chunk holds a valid key of the token
          rb.template chunk<G::RSK, G::RSV>(slot, slot + G::VOFF, 0, lane, p.sl2,
                                            task_ok ? max(lo2 - kfirst, 0) : kChunk,
                                            task_ok ? min(pos - kfirst, kChunk - 1) : -1, task_ok && c == cbeg);
        }
      }
      block_barrier();  // tile and row-offset reads of this segment done
      if constexpr (!MULTI) break;
    }
  } else {
    if constexpr (kV1Regs) {
#pragma unroll
      for (int sl = 0; sl < D / 64; ++sl)
#pragma unroll
        for (int dbl = 0; dbl < 2; ++dbl)
#pragma unroll
          for (int q4 = 0; q4 < 4; ++q4) v1r[sl][dbl][q4] = bf16x4{};
    }
    rb.reset(false);
  }

  // ---- epilogue: merge this wave's 32 rows, write one partial (or, when
  // this workgroup is the only contributor, the final output)
  const float zrow = pair_sum(rb.z);
  const float mrow = row_ok ? rb.m : -INFINITY;
  const float Mw = wave_max(mrow);
  const float wgt = (row_ok && Mw > -INFINITY) ? fast_exp2(mrow - Mw) : 0.f;
  const float Zw = half_sum(wgt * zrow);
  float* red = (float*)lds + wid * (64 * 36);
  const int pidx = split * p.nr + r;
  const int64_t prow = ((int64_t)pidx * p.tokens + token) * p.hq + h;
#pragma unroll
  for (int sl = 0; sl < D / 64; ++sl) {
#pragma unroll
    for (int dbl = 0; dbl < 2; ++dbl) {
      const int db = 2 * sl + dbl;
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const int dd = 32 * dbl + 8 * q4 + 4 * half;
        bf16x4 vv;
        if constexpr (kV1Regs) vv = row_ok ? v1r[sl][dbl][q4] : bf16x4{};
        else vv = row_ok ? *(const bf16x4*)(p.sc + soff + p.sc_a + 64 * sl + dd) : bf16x4{};
#pragma unroll
        for (int e = 0; e < 4; ++e) red[(dd + e) * 36 + n] = wgt * (float)vv[e] * rb.o[db][4 * q4 + e];
      }
    }
    // `red` is private to this wave and a wave's LDS accesses execute in order
    float acc = 0.f;
    const floatx4* row4 = (const floatx4*)(red + lane * 36);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      floatx4 x = row4[i];
      acc += (x[0] + x[1]) + (x[2] + x[3]);
    }
    if (task_ok) {
      if (p.direct) p.out[(int64_t)token * p.o_st + (int64_t)h * p.o_sh + 64 * sl + lane] = acc / Zw;
      else p.part_o[prow * D + 64 * sl + lane] = acc;
    }
  }
  if (task_ok && lane == 0) {
    if (p.direct) {
      if (p.lse) p.lse[(int64_t)token * p.hq + h] = (Mw + __log2f(Zw)) * kLn2;
    } else {
      p.part_m[prow] = Mw;
      p.part_z[prow] = Zw;
    }
  }
}

// Merge P = splits * row-groups partials per (token, head) in a fixed order.
// One wave per (token, head); D/64 output values per lane.
__global__ __launch_bounds__(256) void paged_combine_kernel(const float* __restrict__ part_o,
                                                            const float* __restrict__ part_m,
                                                            const float* __restrict__ part_z, int P, int tokens,
                                                            int hq, int D, float* __restrict__ out, int64_t o_st,
                                                            int64_t o_sh, float* __restrict__ lse) {
  const int wid = tid_x() >> 6, lane = tid_x() & 63;
  const int64_t th = (int64_t)bid_x() * 4 + wid;
  if (th >= (int64_t)tokens * hq) return;
  const int token = (int)(th / hq), h = (int)(th % hq);
  const int64_t stride = (int64_t)tokens * hq;
  float M = -INFINITY;
  for (int i = 0; i < P; ++i) M = fmaxf(M, part_m[i * stride + th]);
  float Z = 0.f;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  for (int i = 0; i < P; ++i) {
    const float mi = part_m[i * stride + th];
    const float w = mi > -INFINITY ? fast_exp2(mi - M) : 0.f;
    Z += w * part_z[i * stride + th];
    const float* po = part_o + (i * stride + th) * D;
#pragma unroll
    for (int s = 0; s < 4; ++s)
      if (64 * s < D) acc[s] += w * po[64 * s + lane];
  }
  const float inv = 1.f / Z;
  float* orow = out + (int64_t)token * o_st + (int64_t)h * o_sh;
#pragma unroll
  for (int s = 0; s < 4; ++s)
    if (64 * s < D) orow[64 * s + lane] = acc[s] * inv;
  if (lse && lane == 0) lse[th] = (M + __log2f(Z)) * kLn2;
}

// ---------------------------------------------------------------------------
// Generic paged kernel: one workgroup per (token, query head), any dtype / D.
struct GenericPagedParams {
  const void* q;
  int64_t q_st, q_sh;
  PagedRows rows;
  const void* tseq;
  const void* tpos;
  const int32_t* caps;
  int seq64, pos64;
  int num_seqs;
  int group, ws, wl, d;
  float scale;
  float* out;
  int64_t o_st, o_sh;
  float* lse;
  int hq;
};

template <typename QT, typename SCT, typename LCT>
__global__ __launch_bounds__(kGenThreads) void paged_generic_kernel(GenericPagedParams gp) {
  const int token = bid_x(), h = bid_y();
  PagedRows rows = gp.rows;
  rows.seq = clamp64(load_index(gp.tseq, token, gp.seq64), 0, gp.num_seqs - 1);
  const int pos = (int)load_index(gp.tpos, token, gp.pos64);
  int ws = gp.ws, wl = gp.wl;
  if (gp.caps) {
    ws = max(1, min(ws, gp.caps[2 * token]));
    wl = max(1, min(wl, gp.caps[2 * token + 1]));
  }
  const QT* q = (const QT*)gp.q + (int64_t)token * gp.q_st + (int64_t)h * gp.q_sh;
  float* out = gp.out + (int64_t)token * gp.o_st + (int64_t)h * gp.o_sh;
  float* lse = gp.lse ? gp.lse + (int64_t)token * gp.hq + h : nullptr;
  generic_query<QT, SCT, LCT, float>(q, rows, h / gp.group, pos, ws, wl, gp.d, gp.d, gp.scale, out, lse);
}

// ---------------------------------------------------------------------------
// Host side

int paged_mfma_supported(const sa_paged_args* a) {
  if (a->flags & SA_FLAG_FORCE_GENERIC) return 0;
  // bf16 caches; the query in bf16 or fp32 (fp32: hi/lo bf16 terms)
  if (a->cache_dtype != SA_DTYPE_BF16 || a->long_cache_dtype != SA_DTYPE_BF16) return 0;
  if (a->q_dtype != SA_DTYPE_BF16 && a->q_dtype != SA_DTYPE_F32) return 0;
  if (a->head_dim != 64 && a->head_dim != 128 && a->head_dim != 256) return 0;
  // 16-byte row alignment for the vector gathers
  const int64_t* s = a->sc_stride;
  const int64_t* l = a->lc_stride;
  for (int i = 0; i < 4; ++i)
    if ((s[i] % 8) || (l[i] % 8)) return 0;
  if ((a->q_stride_t % 8) || (a->q_stride_h % 8)) return 0;
  if (((uintptr_t)a->q | (uintptr_t)a->short_cache | (uintptr_t)a->long_cache) & 15) return 0;
  if (a->q_dtype == SA_DTYPE_F32 && a->head_dim > 128) return 0;  // registers: fp32 queries up to D = 128
  return 1;
}

static int paged_nw(const sa_paged_args* a) {
  const int tasks = (a->heads_q / a->heads_kv) * ((a->short_window + 31) / 32);
  return tasks >= 4 ? 4 : (tasks >= 2 ? 2 : 1);
}

// Expects windows already clipped to the tables' reach (sa_capi.hip), so the
// chunk count, and with it the split count and the workspace, stay bounded by
// the block-table capacity whatever window a global layer passes.
int paged_choose_splits(const sa_paged_args* a) {
  if (!paged_mfma_supported(a)) return 1;
  const int nc = (int)(((int64_t)a->long_window + kChunk - 1) / kChunk);
  if (a->splits > 0) return a->splits < nc ? a->splits : nc;
  const int group = a->heads_q / a->heads_kv;
  const int tasks = group * ((a->short_window + 31) / 32);
  const int nw = paged_nw(a);
  const int64_t wgs = (int64_t)a->tokens * a->heads_kv * ((tasks + nw - 1) / nw);
  const int64_t cus = device_cu_count();
  // Two resident workgroups per CU keep enough tile loads in flight; split
  // the long window only when (token, KV group) pairs alone cannot fill that.
  int64_t s = (2 * cus + wgs - 1) / wgs;
  // Long windows (more than 64 chunks) get one split per 64 chunks while the
  // grid stays within eight workgroups per CU: shorter workgroups balance
  // tokens whose valid windows differ in length.
  const int64_t s_long = ((int64_t)nc + 63) / 64, s_room = (8 * cus) / wgs;
  const int64_t s2 = s_long < s_room ? s_long : s_room;
  if (s2 > s) s = s2;
  const int64_t cap = nc / 2 > 0 ? nc / 2 : 1;  // at least 2 chunks per split
  if (s > cap) s = cap;
  return s < 1 ? 1 : (int)s;
}

size_t paged_workspace_bytes(const sa_paged_args* a, int splits) {
  if (!paged_mfma_supported(a)) return 0;
  if (splits * ((a->short_window + 31) / 32) == 1) return 0;  // direct output, no partials
  const size_t P = (size_t)splits * ((a->short_window + 31) / 32);
  const size_t th = (size_t)a->tokens * a->heads_q;
  size_t b = P * th * (size_t)a->head_dim * 4;
  b = (b + 255) & ~(size_t)255;
  size_t m = (P * th * 4 + 255) & ~(size_t)255;
  return b + 2 * m;
}

constexpr int kPagedDepth = 2;  // tiles in flight per workgroup (2 workgroups fit one CU)

template <int D, int NW, bool QF32>
static hipError_t launch_paged_mfma_t(PagedParams p, hipStream_t stream) {
  constexpr int P = D >= 256 ? 2 : kPagedDepth;
  // ring, row offsets, the short-row offsets and the staged q rows; the
  // epilogue's per-wave reduction area overlays the ring
  // a split holds at most ceil(nc / splits) chunks
  const bool multi = (p.nc + p.splits - 1) / p.splits > kSegChunks;
  // staged bf16 q rows (D <= 128, one segment) are also widened to fp32
  const bool widen = !QF32 && D <= 128 && !multi;
  const size_t qbytes = (size_t)NW * (QF32 ? 4 : 2) * D + (widen ? (size_t)NW * 4 * D : 0);
  const size_t lds_ring = (size_t)(P + 1) * FwdGeom<D, D, kChunk, NW>::SLOT + kPosCache * sizeof(int64_t) +
                          32 * sizeof(int64_t) + (qbytes + 1023) / 1024 * 1024;
  const size_t lds_red = (size_t)NW * 64 * 36 * sizeof(float);
  const size_t lds = lds_ring > lds_red ? lds_ring : lds_red;
  auto kern = multi ? paged_mfma_kernel<D, NW, P, true, QF32> : paged_mfma_kernel<D, NW, P, false, QF32>;
  hipError_t e = set_lds_limit((const void*)kern, lds);
  if (e != hipSuccess) return e;
  const int64_t nb = (int64_t)p.tokens * p.hk * p.splits * p.tblocks;
  hipLaunchKernelGGL(kern, dim3((unsigned)nb), dim3(64 * NW), lds, stream, p);
  return hipGetLastError();
}

template <int D, bool QF32>
static hipError_t launch_paged_mfma_d(const PagedParams& p, int nw, hipStream_t stream) {
  if (nw == 4) return launch_paged_mfma_t<D, 4, QF32>(p, stream);
  if (nw == 2) return launch_paged_mfma_t<D, 2, QF32>(p, stream);
  return launch_paged_mfma_t<D, 1, QF32>(p, stream);
}

// Portable kernel for one combination of query and cache element types
// (caches: fp32, bf16 or fp16, each axis on its own).
template <typename QT, typename SCT, typename LCT>
static hipError_t launch_paged_generic_t(const GenericPagedParams& gp, const sa_paged_args* a, size_t lds,
                                         hipStream_t stream) {
  auto kern = paged_generic_kernel<QT, SCT, LCT>;
  hipError_t e = set_lds_limit((const void*)kern, lds);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(kern, dim3(a->tokens, a->heads_q), dim3(kGenThreads), lds, stream, gp);
  return hipGetLastError();
}

template <typename QT, typename SCT>
static hipError_t launch_paged_generic_l(const GenericPagedParams& gp, const sa_paged_args* a, size_t lds,
                                         hipStream_t stream) {
  switch (a->long_cache_dtype) {
    case SA_DTYPE_F32: return launch_paged_generic_t<QT, SCT, float>(gp, a, lds, stream);
    case SA_DTYPE_F16: return launch_paged_generic_t<QT, SCT, _Float16>(gp, a, lds, stream);
    default: return launch_paged_generic_t<QT, SCT, bf16>(gp, a, lds, stream);
  }
}

template <typename QT>
static hipError_t launch_paged_generic_q(const GenericPagedParams& gp, const sa_paged_args* a, size_t lds,
                                         hipStream_t stream) {
  switch (a->cache_dtype) {
    case SA_DTYPE_F32: return launch_paged_generic_l<QT, float>(gp, a, lds, stream);
    case SA_DTYPE_F16: return launch_paged_generic_l<QT, _Float16>(gp, a, lds, stream);
    default: return launch_paged_generic_l<QT, bf16>(gp, a, lds, stream);
  }
}

hipError_t launch_paged(const sa_paged_args* a, int splits, void* ws, size_t ws_bytes, hipStream_t stream) {
  if (a->tokens == 0) return hipSuccess;
  if (paged_mfma_supported(a)) {
    PagedParams p{};
    p.q = a->q;
    p.q_st = a->q_stride_t;
    p.q_sh = a->q_stride_h;
    p.sc = (const bf16*)a->short_cache;
    p.lc = (const bf16*)a->long_cache;
    p.sc_a = a->sc_stride[0];
    p.sc_b = a->sc_stride[1];
    p.sc_s = a->sc_stride[2];
    p.sc_h = a->sc_stride[3];
    p.lc_a = a->lc_stride[0];
    p.lc_b = a->lc_stride[1];
    p.lc_s = a->lc_stride[2];
    p.lc_h = a->lc_stride[3];
    p.stable = a->short_table;
    p.ltable = a->long_table;
    p.st_s = a->st_stride;
    p.lt_s = a->lt_stride;
    p.tseq = a->token_seq;
    p.tpos = a->token_pos;
    p.stab64 = a->table_index_dtype == SA_INDEX_I64;
    p.ltab64 = a->long_table_index_dtype == SA_INDEX_I64;
    p.seq64 = a->token_index_dtype == SA_INDEX_I64;
    p.pos64 = a->token_pos_index_dtype == SA_INDEX_I64;
    p.st_w = a->short_table_width;
    p.lt_w = a->long_table_width;
    p.num_seqs = a->num_seqs;
    p.s_blocks = a->short_blocks;
    p.l_blocks = a->long_blocks;
    p.tokens = a->tokens;
    p.hq = a->heads_q;
    p.hk = a->heads_kv;
    p.group = a->heads_q / a->heads_kv;
    p.bs = a->block_size;
    p.ws = a->short_window;
    p.wl = a->long_window;
    p.nc = (int)(((int64_t)a->long_window + kChunk - 1) / kChunk);
    p.nr = (a->short_window + 31) / 32;
    p.sl2 = fmaxf(fabsf(a->scale) * kLog2e, 1e-30f);  // > 0: a masked score (-inf) maps to p = 0
    p.q_neg = a->scale < 0.f;
    p.splits = splits;
    p.tasks = p.group * p.nr;
    const int nw = paged_nw(a);
    p.tblocks = (p.tasks + nw - 1) / nw;
    const size_t P = (size_t)splits * p.nr;
    const size_t th = (size_t)a->tokens * a->heads_q;
    p.direct = P == 1;
    p.out = a->out;
    p.o_st = a->o_stride_t;
    p.o_sh = a->o_stride_h;
    p.lse = a->lse;
    p.caps = a->token_window_caps;
    if (!p.direct) {
      char* w = (char*)ws;
      size_t ob = (P * th * (size_t)a->head_dim * 4 + 255) & ~(size_t)255;
      size_t mb = (P * th * 4 + 255) & ~(size_t)255;
      if (ws_bytes < ob + 2 * mb || ((uintptr_t)ws & 255)) return hipErrorInvalidValue;
      p.part_o = (float*)w;
      p.part_m = (float*)(w + ob);
      p.part_z = (float*)(w + ob + mb);
    }
    hipError_t e;
    if (a->q_dtype == SA_DTYPE_F32) {
      e = a->head_dim == 64 ? launch_paged_mfma_d<64, true>(p, nw, stream)
                            : launch_paged_mfma_d<128, true>(p, nw, stream);
    } else {
      switch (a->head_dim) {
        case 64: e = launch_paged_mfma_d<64, false>(p, nw, stream); break;
        case 128: e = launch_paged_mfma_d<128, false>(p, nw, stream); break;
        default: e = launch_paged_mfma_d<256, false>(p, nw, stream); break;
      }
    }
    if (e != hipSuccess) return e;
    if (p.direct) return hipSuccess;
    const int64_t nth = (int64_t)a->tokens * a->heads_q;
    hipLaunchKernelGGL(paged_combine_kernel, dim3((unsigned)((nth + 3) / 4)), dim3(256), 0, stream, p.part_o,
                       p.part_m, p.part_z, (int)P, a->tokens, a->heads_q, a->head_dim, a->out, a->o_stride_t,
                       a->o_stride_h, a->lse);
    return hipGetLastError();
  }
  GenericPagedParams gp{};
  gp.q = a->q;
  gp.q_st = a->q_stride_t;
  gp.q_sh = a->q_stride_h;
  gp.rows.sc = a->short_cache;
  gp.rows.lc = a->long_cache;
  gp.rows.sc_a = a->sc_stride[0];
  gp.rows.sc_b = a->sc_stride[1];
  gp.rows.sc_s = a->sc_stride[2];
  gp.rows.sc_h = a->sc_stride[3];
  gp.rows.lc_a = a->lc_stride[0];
  gp.rows.lc_b = a->lc_stride[1];
  gp.rows.lc_s = a->lc_stride[2];
  gp.rows.lc_h = a->lc_stride[3];
  gp.rows.stable = a->short_table;
  gp.rows.ltable = a->long_table;
  gp.rows.st_s = a->st_stride;
  gp.rows.lt_s = a->lt_stride;
  gp.rows.stab64 = a->table_index_dtype == SA_INDEX_I64;
  gp.rows.ltab64 = a->long_table_index_dtype == SA_INDEX_I64;
  gp.rows.st_w = a->short_table_width;
  gp.rows.lt_w = a->long_table_width;
  gp.rows.s_blocks = a->short_blocks;
  gp.rows.l_blocks = a->long_blocks;
  gp.rows.block_size = a->block_size;
  gp.rows.seq = 0;
  gp.tseq = a->token_seq;
  gp.tpos = a->token_pos;
  gp.caps = a->token_window_caps;
  gp.seq64 = a->token_index_dtype == SA_INDEX_I64;
  gp.pos64 = a->token_pos_index_dtype == SA_INDEX_I64;
  gp.num_seqs = a->num_seqs;
  gp.group = a->heads_q / a->heads_kv;
  gp.ws = a->short_window;
  gp.wl = a->long_window;
  gp.d = a->head_dim;
  gp.scale = a->scale;
  gp.out = a->out;
  gp.o_st = a->o_stride_t;
  gp.o_sh = a->o_stride_h;
  gp.lse = a->lse;
  gp.hq = a->heads_q;
  const size_t lds = gen_lds_bytes(gp.d, gp.d);
  return a->q_dtype == SA_DTYPE_F32 ? launch_paged_generic_q<float>(gp, a, lds, stream)
                                    : launch_paged_generic_q<bf16>(gp, a, lds, stream);
}

}  // namespace sa
