// Prefill forward (dense [B,S,H,D] or packed variable-length) for the
// 2-simplicial attention library.  Replaces the reference's Triton _forward
// (archlab/architectures/simplicial_kernels.py:16-52) behind
// simplicial_attention (simplicial_attention.py:77-97).
//
// bf16 MFMA kernel (score width DK, value width DV: DK == DV in {64, 128, 256},
// or DK == 2 DV in {128, 256}, the determinant-score expansion)
// ------------------------------------------------------------------------------
// A workgroup of 4 waves owns NQ consecutive query tokens t0 .. t0+NQ-1 and
// NH query heads of one KV group (NQ * NH == 4).  Wave w handles token
// t0 + w / NH, head w % NH: its 32 A rows a_j = bf16(q_t ⊙ k1_j).  Every query
// walks its long window in 32-key chunks that start at t - long_window + 1,
// so ceil(long_window / 32) chunks cover it exactly.  Chunk c of the NQ
// queries together spans 32 + NQ - 1 keys; that K/V tile is loaded once per
// step and wave w reads it from row w / NH.  Tiles stream through a
// two-slot LDS ring by direct global->LDS DMA, one tile ahead of use, one
// barrier per step.  The A-row inputs (q, k1 rows) are read per lane from
// global memory.
//
// Score and value widths up to 128: the ring plus an area for the pass's v1
// rows is all the LDS the workgroup holds, so three workgroups share a CU
// (three waves per SIMD hide each other's barrier and load latencies).
// Widths of 256: 256 registers per wave, two waves per SIMD; the v1 rows use
// the ring slot that is free during the last chunk, so two workgroups share
// a CU.
//
// The joint softmax of a query and head has one running reference max per
// wave (all its rows belong to that query and head); the epilogue sums the
// rows against v1:  out = sum_j v1_j ⊙ O_j / sum_j z_j.  Short windows longer
// than 32 are processed in passes of 32 rows merged by their log-sum-exp
// weights.
#include "sa_generic.h"
#include "sa_mfma.h"
#include "sa_launch.h"

namespace sa {

struct PrefillParams {
  const void* q;   // bf16, or fp32 (F32 kernels)
  const void* k1;  // bf16, or fp32 (F32 kernels)
  const bf16* k2;  // F32 kernels: rows of [hi: D | lo: D] terms (split_hilo_kernel)
  const bf16* v1;  // likewise
  const bf16* v2;  // likewise
  void* out;       // bf16, or fp32 (F32 kernels)
  float* lse;
  const int32_t* cu;
  int64_t q_st, q_sh, k_st, k_sh, v_st, v_sh, o_st, o_sh, lse_st;
  int64_t k1_st, k1_sh;  // strides of k1 (those of k2 in the bf16 kernels)
  int total;      // tokens
  int seqlen;     // dense sequence length (cu == nullptr)
  int num_seqs;
  int hq, hk, group;
  int ws, wl;
  int nc;         // chunks per query: ceil(wl / 32)
  int nr;         // short row groups: ceil(ws / 32)
  float sl2;      // |scale| * log2(e)
  int q_neg;      // scale < 0
  int qblocks;    // query blocks per head group
  int hsub;       // head sub-groups per KV group (group / NH)
  int nblocks;    // total blocks
  FastDiv qbd, hsd, sld;  // division by qblocks, hsub and seqlen
};

constexpr int kPrefillWavesPerSimd = 3;  // widths <= 128, bf16
// V fragments read ahead of the PV MFMAs in the chunk loop (2 measured
// 0.1-0.9 % ahead of 3 and 4; at score width 512, one wave per SIMD, 4)
constexpr int kPrefillChunkPF = 2, kPrefillChunkPFWide = 4;

// One wave per (token, head), NQ x NH = 4 of them per workgroup; one K/V
// tile in flight (a two-slot ring).
// F32: fp32 inputs (the reference's fp32 path, tf32x3 dots, simplicial_kernels.py:42,48):
// q and k1 are read as fp32 and a = q ⊙ k1 is kept as hi + lo bf16 terms;
// k2, v2 and v1 arrive as rows of hi and lo terms, P is split the same way,
// and every product runs on three term pairs; the output is fp32.
template <int DK, int DV, int NQ, int NH, bool F32 = false>
// (score width 512, the determinant expansion of 256-wide heads: one wave per
// SIMD, the whole register file for 32 A fragments and 8 accumulator tiles)
__global__ __launch_bounds__(64 * NQ * NH, (DK >= 512 ? 1 : (DK >= 256 || DV >= 256 ? 2 : (F32 ? 2 : kPrefillWavesPerSimd))))
void prefill_mfma_kernel(PrefillParams p) {
  static_assert(NQ * NH == 4, "4 (token, head) pairs per block");
  constexpr int NW = NQ * NH;
  constexpr int ROWS = kChunk + NQ - 1;  // tile rows: one chunk of all NQ queries
  // F32 tile rows hold the hi and lo terms: twice the widths
  using G = FwdGeom<F32 ? 2 * DK : DK, F32 ? 2 * DV : DV, ROWS, NW>;
  // Widths of 256 (two waves per SIMD) and fp32 inputs' double-width tiles:
  // the pass's v1 rows go to the ring slot that is free during the last
  // chunk, so that the ring is all the LDS a workgroup holds and two
  // workgroups share a CU; widths up to 128 give them an area of their own
  // after the ring (three workgroups per CU).
  constexpr bool kV1Ring = F32 || DK >= 256 || DV >= 256;
  static_assert(!F32 || (DK <= 128 && DV <= 128), "fp32 inputs up to widths of 128");
  constexpr int R = 2;  // ring slots for the long-axis tiles: one tile in flight
  constexpr int NI = G::NI;
  extern __shared__ __attribute__((aligned(16))) char lds[];
  // The pass's v1 rows (rows kbs.. in the V-tile layout, read by the row
  // merge): placed so that their V region is the area after the ring (widths
  // up to 128; otherwise a ring slot chosen per pass, below).
  char* const v1slot = lds + R * G::SLOT - G::VOFF;
  // bf16: the A-row inputs are staged in LDS (k1 rows in the K region, q rows
  // in the V region of a free ring slot) at every width; fp32 inputs form A
  // from global memory
  constexpr bool kStageA = !F32;

  const int tid = tid_x();
  const int lane = tid & 63;
  // wave index as a uniform (scalar) value: everything derived from it stays
  // in SGPRs and the control flow below stays scalar
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int hw = wid % NH, qo = wid / NH;  // (token, head) of this wave in the block

  const int lb = xcd_remap(bid_x(), p.nblocks);
  const int hg = fdiv(lb, p.qbd);  // = g * hsub + hs
  const int qb = lb - hg * p.qblocks;
  const int g = fdiv(hg, p.hsd), hs = hg - g * p.hsub;
  const int t0 = qb * NQ;
  if (t0 >= p.total) return;
  // sequence starts of the block's tokens: one lookup for t0, shared by the
  // tokens before the next sequence (a block straddles a start rarely)
  int snext;
  const int sblk = seq_span(p.cu, p.num_seqs, p.seqlen, p.sld, t0, snext);
  auto start_of = [&](int tw) {  // tw >= t0
    int unused;
    return tw < snext ? sblk : seq_span(p.cu, p.num_seqs, p.seqlen, p.sld, tw, unused);
  };

  // per-wave scalars (readfirstlane pins them to SGPRs)
  const int t = __builtin_amdgcn_readfirstlane(t0 + qo);
  const bool qvalid = t < p.total;
  const int h = __builtin_amdgcn_readfirstlane(g * p.group + hs * NH + hw);
  const int s0 = qvalid ? start_of(t) : 0;
  const int lo2 = __builtin_amdgcn_readfirstlane(max(s0, t - p.wl + 1));
  const int lo1 = __builtin_amdgcn_readfirstlane(max(s0, t - p.ws + 1));
  const int cfirst = __builtin_amdgcn_readfirstlane(qvalid ? (lo2 - (t - p.wl + 1)) / kChunk : p.nc);
  int c0 = p.nc;  // first step in which any query of the block has a valid key
#pragma unroll
  for (int w = 0; w < NQ; ++w) {
    const int tw = t0 + w;
    if (tw < p.total) {
      const int sw = start_of(tw);
      c0 = min(c0, (max(sw, tw - p.wl + 1) - (tw - p.wl + 1)) / kChunk);
    }
  }
  c0 = __builtin_amdgcn_readfirstlane(c0);

  const int kb0 = t0 - p.wl + 1;  // key of tile row 0 at chunk 0
  const int last = p.total - 1;
  const int64_t k_st = p.k_st, v_st = p.v_st;
  const int64_t k_g = (int64_t)g * p.k_sh, v_g = (int64_t)g * p.v_sh;

  // Per lane and DMA instruction: byte offset of its 16 bytes from the tile's
  // first row (interior tiles: uniform base + this offset).
  // Decoded per wave index, so that each instruction's tensor and row
  // stride are compile-time values (row divisions by constants).
  uint32_t voff[NI];
  static_for<0, NW>([&](auto wc) {
    constexpr int W = decltype(wc)::value;
    if (wid == W) {
#pragma unroll
      for (int k = 0; k < NI; ++k) {
        int is_v, row, seg;
        G::decode(W, k, lane, is_v, row, seg);
        voff[k] = ((uint32_t)row * (uint32_t)(is_v ? v_st : k_st) + (uint32_t)seg * 8u) * 2u;
      }
    }
  });
  // DMA of one tile of rows kb .. kb+ROWS-1 into `slot`: the K region from
  // tensor kt (k strides), the V region from vt (v strides).  PART selects
  // both regions (0), the K region only (1) or the V region only (2).
  auto dma_tile = [&](auto part_c, char* slot, int kb_in, const bf16* kt, const bf16* vt) {
    constexpr int PART = decltype(part_c)::value;
    const int kb = __builtin_amdgcn_readfirstlane(kb_in);  // uniform: scalar test and tile bases
    if (kb >= 0 && kb + ROWS - 1 <= last) {
      const char* kbase = (const char*)(kt + (int64_t)kb * k_st + k_g);
      const char* vbase = (const char*)(vt + (int64_t)kb * v_st + v_g);
#pragma unroll
      for (int k = 0; k < NI; ++k) {
        const bool is_v = G::instr_is_v(wid, k);
        if ((PART == 1 && is_v) || (PART == 2 && !is_v)) continue;
        // the empty asm keeps the 32-bit offsets from being widened outside the
        // loop (held as 64-bit pairs they cost NI more VGPRs, which the
        // allocator then spills)
        uint32_t o = voff[k];
        asm volatile("" : "+v"(o));
        dma16(uniform_ptr(is_v ? vbase : kbase) + o, G::dst(slot, wid, k));
      }
    } else {  // tile crosses the tensor edge: clamp every row into [0, total)
      // rows and segments derived afresh from the lane id: hoisted out of the
      // loops, the per-instruction row offsets and row pointers of this rare
      // path took registers the allocator then spilled
      const int lf = fresh_lane();
#pragma unroll
      for (int k = 0; k < NI; ++k) {
        int is_v, row, seg;
        G::decode(wid, k, lf, is_v, row, seg);
        if ((PART == 1 && G::instr_is_v(wid, k)) || (PART == 2 && !G::instr_is_v(wid, k))) continue;
        const int64_t key = min(max(kb + row, 0), last);
        const bf16* src = is_v ? vt + key * v_st + v_g : kt + key * k_st + k_g;
        dma16(src + seg * 8, G::dst(slot, wid, k));
      }
    }
  };
  auto slot_of = [&](int c) { return lds + ((unsigned)c % (unsigned)R) * G::SLOT; };
  auto issue = [&](int c) { dma_tile(std::integral_constant<int, 0>{}, slot_of(c), kb0 + kChunk * c, p.k2, p.v2); };
  // OT layout: the output accumulators hold O (lane = d, registers = rows)
  using RB = RowBlock<DK, DV, F32, true, F32>;
  RB rb;
  // Running merge over the row-group passes: out values of this wave's columns
  // d = 64*i + lane (half 0: d block 2i, half 1: block 2i+1; live through the
  // key loops, so one copy, not one per half), plus (M, Z) in the log2 domain.
  static_assert(DV % 64 == 0, "value columns in pairs of 32-wide blocks");
  float orun[DV / 64];
#pragma unroll
  for (int i = 0; i < DV / 64; ++i) orun[i] = 0.f;
  float Mrun = -INFINITY, Zrun = 0.f;

  for (int r = 0; r < p.nr; ++r) {
    // Passes alternate the direction of their chunk walk (even passes
    // ascending, odd ones descending), so that every pass after the first
    // starts on the tile the previous one ended with, still in its ring slot:
    // no DMA and no wait for it.  The direction changes only the order of the
    // online softmax's sums, which is fixed for a given shape.
    const bool rev = (r & 1) != 0;                // uniform
    const int cf = rev ? p.nc - 1 : c0;           // first chunk of the pass
    const int cl = rev ? c0 : p.nc - 1;           // last chunk of the pass
    const bool resident = r > 0 && c0 < p.nc;     // first tile already in LDS
    // widths of 256 / fp32: the pass's v1 rows go to the slot that does not
    // hold its last chunk (free while that chunk is processed)
    char* const v1s = kV1Ring ? slot_of(cl + 1) : v1slot;
    // lane-derived values from a fresh lane index: computed per pass, not
    // kept (or spilled) through the key loops of a multi-pass query
    const int lp = fresh_lane();
    const int n = lp & 31, half = lp >> 5;
    const int j = t - 32 * r - n;  // this lane's short-axis key
    const bool row_ok = qvalid && j >= lo1;
    const int jc = min(max(j, 0), last);  // a readable row for every lane
    // Pass prologue: the v1 rows (widths up to 128), the first tile and the
    // A-row inputs go out together; A is formed once the inputs have landed.
    const int kbs = t0 - 31 - 32 * r;  // v1 row 0 (short key of tile row 0)
    if constexpr (!kV1Ring) {
      // the pass's v1 rows into their own area, ahead of the first tiles (the
      // in-order completion of this wave's loads makes the chunk loop's
      // waits cover them)
      dma_tile(std::integral_constant<int, 2>{}, v1slot, kbs, p.k2, p.v1);
    }
    // bf16: the block's k1 rows (rows kbs.., the K region of the ring slot
    // that tile c0+1 fills only after the key loop's first barrier) and its q
    // rows (that slot's V region) are staged once per block by DMA ahead of
    // the first tile, and the A rows are formed from LDS while the tile
    // streams (vector loads would retire behind the tile's DMA, and each wave
    // would fetch its own overlapping k1 rows)
    char* const kslot = slot_of(cf + 1);
    char* const qslot = kslot + G::VOFF;
    if constexpr (kStageA) {
      dma_tile(std::integral_constant<int, 1>{}, kslot, kbs, (const bf16*)p.k1, p.v1);
      if (wid == 0) {
        constexpr int kQI = (NQ * NH * 2 * DK + 1023) / 1024;
        // addresses from a fresh lane id: the same in every pass, they were
        // hoisted out of the pass loop and spilled at widths of 256
        const int lq = fresh_lane();
#pragma unroll
        for (int k = 0; k < kQI; ++k) {
          const int b = 1024 * k + 16 * lq;
          const int pr = min(b / (2 * DK), NQ * NH - 1), seg = (b % (2 * DK)) / 16;  // pair (query, head)
          const int tq = min(t0 + pr / NH, last), hq = g * p.group + hs * NH + pr % NH;
          dma16((const bf16*)p.q + (int64_t)tq * p.q_st + (int64_t)hq * p.q_sh + 8 * seg, qslot + b);
        }
      }
    }
    if (!resident) issue(cf);
    if constexpr (kStageA) {
      // the staged rows (the first tile, when issued, may still be in flight)
      if (resident) wait_vmcnt<0>();
      else wait_vmcnt<G::NI>();
      block_barrier();
      // the wave's q row widened to fp32 after the staged rows (same slot
      // region), then lane n's k1 row j = t - 32r - n is slot row qo + 31 - n;
      // rows outside the window are masked
      char* const qf = qslot + NQ * NH * 2 * DK + wid * 4 * DK;
      static_assert(NQ * NH * 6 * DK <= G::SLOT - G::VOFF, "staged and widened q rows fit the V region");
      RB::widen_q(qslot + wid * 2 * DK, qf, fresh_lane(), p.q_neg != 0);
      rb.form_a_qf(kslot + (qo + 31 - n) * G::RSK, qf, row_ok, half);
    } else {
      // fp32 inputs: A formed in fp32 from the rows in global memory and split
      // into hi/lo terms
      static_assert(F32, "bf16 A-row inputs are staged");
      const int64_t qoff = (int64_t)min(t, last) * p.q_st + (int64_t)h * p.q_sh;
      const int64_t k1off = (int64_t)jc * p.k1_st + (int64_t)g * p.k1_sh;
      rb.form_a_f32((const float*)p.q + qoff, (const float*)p.k1 + k1off, row_ok, half, p.q_neg != 0);
    }
    rb.reset(row_ok);
    {
      // Tile addresses of the chunk issued next, advanced by one chunk per
      // step (no 64-bit multiply in the loop); used when the tile lies inside
      // the tensor, the general tile DMA otherwise.
      const int dir = rev ? -1 : 1;
      const int64_t kstep = dir * (int64_t)kChunk * k_st * 2, vstep = dir * (int64_t)kChunk * v_st * 2;
      int kbn = kb0 + kChunk * (cf + dir);  // key of the next tile's row 0
      const char* kn = (const char*)(p.k2 + k_g) + (int64_t)kbn * k_st * 2;
      const char* vn = (const char*)(p.v2 + v_g) + (int64_t)kbn * v_st * 2;
      const int nsteps = p.nc - c0;
      for (int i = 0; i < nsteps; ++i) {
        const int c = cf + dir * i;
        wait_vmcnt<0>();
        block_barrier();  // tile c complete for every wave; slot of the previous tile free
        if (i + 1 < nsteps) {
          char* const ns = slot_of(c + dir);
          if (kbn >= 0 && kbn + ROWS - 1 <= last) {
            // buffer loads into LDS: scalar descriptors for the two tiles and
            // the 32-bit per-lane offsets as they are (no 64-bit address)
            const __amdgpu_buffer_rsrc_t rk = raw_rsrc(kn), rv = raw_rsrc(vn);
#pragma unroll
            for (int k = 0; k < NI; ++k)
              dma16_buf(G::instr_is_v(wid, k) ? rv : rk, voff[k], G::dst(ns, wid, k));
          } else {
            issue(c + dir);
          }
        }
        kbn += dir * kChunk;
        kn += kstep;
        vn += vstep;
        if constexpr (kV1Ring)
          if (i + 1 == nsteps) dma_tile(std::integral_constant<int, 2>{}, v1s, kbs, p.k2, p.v1);  // v1 rows
        // Unconditional: a wave without valid keys in this step gets an empty
        // key range (every p = 0, an exact no-op).  A branch here would give
        // the accumulators two incoming values at the loop latch, which the
        // register allocator resolves by keeping a second copy of all of O.
        const bool active = qvalid && c >= cfirst;
        // the pass's first chunk with a valid key for this wave: cfirst when
        // ascending, the last chunk (it holds key t) when descending.  Widths
        // of 256 only (C4 -0.9 %): over 16 chunks at widths up to 128 the
        // per-chunk test cost as much as it saved (NS +0.2 %, C3 +0.9 %), and
        // the first chunk there computes its probabilities twice instead.
        const bool first = (DK >= 256 || DV >= 256) && qvalid && c == (rev ? p.nc - 1 : cfirst);
        const int kfirst = t - p.wl + 1 + kChunk * c;  // key of this wave's chunk row 0
        const char* slot = slot_of(c);
        rb.template chunk<G::RSK, G::RSV, (DK >= 512 ? kPrefillChunkPFWide : kPrefillChunkPF)>(slot, slot + G::VOFF, qo, lane, p.sl2,
                                                               active ? max(lo2 - kfirst, 0) : kChunk,
                                                               active ? min(t - kfirst, kChunk - 1) : -1, first);
      }
      if constexpr (kV1Ring)
        if (nsteps <= 0) dma_tile(std::integral_constant<int, 2>{}, v1s, kbs, p.k2, p.v1);
    }
    wait_vmcnt<0>();  // this wave's part of the v1 rows
    block_barrier();  // ring reads done; v1 rows complete

    // ---- epilogue of this pass.  One reference max for the wave's rows, so
    // the joint softmax of the pass is  out = sum_n v1_n ⊙ O_n / sum_n z_n:
    // with O in the OT layout each lane sums its 16 rows (registers) for its
    // column d, then adds the other half's 16 rows.  The v1 values come from
    // the staged rows by transposing reads: group g of 4 reads rows
    // n = 8g + 4*half + e (e = 0..3), short-slot row qo + 31 - n.
    const float Zw = uniform_f(half_sum(pair_sum(rb.z)));  // rows outside the window hold z = 0
    const bool any_row = __builtin_amdgcn_ballot_w64(row_ok) != 0ull;
    const float Mw = any_row ? uniform_f(rb.m) : -INFINITY;
    const float Mn = fmaxf(Mrun, Mw);
    const float a0 = Mrun > -INFINITY ? fast_exp2(Mrun - Mn) : 0.f;
    const float a1 = Mw > -INFINITY ? fast_exp2(Mw - Mn) : 0.f;
    // rows n < nv lie inside the short window (p = 0 outside: those rows are
    // dropped from the sum also when a stale v1 row is not finite)
    const int nv = qvalid ? min(32, t - 32 * r - lo1 + 1) : 0;
    // lane-derived addresses from a fresh lane index: computed here, not
    // hoisted and kept live (or spilled) through the key loop
    const int lf = fresh_lane();
    const int hf = lf >> 5, g16 = (lf >> 4) & 1, i16 = lf & 15;
    const uint32_t v1p = lds_addr(v1s + G::VOFF + (qo + 7 - 4 * hf - (i16 >> 2)) * G::RSV + 32 * g16 +
                                  8 * (i16 & 3));
    static_for<0, DV / 32>([&](auto dd) {
      constexpr int db = decltype(dd)::value;
      shortx4 x[4], xl[F32 ? 4 : 1];
      static_for<0, 4>([&](auto gg) {
        constexpr int g = decltype(gg)::value;
        x[g] = ds_read_tr16<(24 - 8 * g) * G::RSV + 64 * db>(v1p);
        if constexpr (F32) xl[g] = ds_read_tr16<(24 - 8 * g) * G::RSV + 64 * db + 2 * DV>(v1p);  // lo terms
      });
      lds_wait(x[0], x[1]);
      lds_wait(x[2], x[3]);
      if constexpr (F32) {
        lds_wait(xl[0], xl[1]);
        lds_wait(xl[2], xl[3]);
      }
      // v1 value of row 8g + 4*half + e (hi + lo terms for fp32 inputs)
      auto v1val = [&](int g, int e) {
        float v = bf16_bits_to_f32(x[g][e]);
        if constexpr (F32) v += bf16_bits_to_f32(xl[g][e]);
        return v;
      };
      float acc = 0.f;
      if (nv >= 32) {
#pragma unroll
        for (int g = 0; g < 4; ++g)
#pragma unroll
          for (int e = 0; e < 4; ++e) acc = fmaf(v1val(g, e), rb.o[db][4 * g + e], acc);
      } else {
        // an opaque copy of nv keeps the row tests inside this rare branch
        // (speculated above it, they would run in every pass)
        int nvm = nv;
        asm volatile("" : "+s"(nvm));
#pragma unroll
        for (int g = 0; g < 4; ++g)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float v = (8 * g + 4 * hf + e < nvm) ? v1val(g, e) : 0.f;
            acc = fmaf(v, rb.o[db][4 * g + e], acc);
          }
      }
      // both halves hold the sum for column 32*db + lane % 32; the half of
      // block db's parity keeps it
      const float upd = orun[db >> 1] * a0 + pair_sum(acc) * a1;
      orun[db >> 1] = hf == (db & 1) ? upd : orun[db >> 1];
    });
    Zrun = uniform_f(Zrun * a0 + Zw * a1);
    Mrun = uniform_f(Mn);
    if (r + 1 < p.nr) block_barrier();  // every wave's v1 reads done before the next pass refills the slots
  }

  if (qvalid) {
    // half 0 stores the even 32-wide blocks, half 1 the odd ones
    const float inv = 1.f / Zrun;
    using OT_ = std::conditional_t<F32, float, bf16>;
    OT_* orow = (OT_*)p.out + (int64_t)t * p.o_st + (int64_t)h * p.o_sh;
    const int lf = fresh_lane();
#pragma unroll
    for (int i = 0; i < DV / 64; ++i) orow[64 * i + lf] = (OT_)(orun[i] * inv);
    if (p.lse && lf == 0) p.lse[(int64_t)t * p.lse_st + h] = (Mrun + __log2f(Zrun)) * kLn2;
  }
}

// ---------------------------------------------------------------------------
// Generic (portable) prefill kernel: one workgroup per (token, query head).
template <typename T>
__global__ __launch_bounds__(kGenThreads) void prefill_generic_kernel(GenericPrefillParams gp) {
  const int t = bid_x();
  const int h = bid_y();
  const int s0 = seq_start(gp.cu, gp.num_seqs, gp.seqlen, t);
  const int g = h / gp.group;
  DenseRows rows{gp.k1, gp.k2, gp.v1, gp.v2, gp.k_st, gp.k_sh, gp.v_st, gp.v_sh, (int64_t)s0};
  const T* q = (const T*)gp.q + (int64_t)t * gp.q_st + (int64_t)h * gp.q_sh;
  T* out = (T*)gp.out + (int64_t)t * gp.o_st + (int64_t)h * gp.o_sh;
  float* lse = gp.lse ? gp.lse + (int64_t)t * gp.lse_st + h : nullptr;
  generic_query<T, T, T, T>(q, rows, g, t - s0, gp.ws, gp.wl, gp.d, gp.dv, gp.scale, out, lse);
}

// ---------------------------------------------------------------------------
// Host launchers

// fp32 rows [tokens][heads][d] (element strides st_t, st_h; 16-byte aligned
// rows) -> bf16 rows [tokens][heads][hi: d | lo: d] with hi + lo = x to 2^-17
// relative (split_bf16).  One thread per 4 consecutive values.
__global__ __launch_bounds__(256) void split_hilo_kernel(const float* __restrict__ src, int64_t st_t, int64_t st_h,
                                                         int64_t rows, int heads, int d, bf16* __restrict__ dst) {
  const int64_t i = (int64_t)bid_x() * 256 + tid_x();
  const int per = d / 4;
  const int64_t row = i / per;
  if (row >= rows) return;
  const int c = (int)(i % per) * 4;
  const int64_t t = row / heads, h = row % heads;
  const floatx4 x = *(const floatx4*)(src + t * st_t + h * st_h + c);
  bf16x4 hi, lo;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    bf16 xh, xl;
    split_bf16(x[e], xh, xl);
    hi[e] = xh;
    lo[e] = xl;
  }
  bf16* o = dst + row * 2 * d;
  *(bf16x4*)(o + c) = hi;
  *(bf16x4*)(o + d + c) = lo;
}

template <int DK, int DV, int NQ, int NH, bool F32 = false>
static hipError_t launch_prefill_mfma(const PrefillParams& base_p, hipStream_t stream) {
  PrefillParams p = base_p;
  p.qblocks = (p.total + NQ - 1) / NQ;
  p.hsub = p.group / NH;
  p.nblocks = p.qblocks * p.hk * p.hsub;
  p.qbd = make_fastdiv(p.qblocks);
  p.hsd = make_fastdiv(p.hsub);
  p.sld = make_fastdiv(p.seqlen > 0 ? p.seqlen : 1);
  constexpr int NW = NQ * NH;
  using G = FwdGeom<F32 ? 2 * DK : DK, F32 ? 2 * DV : DV, kChunk + NQ - 1, NW>;
  constexpr bool kV1Ring = F32 || DK >= 256 || DV >= 256;
  // two ring slots, then (widths up to 128) the v1 area: 50 KB per workgroup
  // at D = 128 (three per CU), 80 KB at D = 256 (two per CU)
  // ring; v1 rows (a slot's V region: its DMA spans SLOT - VOFF bytes, the
  // slot's instruction count being rounded to the waves) below widths of 256
  const size_t lds = (size_t)2 * G::SLOT + (kV1Ring ? (size_t)0 : (size_t)(G::SLOT - G::VOFF));
  auto kern = prefill_mfma_kernel<DK, DV, NQ, NH, F32>;
  hipError_t e = set_lds_limit((const void*)kern, lds);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(kern, dim3(p.nblocks), dim3(64 * NW), lds, stream, p);
  return hipGetLastError();
}

// Blocking by the group size: four heads of one KV group per token, two
// tokens x two heads, or four tokens of one head.
template <int DK, int DV>
static hipError_t dispatch_prefill_mfma_d(const PrefillParams& p, hipStream_t stream) {
  const int G = p.group;
  if (G % 4 == 0) return launch_prefill_mfma<DK, DV, 1, 4>(p, stream);
  if (G % 2 == 0) return launch_prefill_mfma<DK, DV, 2, 2>(p, stream);
  return launch_prefill_mfma<DK, DV, 4, 1>(p, stream);
}

// fp32 inputs: double-width tiles, two workgroups per CU
template <int D>
static hipError_t dispatch_prefill_mfma_f32(const PrefillParams& p, hipStream_t stream) {
  const int G = p.group;
  if (G % 4 == 0) return launch_prefill_mfma<D, D, 1, 4, true>(p, stream);
  if (G % 2 == 0) return launch_prefill_mfma<D, D, 2, 2, true>(p, stream);
  return launch_prefill_mfma<D, D, 4, 1, true>(p, stream);
}

hipError_t launch_split_hilo(const float* src, int64_t st_t, int64_t st_h, int64_t tokens, int heads, int d,
                             bf16* dst, hipStream_t stream) {
  const int64_t rows = tokens * heads;
  if (rows == 0) return hipSuccess;
  const unsigned blocks = (unsigned)((rows * (d / 4) + 255) / 256);
  hipLaunchKernelGGL(split_hilo_kernel, dim3(blocks), dim3(256), 0, stream, src, st_t, st_h, rows, heads, d, dst);
  return hipGetLastError();
}

size_t prefill_f32_workspace_bytes(const sa_prefill_args* a) {
  // k2, v2 and v1 as rows of hi and lo bf16 terms: 4 bytes per element each
  const size_t e = (size_t)a->total_tokens * a->heads_kv * a->head_dim;
  return ((3 * e * 4) + 255) & ~(size_t)255;
}

hipError_t launch_prefill_mfma(const sa_prefill_args* a, hipStream_t stream) {
  const bool f32 = a->dtype == SA_DTYPE_F32;
  PrefillParams p{};
  p.q = a->q;
  p.k1 = a->k1;
  p.k2 = (const bf16*)a->k2;
  p.v1 = (const bf16*)a->v1;
  p.v2 = (const bf16*)a->v2;
  p.out = a->out;
  p.lse = a->lse;
  p.cu = a->cu_seqlens;
  p.q_st = a->q_stride_t;
  p.q_sh = a->q_stride_h;
  p.k_st = a->k_stride_t;
  p.k_sh = a->k_stride_h;
  p.v_st = a->v_stride_t;
  p.v_sh = a->v_stride_h;
  p.k1_st = a->k_stride_t;
  p.k1_sh = a->k_stride_h;
  p.o_st = a->o_stride_t;
  p.o_sh = a->o_stride_h;
  p.lse_st = a->lse_stride_t;
  p.total = a->total_tokens;
  p.seqlen = a->seqlen;
  p.num_seqs = a->num_seqs;
  p.hq = a->heads_q;
  p.hk = a->heads_kv;
  p.group = a->heads_q / a->heads_kv;
  p.ws = a->short_window;
  p.wl = a->long_window;
  p.nc = (a->long_window + kChunk - 1) / kChunk;
  p.nr = (a->short_window + 31) / 32;
  // > 0 even for scale == 0, so that a masked score (-inf) maps to p = 0
  p.sl2 = fmaxf(fabsf(a->scale) * kLog2e, 1e-30f);
  p.q_neg = a->scale < 0.f;
  const int dk = a->head_dim, dv = a->value_dim;
  if (f32) {
    // split k2, v2, v1 into rows of hi and lo terms in the workspace, then run
    // the fp32 kernel on them (k1 and q are read as fp32 by the kernel)
    const int64_t rows = (int64_t)a->total_tokens * a->heads_kv;
    const int64_t e = rows * dk;
    bf16* k2s = (bf16*)a->workspace;
    bf16* v2s = k2s + 2 * e;
    bf16* v1s = v2s + 2 * e;
    const unsigned blocks = (unsigned)((rows * (dk / 4) + 255) / 256);
    hipLaunchKernelGGL(split_hilo_kernel, dim3(blocks), dim3(256), 0, stream, (const float*)a->k2, a->k_stride_t,
                       a->k_stride_h, rows, a->heads_kv, dk, k2s);
    hipLaunchKernelGGL(split_hilo_kernel, dim3(blocks), dim3(256), 0, stream, (const float*)a->v2, a->v_stride_t,
                       a->v_stride_h, rows, a->heads_kv, dk, v2s);
    hipLaunchKernelGGL(split_hilo_kernel, dim3(blocks), dim3(256), 0, stream, (const float*)a->v1, a->v_stride_t,
                       a->v_stride_h, rows, a->heads_kv, dk, v1s);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
    p.k2 = k2s;
    p.v2 = v2s;
    p.v1 = v1s;
    p.k_st = p.v_st = (int64_t)a->heads_kv * 2 * dk;
    p.k_sh = p.v_sh = 2 * dk;
    if (dk == 64) return dispatch_prefill_mfma_f32<64>(p, stream);
    if (dk == 128) return dispatch_prefill_mfma_f32<128>(p, stream);
    return hipErrorInvalidValue;
  }
  if (dk == dv) {
    switch (dk) {
      case 64: return dispatch_prefill_mfma_d<64, 64>(p, stream);
      case 128: return dispatch_prefill_mfma_d<128, 128>(p, stream);
      case 256: return dispatch_prefill_mfma_d<256, 256>(p, stream);
      default: return hipErrorInvalidValue;
    }
  }
  if (dk == 128 && dv == 64) return dispatch_prefill_mfma_d<128, 64>(p, stream);
  if (dk == 256 && dv == 128) return dispatch_prefill_mfma_d<256, 128>(p, stream);
  if (dk == 512 && dv == 256) return dispatch_prefill_mfma_d<512, 256>(p, stream);
  return hipErrorInvalidValue;
}

hipError_t launch_prefill_generic(const sa_prefill_args* a, hipStream_t stream) {
  GenericPrefillParams gp{};
  gp.q = a->q;
  gp.k1 = a->k1;
  gp.k2 = a->k2;
  gp.v1 = a->v1;
  gp.v2 = a->v2;
  gp.out = a->out;
  gp.lse = a->lse;
  gp.cu = a->cu_seqlens;
  gp.q_st = a->q_stride_t;
  gp.q_sh = a->q_stride_h;
  gp.k_st = a->k_stride_t;
  gp.k_sh = a->k_stride_h;
  gp.v_st = a->v_stride_t;
  gp.v_sh = a->v_stride_h;
  gp.o_st = a->o_stride_t;
  gp.o_sh = a->o_stride_h;
  gp.lse_st = a->lse_stride_t;
  gp.seqlen = a->seqlen;
  gp.num_seqs = a->num_seqs;
  gp.group = a->heads_q / a->heads_kv;
  gp.ws = a->short_window;
  gp.wl = a->long_window;
  gp.d = a->head_dim;
  gp.dv = a->value_dim;
  gp.scale = a->scale;
  const size_t lds = gen_lds_bytes(gp.d, gp.dv);
  dim3 grid(a->total_tokens, a->heads_q);
  if (a->dtype == SA_DTYPE_F32) {
    auto kern = prefill_generic_kernel<float>;
    hipError_t e = set_lds_limit((const void*)kern, lds);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(kern, grid, dim3(kGenThreads), lds, stream, gp);
  } else {
    auto kern = prefill_generic_kernel<bf16>;
    hipError_t e = set_lds_limit((const void*)kern, lds);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(kern, grid, dim3(kGenThreads), lds, stream, gp);
  }
  return hipGetLastError();
}

}  // namespace sa
