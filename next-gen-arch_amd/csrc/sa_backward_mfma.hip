// MFMA backward passes of the 2-simplicial prefill (bf16, score width ==
// value width D in {64, 128}).  Same mathematics, rounding points and
// atomics-free three-pass split as the portable kernels of sa_backward.hip
// (archlab/architectures/simplicial_kernels.py:55-106), on 32x32x16 bf16 MFMA
// tiles:
//
// Per query t, head h, short key j, long key k (a_j = bf16(q ⊙ k1_j),
// b_j = bf16(dout ⊙ v1_j), P = exp(scale a_j·k2_k - lse_t)):
//   dq pass   (one wave per (t, h), 32 rows j; K2/V2 tiles stream through LDS)
//     S^T  = K2 · A^T,  dP^T = V2 · B^T          (keys x j)
//     dS   = bf16(P (dP - delta_t) scale)
//     dA^T += K2^T · dS^T                        (d x j; transposing K reads)
//     dq_t = Σ_j dA_j ⊙ k1_j
//     with one or two 32-row groups of short keys, also dk1: per row group
//     the NQ queries x NH heads of a workgroup write a partial Σ dA_{t,j} ⊙
//     q_{t,h} for their 31 + NQ short keys j, and a fixed-order sum over the
//     partials holding each key gives dk1 (dA_{t,j} is the dk1 pass's
//     G_{t,j}); the dk1 pass below is then not launched
//   dk1/dv1 pass (one wave per (j, h); its 32 rows are the queries
//   t = j + 32r + n whose short window holds j; tiles span the rows' union of
//   long windows, masked per row)
//     S^T, dP^T, dS as above (A rows q_t ⊙ k1_j, B rows dout_t ⊙ v1_j)
//     G^T  += K2^T · dS^T,  O''^T += V2^T · bf16(P)^T     (d x t)
//     dk1_j = Σ_h Σ_t G_t ⊙ q_t,   dv1_j = Σ_h Σ_t O''_t ⊙ dout_t
//   dk2/dv2 pass (one wave per 32 long keys, their K2/V2 rows held as MFMA
//   fragments; the workgroup streams every (t, h) that reaches its keys and
//   builds that step's A_t / B_t rows (32 short keys j) in LDS)
//     S^T = A_t · K2^T, dP^T = B_t · V2^T                (j x keys)
//     dK2^T += A_t^T · dS^T,  dV2^T += B_t^T · bf16(P)^T  (d x keys)
//
// The tile machinery (LDS ring filled by global->LDS DMA, TileGeom layouts,
// the transposing-read accumulation) is the forward kernel's (sa_mfma.h).
#include "sa_mfma.h"
#include "sa_launch.h"
#include "sa_backward.h"

namespace sa {

namespace {

// LDS fragments read ahead of their MFMA in each pass (see BwdOps; dq two
// ahead at widths up to 128: NS forward + backward 17.05 -> 16.96 ms, the
// adapter shape 8.85 -> 8.74 ms); at score width 256 (one wave per SIMD: no
// other wave hides the LDS latency) the dq and dk2 / dv2 passes read further
// ahead (C4 forward + backward 29.1 -> 28.7 and 28.9 ms)
constexpr int kDqPF = 2, kDqPFWide = 3;      // dq pass
constexpr int kDk1PF = 1;                    // dk1 / dv1 pass (dv1 reads two ahead)
constexpr int kDkv2PF = 2, kDkv2PFWide = 4;  // dk2 / dv2 pass

constexpr size_t kLdsPerCu = 160 * 1024;  // gfx950
constexpr int kMaxWalkSplits = 8;         // dk2 / dv2 walk pieces per (key block, KV head)

// Wave-level tile products used by the backward passes (D = head dim).
template <int D>
struct BwdOps {
  using RB = RowBlock<D, D>;

  // C = Tile · X^T over D: A operand = tile rows row0 .. row0+31 (row stride
  // RS bytes), B operand = the fragments x[D/16] (one 32-row block, k = d).
  // Lane (n, half) receives C[tile row 8*(r/4) + 4*half + r%4][x row n].
  // PF: fragments read that many MFMAs ahead (more LDS latency hidden per
  // wave, 4 VGPRs each).
  template <int RS, int PF = 1>
  __device__ static __forceinline__ floatx16 rows_x(const char* tile, int row0, int lane, const bf16x8* x) {
    const int n = lane & 31, half = lane >> 5;
    const char* kp = tile + (row0 + n) * RS + 16 * half;
    floatx16 c = floatx16{};
    if constexpr (PF > 1) {
      // explicit reads and counted waits (the compiler's waits for plain
      // loads here would also wait for the reads issued ahead)
      const uint32_t ka = lds_addr(kp);
      bf16x8 f[D / 16];
      static_for<0, (PF < D / 16 ? PF : D / 16)>(
          [&](auto s) { f[s] = ds_read_b128_at<32 * decltype(s)::value>(ka); });
      static_for<0, D / 16>([&](auto st) {
        constexpr int s = decltype(st)::value;
        if constexpr (s + PF < D / 16) f[s + PF] = ds_read_b128_at<32 * (s + PF)>(ka);
        lds_wait_k<(s + PF < D / 16 ? s + PF : D / 16 - 1) - s>(f[s]);  // reads issued after f[s]'s
        __builtin_amdgcn_sched_barrier(0);
        c = mfma32x32x16(f[s], x[s], c);
        __builtin_amdgcn_sched_barrier(0);
      });
      return c;
    }
    // fragments are read one step ahead of their MFMA; the scheduling barriers
    // keep the compiler from hoisting all D/16 reads (D/4 more live VGPRs)
    bf16x8 f = *(const bf16x8*)kp;
#pragma unroll
    for (int t = 0; t < D / 16; ++t) {
      bf16x8 fn;
      if (t + 1 < D / 16) fn = *(const bf16x8*)(kp + 32 * (t + 1));
      __builtin_amdgcn_sched_barrier(0);
      c = mfma32x32x16(f, x[t], c);
      __builtin_amdgcn_sched_barrier(0);
      f = fn;
    }
    return c;
  }

  // acc[db] += Tile^T · PB: A operand = the tile's rows row0 .. row0+31
  // transposed (d x rows, read with ds_read_b64_tr_b16), B operand = {pb0,
  // pb1}: the 32 x 32 values of a rows_x result (rows x columns) packed by
  // pack_c.  acc[db] holds d = 32*db + acc_row(r, half), column lane % 32.
  // OT: the same product with the operands swapped, (PB^T · Tile): acc[db]
  // holds column d = 32*db + lane % 32 and, in register r, the rows_x column
  // (x row) 8*(r/4) + 4*half + r%4.
  // PF: transposed reads issued that many MFMAs ahead.
  template <int RS, int PF = 1, bool OT = false>
  __device__ static __forceinline__ void tr_acc(floatx16* acc, const char* tile, int row0, int lane,
                                                const bf16x8& pb0, const bf16x8& pb1) {
    auto mm = [](const bf16x8& v, const bf16x8& b, const floatx16& c) {
      if constexpr (OT) return mfma32x32x16(b, v, c);
      else return mfma32x32x16(v, b, c);
    };
    const int half = lane >> 5, g16 = (lane >> 4) & 1, i16 = lane & 15;
    const int e_src = i16 >> 2, q_src = i16 & 3;
    const uint32_t vp = lds_addr(tile + (row0 + 4 * half + e_src) * RS + 32 * g16 + 8 * q_src);
    constexpr int kSteps = 2 * (D / 32);
    if constexpr (PF > 1) {
      shortx4 va[kSteps], vb[kSteps];
      static_for<0, (PF < kSteps ? PF : kSteps)>([&](auto s) { RB::template vread<RS, s>(vp, va[s], vb[s]); });
      static_for<0, kSteps>([&](auto st) {
        constexpr int s = decltype(st)::value;
        if constexpr (s + PF < kSteps) RB::template vread<RS, s + PF>(vp, va[s + PF], vb[s + PF]);
        // reads issued after step s's: 2 per later step in flight
        constexpr int later = (s + PF < kSteps ? s + PF : kSteps - 1) - s;
        lds_wait_n<2 * later>(va[s], vb[s]);
        shortx8 vv = {va[s][0], va[s][1], va[s][2], va[s][3], vb[s][0], vb[s][1], vb[s][2], vb[s][3]};
        const bf16x8 vf = __builtin_bit_cast(bf16x8, vv);
        __builtin_amdgcn_sched_barrier(0);
        acc[s % (D / 32)] = mm(vf, s / (D / 32) == 0 ? pb0 : pb1, acc[s % (D / 32)]);
        __builtin_amdgcn_sched_barrier(0);
      });
      return;
    }
    shortx4 v1, v2;
    RB::template vread<RS, 0>(vp, v1, v2);
    lds_wait(v1, v2);
    static_for<0, kSteps>([&](auto st) {
      constexpr int step = decltype(st)::value;
      shortx8 vv = {v1[0], v1[1], v1[2], v1[3], v2[0], v2[1], v2[2], v2[3]};
      const bf16x8 vf = __builtin_bit_cast(bf16x8, vv);
      shortx4 n1, n2;
      if constexpr (step + 1 < kSteps) RB::template vread<RS, step + 1>(vp, n1, n2);
      __builtin_amdgcn_sched_barrier(0);
      acc[step % (D / 32)] = mm(vf, step / (D / 32) == 0 ? pb0 : pb1, acc[step % (D / 32)]);
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (step + 1 < kSteps) {
        lds_wait(n1, n2);
        v1 = n1;
        v2 = n2;
      }
    });
  }

  // 16 C-layout values (rows x this lane's column) -> the B operand of tr_acc
  // (bf16, round to nearest even).
  __device__ static __forceinline__ void pack_c(const float* x, bf16x8& pb0, bf16x8& pb1) {
    uint32_t pk[8];
#pragma unroll
    for (int r = 0; r < 16; r += 2) pk[r >> 1] = pack_bf16(x[r], x[r + 1]);
    pb0 = __builtin_bit_cast(bf16x8, u32x4{pk[0], pk[1], pk[2], pk[3]});
    pb1 = __builtin_bit_cast(bf16x8, u32x4{pk[4], pk[5], pk[6], pk[7]});
  }

  // ---- fp32 inputs: every operand as hi + lo bf16 terms (split_bf16), each
  // product on three term pairs (hi·hi + hi·lo + lo·hi), as the forward's
  // fp32 path; the reference computes these dots with tf32x3
  // (simplicial_kernels.py:75-101).  Tile rows hold [hi: D | lo: D].

  // rows_x with hi/lo tile rows and hi (x) / lo (xl) fragments
  template <int RS>
  __device__ static __forceinline__ floatx16 rows_x_hl(const char* tile, int row0, int lane, const bf16x8* x,
                                                       const bf16x8* xl) {
    const int n = lane & 31, half = lane >> 5;
    const uint32_t ka = lds_addr(tile + (row0 + n) * RS + 16 * half);
    floatx16 c = floatx16{};
    // hi and lo fragments read two steps ahead with counted waits (the
    // compiler's own waits would also wait for the reads issued ahead)
    constexpr int T = D / 16, KA = T < 2 ? T : 2;
    bf16x8 fh[T], fl[T];
    auto rd = [&](auto tt) {
      constexpr int t = decltype(tt)::value;
      fh[t] = ds_read_b128_at<32 * t>(ka);
      fl[t] = ds_read_b128_at<2 * D + 32 * t>(ka);
    };
    static_for<0, KA>([&](auto tt) { rd(tt); });
    static_for<0, T>([&](auto tt) {
      constexpr int t = decltype(tt)::value;
      if constexpr (t + KA < T) rd(std::integral_constant<int, t + KA>{});
      constexpr int later = 2 * ((t + KA < T ? t + KA : T - 1) - t);  // reads issued after step t's pair
      lds_wait_k<later + 1>(fh[t]);
      lds_wait_k<later>(fl[t]);
      __builtin_amdgcn_sched_barrier(0);
      c = mfma32x32x16(fh[t], x[t], c);
      c = mfma32x32x16(fh[t], xl[t], c);
      c = mfma32x32x16(fl[t], x[t], c);
      __builtin_amdgcn_sched_barrier(0);
    });
    return c;
  }

  // tr_acc with hi/lo tile rows and the B operand as hi (pb0, pb1) and lo
  // (pl0, pl1) terms
  template <int RS>
  __device__ static __forceinline__ void tr_acc_hl(floatx16* acc, const char* tile, int row0, int lane,
                                                   const bf16x8& pb0, const bf16x8& pb1, const bf16x8& pl0,
                                                   const bf16x8& pl1) {
    const int half = lane >> 5, g16 = (lane >> 4) & 1, i16 = lane & 15;
    const int e_src = i16 >> 2, q_src = i16 & 3;
    const uint32_t vp = lds_addr(tile + (row0 + 4 * half + e_src) * RS + 32 * g16 + 8 * q_src);
    constexpr int kSteps = 2 * (D / 32);
    // the fragments of step s+1 are read while step s's MFMAs run (the fp32
    // passes hold one wave per SIMD: nothing else hides the LDS latency)
    shortx4 h1[kSteps], h2[kSteps], l1[kSteps], l2[kSteps];
    auto rd = [&](auto st) {
      constexpr int s = decltype(st)::value;
      RB::template vread<RS, s>(vp, h1[s], h2[s]);
      RB::template vread<RS, s, 2 * D>(vp, l1[s], l2[s]);
    };
    rd(std::integral_constant<int, 0>{});
    static_for<0, kSteps>([&](auto st) {
      constexpr int s = decltype(st)::value;
      if constexpr (s + 1 < kSteps) rd(std::integral_constant<int, s + 1>{});
      constexpr int later = s + 1 < kSteps ? 4 : 0;  // reads issued after step s's
      lds_wait_n<later>(h1[s], h2[s]);
      lds_wait_n<later>(l1[s], l2[s]);
      const bf16x8 vh =
          __builtin_bit_cast(bf16x8, shortx8{h1[s][0], h1[s][1], h1[s][2], h1[s][3], h2[s][0], h2[s][1], h2[s][2], h2[s][3]});
      const bf16x8 vl =
          __builtin_bit_cast(bf16x8, shortx8{l1[s][0], l1[s][1], l1[s][2], l1[s][3], l2[s][0], l2[s][1], l2[s][2], l2[s][3]});
      const bf16x8& bh = s / (D / 32) == 0 ? pb0 : pb1;
      const bf16x8& bl = s / (D / 32) == 0 ? pl0 : pl1;
      __builtin_amdgcn_sched_barrier(0);
      acc[s % (D / 32)] = mfma32x32x16(vh, bh, acc[s % (D / 32)]);
      acc[s % (D / 32)] = mfma32x32x16(vh, bl, acc[s % (D / 32)]);
      acc[s % (D / 32)] = mfma32x32x16(vl, bh, acc[s % (D / 32)]);
      __builtin_amdgcn_sched_barrier(0);
    });
  }

  // pack_c with the low-order terms: x = hi + lo to 2^-17 relative
  __device__ static __forceinline__ void pack_c_hl(const float* x, bf16x8& pb0, bf16x8& pb1, bf16x8& pl0,
                                                   bf16x8& pl1) {
    uint32_t ph[8], pl[8];
#pragma unroll
    for (int r = 0; r < 16; r += 2) pack_bf16_split(x[r], x[r + 1], ph[r >> 1], pl[r >> 1]);
    pb0 = __builtin_bit_cast(bf16x8, u32x4{ph[0], ph[1], ph[2], ph[3]});
    pb1 = __builtin_bit_cast(bf16x8, u32x4{ph[4], ph[5], ph[6], ph[7]});
    pl0 = __builtin_bit_cast(bf16x8, u32x4{pl[0], pl[1], pl[2], pl[3]});
    pl1 = __builtin_bit_cast(bf16x8, u32x4{pl[4], pl[5], pl[6], pl[7]});
  }

  // A^T fragments (hi a, lo al) of rows x ⊙ y from fp32 rows in LDS: lane
  // (n, half) holds d = 16t + 8 half .. +7 of its row; zero where !valid
  __device__ static __forceinline__ void form_hl_lds(const char* xrow, const char* yrow, bool valid, int half,
                                                     bf16x8* a, bf16x8* al) {
#pragma unroll
    for (int t = 0; t < D / 16; ++t) {
      const int d0 = 16 * t + 8 * half;
      const floatx4 x0 = *(const floatx4*)(xrow + 4 * d0), x1 = *(const floatx4*)(xrow + 4 * d0 + 16);
      const floatx4 y0 = *(const floatx4*)(yrow + 4 * d0), y1 = *(const floatx4*)(yrow + 4 * d0 + 16);
      bf16x8 h, l;
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const float v = valid ? (u < 4 ? x0[u] * y0[u] : x1[u - 4] * y1[u - 4]) : 0.f;
        bf16 vh, vl;
        split_bf16(v, vh, vl);
        h[u] = vh;
        l[u] = vl;
      }
      a[t] = h;
      al[t] = l;
    }
  }
};

struct BwdGeo {
  int nc;       // long-axis chunks per query: ceil(wl / 32)
  int nr;       // short-axis row groups: ceil(ws / 32)
  int qblocks;  // query blocks per head group
  int hsub;     // head sub-groups per KV group
  int nblocks;
};

// ---------------------------------------------------------------------------
// dq: a workgroup of 4 waves owns NQ consecutive queries x NH heads of one KV
// group (the forward kernel's blocking); chunk c of the NQ queries' long
// windows is one K2/V2 tile of 32 + NQ - 1 rows.
// FUSE (one or two row groups): the pass also writes the block's dk1
// partials, per row group r Σ over its NQ queries and NH heads of dA_{t,j} ⊙
// q_{t,h} for the short keys j = t0 - 32 r - 31 .. t0 - 32 r + NQ - 1 (the dk1
// pass's G_{t,j} is the same dA_{t,j}).
// F32: fp32 inputs (DK == DV <= 128): K2 / V2 tiles from the hi/lo rows
// (p.k2s, p.v2s), the short slot and the q / dout rows hold fp32 rows (the
// same bytes as a hi/lo row), A and B are split from fp32 products, and every
// product runs on three term pairs; dq (and dk1) in fp32.
// FV (fp32 inputs with FUSE; one wave per SIMD either way): the pass also
// accumulates O''^T += V2^T · P^T per chunk and writes the block's dv1
// partials, Σ O''_{t,j} ⊙ dout_{t,h} over the same rows as dk1's, so that no
// dk1 / dv1 pass recomputes S.
template <int DK, int DV, int NQ, int NH, int P, bool FUSE = false, bool F32 = false, bool FV = false>
__global__ __launch_bounds__(64 * NQ * NH, (DK > 128 || F32) ? 1 : 2) void bwd_dq_mfma_kernel(BwdParams p,
                                                                                            BwdGeo geo) {
  static_assert(NQ * NH == 4, "4 waves per block");
  static_assert(!FV || (F32 && FUSE && DK == DV), "dv1 partials: fp32 inputs, with the dk1 partials");
  static_assert(!F32 || (DK == DV && DK <= 128), "fp32 inputs: equal widths up to 128");
  constexpr int NW = NQ * NH;
  constexpr int ROWS = kChunk + NQ - 1;
  constexpr int EW = F32 ? 2 : 1;  // bf16 units per element of an LDS row (fp32 rows, hi/lo tile rows)
  using G = TileGeom<EW * DK, EW * DV, ROWS, NW, 32, 32>;
  using OPK = BwdOps<DK>;  // products over the score width
  using OPV = BwdOps<DV>;  // ... over the value width
  constexpr int R = P + 1;
  constexpr int NI = G::NI;
  constexpr int kPF = DK >= 256 ? kDqPFWide : kDqPF;
  // dA with the lane on d (the MFMA operands swapped) at score width 256: the
  // epilogue sums the rows in registers instead of through a per-wave LDS
  // transpose of 128 values per lane (C4 forward + backward 28.35 -> 27.6 ms);
  // at widths up to 128 the row layout's 16-byte staging writes of the dk1
  // partials measured ahead (adapter shape 8.8 against 9.0 ms)
  constexpr bool kOT = !F32 && DK >= 256;
  // ring of R tile slots, also the per-wave reduction scratch of the epilogue
  constexpr int RING = R * G::SLOT > NW * 64 * 36 * 4 ? R * G::SLOT : NW * 64 * 36 * 4;
  extern __shared__ __attribute__((aligned(16))) char lds[];
  char* const sslot = lds + RING;         // k1 rows (K region), v1 rows (V region) of the pass
  char* const qslot = sslot + G::SLOT;    // q rows 0..NW-1 (row stride RSK), then NW dout rows (RSV)

  const int tid = tid_x(), lane = tid & 63;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int hw = wid % NH, qo = wid / NH;
  const int half = lane >> 5, n = lane & 31;

  const int lb = xcd_remap(bid_x(), geo.nblocks);
  const int qb = lb % geo.qblocks;
  const int hg = lb / geo.qblocks;
  const int g = hg / geo.hsub, hs = hg % geo.hsub;
  const int t0 = qb * NQ;
  if (t0 >= p.tokens) return;

  const int t = __builtin_amdgcn_readfirstlane(t0 + qo);
  const bool qvalid = t < p.tokens;
  const int h = __builtin_amdgcn_readfirstlane(g * p.group + hs * NH + hw);
  const int s0 = qvalid ? seq_start(p.cu, p.num_seqs, p.seqlen, t) : 0;
  const int lo2 = __builtin_amdgcn_readfirstlane(max(s0, t - p.wl + 1));
  const int lo1 = __builtin_amdgcn_readfirstlane(max(s0, t - p.ws + 1));
  const int cfirst = __builtin_amdgcn_readfirstlane(qvalid ? (lo2 - (t - p.wl + 1)) / kChunk : geo.nc);
  int c0 = geo.nc;  // first step in which any query of the block has a valid key
#pragma unroll
  for (int w = 0; w < NQ; ++w) {
    const int tw = t0 + w;
    if (tw < p.tokens) {
      const int sw = seq_start(p.cu, p.num_seqs, p.seqlen, tw);
      c0 = min(c0, (max(sw, tw - p.wl + 1) - (tw - p.wl + 1)) / kChunk);
    }
  }
  c0 = __builtin_amdgcn_readfirstlane(c0);

  const int kb0 = t0 - p.wl + 1;  // key of tile row 0 at chunk 0
  const int last = p.tokens - 1;
  // strides in bf16 units: the long-axis tiles (bf16 tensors, or the fp32
  // inputs' hi/lo rows [tokens][hk][2 D]) and the short slot (bf16 tensors,
  // or fp32 rows viewed as two bf16 units per element)
  const int64_t k_st = F32 ? (int64_t)p.hk * 2 * DK : p.k_st, v_st = F32 ? (int64_t)p.hk * 2 * DV : p.v_st;
  const int64_t k_g = F32 ? (int64_t)g * 2 * DK : (int64_t)g * p.k_sh;
  const int64_t v_g = F32 ? (int64_t)g * 2 * DV : (int64_t)g * p.v_sh;
  const int64_t ks_st = EW * p.k_st, vs_st = EW * p.v_st;
  const int64_t ks_g = EW * (int64_t)g * p.k_sh, vs_g = EW * (int64_t)g * p.v_sh;
  const bf16* const k1 = (const bf16*)p.k1;
  const bf16* const k2 = F32 ? p.k2s : (const bf16*)p.k2;
  const bf16* const v1 = (const bf16*)p.v1;
  const bf16* const v2 = F32 ? p.v2s : (const bf16*)p.v2;

  uint32_t voff[NI];
#pragma unroll
  for (int k = 0; k < NI; ++k) {
    int is_v, row, seg;
    G::decode(wid, k, lane, is_v, row, seg);
    voff[k] = (uint32_t)(((int64_t)row * (is_v ? v_st : k_st) + seg * 8) * 2);
  }
  // One tile of rows kb .. kb+ROWS-1: K region from kt, V region from vt
  // (row strides kst / vst, head offsets kg / vg, in bf16 units).
  auto dma_tile = [&](char* slot, int kb_in, const bf16* kt, const bf16* vt, int64_t kst, int64_t vst, int64_t kg,
                      int64_t vg, bool same_strides) {
    const int kb = __builtin_amdgcn_readfirstlane(kb_in);
    if (same_strides && kb >= 0 && kb + ROWS - 1 <= last) {
      const char* kbase = (const char*)(kt + (int64_t)kb * kst + kg);
      const char* vbase = (const char*)(vt + (int64_t)kb * vst + vg);
#pragma unroll
      for (int k = 0; k < NI; ++k)
        dma16(uniform_ptr(G::instr_is_v(wid, k) ? vbase : kbase) + voff[k], G::dst(slot, wid, k));
    } else {  // the tile crosses the tensor edge: clamp every row into [0, tokens)
      // rows derived afresh from the lane id (not hoisted into live registers)
      const int lf = fresh_lane();
#pragma unroll
      for (int k = 0; k < NI; ++k) {
        int is_v, row, seg;
        G::decode(wid, k, lf, is_v, row, seg);
        const int64_t key = min(max(kb + row, 0), last);
        const bf16* src = is_v ? vt + key * vst + vg : kt + key * kst + kg;
        dma16(src + seg * 8, G::dst(slot, wid, k));
      }
    }
  };
  auto issue = [&](int c) {
    dma_tile(lds + (c % R) * G::SLOT, kb0 + kChunk * c, k2, v2, k_st, v_st, k_g, v_g, true);
  };
  // q and dout rows of the NW (query, head) pairs (wave 0; QI instructions)
  constexpr int QI = (NW * (G::RSK + G::RSV) + 1023) / 1024;
  auto dma_qd = [&]() {
    if (wid == 0) {
#pragma unroll
      for (int k = 0; k < QI; ++k) {
        const int b = k * 1024 + lane * 16;
        const bool isd = b >= NW * G::RSK;  // the dout rows follow the q rows
        const int bb = isd ? b - NW * G::RSK : b, rs = isd ? G::RSV : G::RSK;
        int row = bb / rs, seg = (bb % rs) >> 4;
        if (row >= NW || seg >= (isd ? G::kSegsV : G::kSegsK)) row = 0, seg = 0;
        const int tq = min(t0 + row / NH, last);
        const int hq = g * p.group + hs * NH + row % NH;
        const bf16* src = isd ? (const bf16*)p.dout + EW * ((int64_t)tq * p.do_st + (int64_t)hq * p.do_sh)
                              : (const bf16*)p.q + EW * ((int64_t)tq * p.q_st + (int64_t)hq * p.q_sh);
        dma16(src + seg * 8, qslot + k * 1024);
      }
    }
  };

  const int64_t th = (int64_t)min(t, last) * p.hq + h;
  const float lse2 = qvalid ? p.lse[(int64_t)min(t, last) * p.lse_st + h] * kLog2e : 0.f;
  const float delta = qvalid ? p.delta[th] : 0.f;
  const float dl = qvalid ? p.dl[th] : 0.f;
  const bool single = t == s0 || (p.ws == 1 && p.wl == 1);  // one valid pair: only the LSE-gradient term
  const float sl2s = p.scale * kLog2e;
  // dS = P (dP - delta) scale, or P dlse scale for a single pair: P (dP dpm + dsm)
  const float dpm = single ? 0.f : p.scale;
  const float dsm = single ? dl * p.scale : -delta * p.scale;

  RowBlock<DK, DV, F32> ra;  // A rows (q ⊙ k1); only the fragments are used
  RowBlock<DV, DV, F32> rbv;  // B rows (dout ⊙ v1)
  float dqrun[DK / 64];
#pragma unroll
  for (int i = 0; i < DK / 64; ++i) dqrun[i] = 0.f;

  for (int r = 0; r < geo.nr; ++r) {
    const int j = t - 32 * r - n;  // this lane's short-axis key
    const bool row_ok = qvalid && j >= lo1;
    const float lse2r = row_ok ? lse2 : INFINITY;  // exp2(x - inf) = 0: rows outside the window
    const int kbs = t0 - 31 - 32 * r;  // short-slot row 0
    dma_tile(sslot, kbs, k1, v1, ks_st, vs_st, ks_g, vs_g, !F32);
    if (r == 0) dma_qd();
#pragma unroll
    for (int e = 0; e < P; ++e) issue(c0 + e);  // unconditional: static count for the wait below
    wait_vmcnt<P * NI>();
    block_barrier();
    const int srow = qo + 31 - n;  // row of key j in the short slot
    if constexpr (F32) {
      OPK::form_hl_lds(sslot + srow * G::RSK, qslot + wid * G::RSK, row_ok, half, ra.a, ra.al);
      OPV::form_hl_lds(sslot + G::VOFF + srow * G::RSV, qslot + NW * G::RSK + wid * G::RSV, row_ok, half, rbv.a,
                       rbv.al);
    } else {
      ra.form_a_lds(sslot + srow * G::RSK, qslot + wid * G::RSK, row_ok, half, false);
      rbv.form_a_lds(sslot + G::VOFF + srow * G::RSV, qslot + NW * G::RSK + wid * G::RSV, row_ok, half, false);
    }

    floatx16 dA[DK / 32];
#pragma unroll
    for (int i = 0; i < DK / 32; ++i) dA[i] = floatx16{};
    floatx16 dO[FV ? DV / 32 : 1];  // O''^T (dv1 partials)
#pragma unroll
    for (int i = 0; i < (FV ? DV / 32 : 1); ++i) dO[i] = floatx16{};
    for (int c = c0; c < geo.nc; ++c) {
      wait_tiles<NI, P>(min(P - 1, geo.nc - 1 - c));
      block_barrier();  // tile c complete for every wave; the slot of tile c-1 is free
      if (c + P < geo.nc) issue(c + P);
      const bool active = qvalid && c >= cfirst;
      const int kfirst = t - p.wl + 1 + kChunk * c;  // key of this wave's chunk row 0
      const int klo = active ? max(lo2 - kfirst, 0) : kChunk;
      const int khi = active ? min(t - kfirst, kChunk - 1) : -1;
      const char* slot = lds + (c % R) * G::SLOT;
      floatx16 s, dp;
      if constexpr (F32) {
        s = OPK::template rows_x_hl<G::RSK>(slot, qo, lane, ra.a, ra.al);
        dp = OPV::template rows_x_hl<G::RSV>(slot + G::VOFF, qo, lane, rbv.a, rbv.al);
      } else {
        s = OPK::template rows_x<G::RSK, kPF>(slot, qo, lane, ra.a);
        dp = OPV::template rows_x<G::RSV, kPF>(slot + G::VOFF, qo, lane, rbv.a);
      }
      // register r holds chunk key 8*(r/4) + r%4 + 4*half of column j = this lane's row
      const int lo_h = klo - 4 * half, hi_h = khi - 4 * half;
      float ds[16], pv[FV ? 16 : 1];  // dS, and (FV) P
      if (klo <= 0 && khi >= kChunk - 1) {  // every key of the chunk valid (uniform test)
        // rows outside the window: exp2(s*c - inf) = 0 with no per-key test
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const float pr = fast_exp2(fmaf(s[e], sl2s, -lse2r));
          if constexpr (FV) pv[e] = pr;
          ds[e] = pr * fmaf(dp[e], dpm, dsm);
        }
      } else {
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int kr = 8 * (e >> 2) + (e & 3);
          const bool ok = row_ok && kr >= lo_h && kr <= hi_h;
          const float pr = ok ? fast_exp2(fmaf(s[e], sl2s, -lse2)) : 0.f;
          if constexpr (FV) pv[e] = pr;
          ds[e] = pr * fmaf(dp[e], dpm, dsm);
        }
      }
      bf16x8 pb0, pb1;
      if constexpr (F32) {
        bf16x8 pl0, pl1;
        OPK::pack_c_hl(ds, pb0, pb1, pl0, pl1);
        OPK::template tr_acc_hl<G::RSK>(dA, slot, qo, lane, pb0, pb1, pl0, pl1);  // dA^T += K2^T · dS^T
        if constexpr (FV) {
          OPK::pack_c_hl(pv, pb0, pb1, pl0, pl1);
          OPV::template tr_acc_hl<G::RSV>(dO, slot + G::VOFF, qo, lane, pb0, pb1, pl0, pl1);  // O''^T += V2^T · P^T
        }
      } else {
        OPK::pack_c(ds, pb0, pb1);
        OPK::template tr_acc<G::RSK, kPF, kOT>(dA, slot, qo, lane, pb0, pb1);  // dA^T += K2^T · dS^T (kOT: dA, lane = d)
      }
    }
    wait_vmcnt<0>();
    block_barrier();  // ring reads done (LDS reused below)

    // rows n of the wave inside the short window: n < nv (j = t - 32 r - n >= lo1)
    const int nv = qvalid ? min(32, t - 32 * r - lo1 + 1) : 0;
    if constexpr (!kOT) {
      // dq[d] += Σ_j dA_j[d] k1_j[d] over the wave's 32 rows (dA^T: lane = row)
      float* red = (float*)lds + wid * (64 * 36);  // [64 d][36] per wave (ring region)
      const char* k1s = sslot + srow * G::RSK;     // this lane's k1 row
      floatx4 kv[DK / 64][2][4];
#pragma unroll
      for (int sl = 0; sl < DK / 64; ++sl)
#pragma unroll
        for (int dbl = 0; dbl < 2; ++dbl)
#pragma unroll
          for (int q4 = 0; q4 < 4; ++q4) {
            const int dd = 64 * sl + 32 * dbl + 8 * q4 + 4 * half;
            if constexpr (F32) {
              kv[sl][dbl][q4] = *(const floatx4*)(k1s + 4 * dd);
            } else {
              const bf16x4 kb = *(const bf16x4*)(k1s + 2 * dd);
#pragma unroll
              for (int e = 0; e < 4; ++e) kv[sl][dbl][q4][e] = (float)kb[e];
            }
          }
#pragma unroll
      for (int sl = 0; sl < DK / 64; ++sl) {
#pragma unroll
        for (int dbl = 0; dbl < 2; ++dbl) {
          const int db = 2 * sl + dbl;
#pragma unroll
          for (int q4 = 0; q4 < 4; ++q4) {
            const int dd = 32 * dbl + 8 * q4 + 4 * half;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const float k = row_ok ? kv[sl][dbl][q4][e] : 0.f;
              red[(dd + e) * 36 + n] = k * dA[db][4 * q4 + e];
            }
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
        dqrun[sl] += acc;
      }
    } else {
      // dA (lane = d) holds column d = 32 db + lane % 32 and, in register
      // 4 g + e, row n = 8 g + 4 half + e (short-slot row qo + 31 - n): dq[d] =
      // Σ_n dA_n[d] k1_n[d] in registers over the 16 rows of this half, the k1
      // values read transposed from the short slot, plus the other half's sum.
      // Rows outside the window hold dA = 0; in a partial window they are also
      // dropped from the sum (a k1 row outside it need not be finite).
      const int lf = fresh_lane();
      const int hf = lf >> 5, g16 = (lf >> 4) & 1, i16 = lf & 15;
      const uint32_t k1p = lds_addr(sslot + (qo + 7 - 4 * hf - (i16 >> 2)) * G::RSK + 32 * g16 + 8 * (i16 & 3));
      // the k1 values of block db + 1 are read while block db is summed
      shortx4 xb[DK / 32][4];
      auto read_k1 = [&](auto dd) {
        constexpr int db = decltype(dd)::value;
        static_for<0, 4>([&](auto gg) {
          constexpr int gi = decltype(gg)::value;
          xb[db][gi] = ds_read_tr16<(24 - 8 * gi) * G::RSK + 64 * db>(k1p);
        });
      };
      read_k1(std::integral_constant<int, 0>{});
      static_for<0, DK / 32>([&](auto dd) {
        constexpr int db = decltype(dd)::value;
        if constexpr (db + 1 < DK / 32) read_k1(std::integral_constant<int, db + 1>{});
        shortx4* const x = xb[db];
        constexpr int kLater = db + 1 < DK / 32 ? 4 : 0;  // reads issued after block db's
        lds_wait_n<kLater>(x[0], x[1]);
        lds_wait_n<kLater>(x[2], x[3]);
        float acc = 0.f;
        if (nv >= 32) {
#pragma unroll
          for (int g4 = 0; g4 < 4; ++g4)
#pragma unroll
            for (int e = 0; e < 4; ++e) acc = fmaf(bf16_bits_to_f32(x[g4][e]), dA[db][4 * g4 + e], acc);
        } else {
          // an opaque copy of nv keeps the row tests inside this rare branch
          int nvm = nv;
          asm volatile("" : "+s"(nvm));
#pragma unroll
          for (int g4 = 0; g4 < 4; ++g4)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const float k = 8 * g4 + 4 * hf + e < nvm ? bf16_bits_to_f32(x[g4][e]) : 0.f;
              acc = fmaf(k, dA[db][4 * g4 + e], acc);
            }
        }
        // both halves hold column d's sum; the half of block db's parity keeps it
        const float tot = pair_sum(acc);
        dqrun[db >> 1] = hf == (db & 1) ? dqrun[db >> 1] + tot : dqrun[db >> 1];
      });
    }
    block_barrier();  // every wave's short-slot (and `red`) reads done before the next pass (or exit) reuses the LDS

    if constexpr (FUSE) {
      // dk1 (and, FV, dv1) partial: row n of wave (qo, hw) is short key j = t0 + qo - 32 r - n,
      // partial row jrow = qo + 31 - n.  Per 64-wide d half, each wave stages
      // its 32 rows x 64 d products (rows of 68 floats), then the block sums
      // every (jrow, 4 d) over its waves in wave order and writes it.
      constexpr int PRS = 68;                   // staged row stride (floats)
      constexpr int ROWS1 = 31 + NQ;            // partial rows
      // 64-wide d halves staged per round: two where the ring region holds
      // them (widths of 256: half the rounds, barriers and LDS latencies; at
      // score width 256 over value width 128 the allocator then spills, so
      // one there)
      constexpr int kPart = NW * 32 * PRS;      // floats of one staged half
      constexpr int DHR = RING / (4 * kPart) >= 2 && DK / 64 >= 2 && DV == DK ? 2 : 1;
      static_assert((DK / 64) % DHR == 0 && DHR * 4 * kPart <= RING, "staged halves fit the ring region");
      // rows of Σ X_{t,j} ⊙ v_{t,h} (X = dA, v = q: dk1; X = O'', v = dout: dv1)
      auto write_partials = [&](const floatx16 (&X)[DK / 32], const char* vrow, float* const dst) {
#pragma unroll
        for (int dr = 0; dr < DK / 64; dr += DHR) {
#pragma unroll
          for (int dh = dr; dh < dr + DHR; ++dh) {
            float* const part = (float*)lds + (dh - dr) * kPart;  // [NW][32][PRS] (ring region)
            if constexpr (!kOT) {
              // X^T (dA^T or O''^T): lane n holds row n, 4 consecutive d per 16-byte write
              float* pw = part + (wid * 32 + (fresh_lane() & 31)) * PRS;
#pragma unroll
              for (int dbl = 0; dbl < 2; ++dbl)
#pragma unroll
                for (int q4 = 0; q4 < 4; ++q4) {
                  const int dd = 32 * dbl + 8 * q4 + 4 * half;
                  floatx4 qv;
                  if constexpr (F32) {
                    qv = *(const floatx4*)(vrow + 4 * (64 * dh + dd));
                  } else {
                    const bf16x4 qb4 = *(const bf16x4*)(vrow + 2 * (64 * dh + dd));
#pragma unroll
                    for (int e = 0; e < 4; ++e) qv[e] = (float)qb4[e];
                  }
                  floatx4 x;
#pragma unroll
                  for (int e = 0; e < 4; ++e) x[e] = row_ok ? qv[e] * X[2 * dh + dbl][4 * q4 + e] : 0.f;
                  *(floatx4*)(pw + dd) = x;
                }
            } else {
              // X (lane = d; dk1 only): lane (i, half) holds column d = 64 dh + 32 dbl + i of
              // rows n = 8 g + 4 half + e; one q value per column
              const int lf = fresh_lane();
              const int hf = lf >> 5, i = lf & 31;
              float* pw = part + wid * 32 * PRS + i;
#pragma unroll
              for (int dbl = 0; dbl < 2; ++dbl) {
                const float qv = (float)*(const bf16*)(vrow + 2 * (64 * dh + 32 * dbl + i));
                if (nv >= 32) {
#pragma unroll
                  for (int g4 = 0; g4 < 4; ++g4)
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                      pw[(8 * g4 + 4 * hf + e) * PRS + 32 * dbl] = qv * X[2 * dh + dbl][4 * g4 + e];
                } else {
                  int nvm = nv;
                  asm volatile("" : "+s"(nvm));
#pragma unroll
                  for (int g4 = 0; g4 < 4; ++g4)
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                      const int nr_ = 8 * g4 + 4 * hf + e;
                      pw[nr_ * PRS + 32 * dbl] = nr_ < nvm ? qv * X[2 * dh + dbl][4 * g4 + e] : 0.f;
                    }
                }
              }
            }
          }
          block_barrier();  // every wave's rows staged
          // thread index from a fresh lane id: the store addresses are not
          // hoisted into registers held through the key loop
          for (int o = fresh_lane() + 64 * wid; o < DHR * ROWS1 * 16; o += 64 * NW) {
            const int u = DHR > 1 ? o / (ROWS1 * 16) : 0;
            const int jrow = (DHR > 1 ? o % (ROWS1 * 16) : o) >> 4, d4 = o & 15;
            const float* const part = (const float*)lds + u * kPart;
            floatx4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int w = 0; w < NW; ++w) {
              const int nn = w / NH + 31 - jrow;  // wave w = (qo, hw) = (w / NH, w % NH)
              if (nn >= 0 && nn < 32) acc += *(const floatx4*)(part + (w * 32 + nn) * PRS + 4 * d4);
            }
            *(floatx4*)(dst + jrow * DK + 64 * (dr + u) + 4 * d4) = acc;
          }
          block_barrier();  // sums read before the next round (or exit) reuses the region
        }
      };
      const int64_t pofs = (((int64_t)hg * geo.qblocks + qb) * geo.nr + r) * (ROWS1 * DK);
      write_partials(dA, qslot + wid * G::RSK, p.dk1p + pofs);  // the wave's q row
      if constexpr (FV) write_partials(dO, qslot + NW * G::RSK + wid * G::RSV, p.dv1p + pofs);  // its dout row
    }
  }

  if (qvalid) {
    if constexpr (F32) {
      float* orow = (float*)p.dq + (int64_t)t * p.dq_st + (int64_t)h * p.dq_sh;
#pragma unroll
      for (int i = 0; i < DK / 64; ++i) orow[64 * i + lane] = dqrun[i];
    } else {
      bf16* orow = (bf16*)p.dq + (int64_t)t * p.dq_st + (int64_t)h * p.dq_sh;
#pragma unroll
      for (int i = 0; i < DK / 64; ++i) orow[64 * i + lane] = (bf16)dqrun[i];
    }
  }
}

template <int DK, int DV, int NQ, int NH, bool FUSE = false, bool F32 = false, bool FV = false>
hipError_t launch_dq_t(const BwdParams& p, BwdGeo geo, hipStream_t stream) {
  // one tile in flight: ring + short slot + q/dout rows stay <= 80 KB (2 per
  // CU; fp32 inputs: rows twice as wide, one per CU)
  constexpr int P = 1;
  geo.qblocks = (p.tokens + NQ - 1) / NQ;
  geo.hsub = p.group / NH;
  geo.nblocks = geo.qblocks * p.hk * geo.hsub;
  constexpr int NW = NQ * NH;
  constexpr int EW = F32 ? 2 : 1;
  using G = TileGeom<EW * DK, EW * DV, kChunk + NQ - 1, NW, 32, 32>;
  const size_t qslot = ((size_t)NW * (G::RSK + G::RSV) + 1023) / 1024 * 1024;
  const size_t ring = (size_t)(P + 1) * G::SLOT, red = (size_t)NW * 64 * 36 * sizeof(float);
  const size_t lds = (ring > red ? ring : red) + G::SLOT + qslot;
  auto kern = bwd_dq_mfma_kernel<DK, DV, NQ, NH, P, FUSE, F32, FV>;
  hipError_t e = set_lds_limit((const void*)kern, lds);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(kern, dim3(geo.nblocks), dim3(64 * NW), lds, stream, p, geo);
  return hipGetLastError();
}

template <int DK, int DV, bool F32 = false>
hipError_t launch_dq_d(const BwdParams& p, BwdGeo geo, hipStream_t stream) {
  if constexpr (F32) {
    if (p.dk1p && p.dv1p) {  // dk1 and dv1 partials
      if (p.group % 4 == 0) return launch_dq_t<DK, DV, 1, 4, true, true, true>(p, geo, stream);
      if (p.group % 2 == 0) return launch_dq_t<DK, DV, 2, 2, true, true, true>(p, geo, stream);
      return launch_dq_t<DK, DV, 4, 1, true, true, true>(p, geo, stream);
    }
  }
  if (p.group % 4 == 0)
    return p.dk1p ? launch_dq_t<DK, DV, 1, 4, true, F32>(p, geo, stream)
                  : launch_dq_t<DK, DV, 1, 4, false, F32>(p, geo, stream);
  if (p.group % 2 == 0)
    return p.dk1p ? launch_dq_t<DK, DV, 2, 2, true, F32>(p, geo, stream)
                  : launch_dq_t<DK, DV, 2, 2, false, F32>(p, geo, stream);
  return p.dk1p ? launch_dq_t<DK, DV, 4, 1, true, F32>(p, geo, stream)
                : launch_dq_t<DK, DV, 4, 1, false, F32>(p, geo, stream);
}


// ---------------------------------------------------------------------------
// dk1, dv1: a workgroup of 4 waves owns 4 consecutive short keys of one KV
// group and loops over the group's query heads, so that every (j, KV group)
// is summed over all its heads inside one workgroup.  Wave (j = j0 + wave,
// head h) has rows t = j + 32r + n (pass r); chunk c of its rows' long windows
// covers keys j + 32r - wl + 1 + 32c + [0, 32).  The 4 waves share one K2/V2
// tile of 35 rows per chunk and one slot of q / dout rows (head h, queries
// j0 + 32r .. +34).
// MODE 1: dk1 only (G), MODE 2: dv1 only (O''), in two launches: one
// accumulator set (and, for dv1, neither the B rows nor dP) fits two waves
// per SIMD; the S recomputation is paid twice.
// F32: fp32 inputs (DK == DV <= 128), as in the dq pass: K2 / V2 tiles from
// the hi/lo rows, fp32 q / dout / k1 / v1 rows in LDS, products split into
// hi/lo terms, three term pairs per product, fp32 output.
template <int DK, int DV, int NQ, int NH, int P, int MODE, bool F32 = false>
__global__ __launch_bounds__(64 * NQ * NH, (DK > 128 || F32) ? 1 : 2) void bwd_dkv1_mfma_kernel(BwdParams p,
                                                                                             BwdGeo geo) {
  static_assert(NQ == 4 && NH == 1, "4 keys per block, one head at a time");
  static_assert(!F32 || (DK == DV && DK <= 128), "fp32 inputs: equal widths up to 128");
  constexpr bool kDK = MODE == 1, kDV = MODE == 2;
  static_assert(kDK || kDV, "one output per launch");
  constexpr int XW = kDK ? DK : DV;  // width of the gradient accumulated
  // G / O'' with the lane on d (MFMA operands swapped) at score width 256:
  // the epilogue sums the rows in registers, as the dq pass does there
  constexpr bool kOT = !F32 && DK >= 256;
  constexpr int NW = NQ * NH;
  constexpr int ROWS = kChunk + NQ - 1;
  constexpr int EW = F32 ? 2 : 1;  // bf16 units per element of an LDS row
  using G = TileGeom<EW * DK, EW * DV, ROWS, NW, 32, 32>;
  using OPK = BwdOps<DK>;
  using OPV = BwdOps<DV>;
  constexpr int R = P + 1;
  constexpr int NI = G::NI;
  constexpr int RING = R * G::SLOT > NW * 64 * 36 * 4 ? R * G::SLOT : NW * 64 * 36 * 4;
  extern __shared__ __attribute__((aligned(16))) char lds[];
  char* const rslot = lds + RING;       // q rows (K region) and dout rows (V region) of the pass's queries
  char* const kslot = rslot + G::SLOT;  // k1 rows 0..NW-1 (row stride RSK), then NW v1 rows (RSV)

  const int tid = tid_x(), lane = tid & 63;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int hw = wid % NH, qo = wid / NH;
  const int half = lane >> 5, n = lane & 31;

  const int lb = xcd_remap(bid_x(), geo.nblocks);
  const int jb = lb % geo.qblocks;
  const int g = lb / geo.qblocks;
  const int j0 = jb * NQ;
  if (j0 >= p.tokens) return;
  const int last = p.tokens - 1;
  const int j = __builtin_amdgcn_readfirstlane(j0 + qo);
  const bool jvalid = j < p.tokens;
  const int jc = min(j, last);
  // the sequence of key j: rows t in [j, send) share it
  const int s0 = seq_start(p.cu, p.num_seqs, p.seqlen, jc);
  int send;
  if (p.cu == nullptr) {
    send = s0 + p.seqlen;
  } else {
    int lo = 0, hi = p.num_seqs - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (p.cu[mid] <= jc) lo = mid;
      else hi = mid - 1;
    }
    send = min(p.cu[lo + 1], p.tokens);
  }
  send = __builtin_amdgcn_readfirstlane(max(send, jc + 1));

  // tile strides in bf16 units (fp32 inputs: the hi/lo rows [tokens][hk][2 D])
  const int64_t k_st = F32 ? (int64_t)p.hk * 2 * DK : p.k_st, v_st = F32 ? (int64_t)p.hk * 2 * DV : p.v_st;
  const int64_t k_g = F32 ? (int64_t)g * 2 * DK : (int64_t)g * p.k_sh;
  const int64_t v_g = F32 ? (int64_t)g * 2 * DV : (int64_t)g * p.v_sh;
  const bf16* const k2 = F32 ? p.k2s : (const bf16*)p.k2;
  const bf16* const v2 = F32 ? p.v2s : (const bf16*)p.v2;

  uint32_t koff[NI];  // this lane's byte offsets in a K2/V2 tile
#pragma unroll
  for (int k = 0; k < NI; ++k) {
    int is_v, row, seg;
    G::decode(wid, k, lane, is_v, row, seg);
    koff[k] = (uint32_t)(((int64_t)row * (is_v ? v_st : k_st) + seg * 8) * 2);
  }
  // One tile of rows kb .. kb+ROWS-1 of (kt: K region, vt: V region), rows
  // clamped into [0, tokens) at the tensor edges.
  auto dma_rows = [&](char* slot, int kb_in, const bf16* kt, int64_t kst, int64_t kof, const bf16* vt, int64_t vst,
                      int64_t vof, const uint32_t* off) {
    const int kb = __builtin_amdgcn_readfirstlane(kb_in);
    if (kb >= 0 && kb + ROWS - 1 <= last) {
      const char* kbase = (const char*)(kt + (int64_t)kb * kst + kof);
      const char* vbase = (const char*)(vt + (int64_t)kb * vst + vof);
#pragma unroll
      for (int k = 0; k < NI; ++k)
        dma16(uniform_ptr(G::instr_is_v(wid, k) ? vbase : kbase) + off[k], G::dst(slot, wid, k));
    } else {
      // rows derived afresh from the lane id (not hoisted into live registers)
      const int lf = fresh_lane();
#pragma unroll
      for (int k = 0; k < NI; ++k) {
        int is_v, row, seg;
        G::decode(wid, k, lf, is_v, row, seg);
        const int64_t key = min(max(kb + row, 0), last);
        const bf16* src = is_v ? vt + key * vst + vof : kt + key * kst + kof;
        dma16(src + seg * 8, G::dst(slot, wid, k));
      }
    }
  };
  // k1 and v1 rows of the NW waves' keys (wave 0)
  constexpr int KI = (NW * (G::RSK + G::RSV) + 1023) / 1024;
  auto dma_kv = [&]() {
    if (wid == 0) {
#pragma unroll
      for (int k = 0; k < KI; ++k) {
        const int b = k * 1024 + lane * 16;
        const bool isv = b >= NW * G::RSK;  // the v1 rows follow the k1 rows
        const int bb = isv ? b - NW * G::RSK : b, rs = isv ? G::RSV : G::RSK;
        int row = bb / rs, seg = (bb % rs) >> 4;
        if (row >= NW || seg >= (isv ? G::kSegsV : G::kSegsK)) row = 0, seg = 0;
        const int jr = min(j0 + row / NH, last);
        const bf16* src = isv ? (const bf16*)p.v1 + EW * ((int64_t)jr * p.v_st + (int64_t)g * p.v_sh)
                              : (const bf16*)p.k1 + EW * ((int64_t)jr * p.k_st + (int64_t)g * p.k_sh);
        dma16(src + seg * 8, kslot + k * 1024);
      }
    }
  };

  const float sl2s = p.scale * kLog2e;
  float xrun[XW / 64];  // dk1 (MODE 1) or dv1 (MODE 2) of this wave's key, d = 64*i + lane
#pragma unroll
  for (int i = 0; i < XW / 64; ++i) xrun[i] = 0.f;
  RowBlock<DK, DV, F32> ra;  // A rows (q_t ⊙ k1_j)
  RowBlock<DV, DV, F32> rbv;  // B rows (dout_t ⊙ v1_j)
  const int nc = (p.wl + 2 * kChunk - 2) / kChunk;  // chunks over wl + 31 keys
  dma_kv();
  bool first = true;

  for (int hs = 0; hs < geo.hsub; ++hs) {
    const int h = __builtin_amdgcn_readfirstlane(g * p.group + hs * NH + hw);
    // q / dout rows of head h: the row slot uses the q and dout strides
    uint32_t roff[NI];
#pragma unroll
    for (int k = 0; k < NI; ++k) {
      int is_v, row, seg;
      G::decode(wid, k, lane, is_v, row, seg);
      roff[k] = (uint32_t)(((int64_t)row * EW * (is_v ? p.do_st : p.q_st) + seg * 8) * 2);
    }
    for (int r = 0; r < geo.nr; ++r) {
      const int t = j + 32 * r + n;  // this lane's row (query)
      const bool row_ok = jvalid && 32 * r + n < p.ws && t < send;
      const int tc = min(t, last);
      const int64_t th = (int64_t)tc * p.hq + h;
      const float lse2 = row_ok ? p.lse[(int64_t)tc * p.lse_st + h] * kLog2e : 0.f;
      const float lse2r = row_ok ? lse2 : INFINITY;  // exp2(x - inf) = 0: rows outside the window
      const bool single = t == s0 || (p.ws == 1 && p.wl == 1);
      const float dpm = single ? 0.f : p.scale;
      const float dsm = row_ok ? (single ? p.dl[th] * p.scale : -p.delta[th] * p.scale) : 0.f;
      const int kb0 = j0 + 32 * r - p.wl + 1;  // key of tile row 0 at chunk 0
      const int tb0 = j0 + 32 * r;             // query of row-slot row 0
      if (!first) block_barrier();  // the previous pass's epilogue reads of the LDS are done
      first = false;
      dma_rows(rslot, tb0, (const bf16*)p.q, EW * p.q_st, EW * (int64_t)h * p.q_sh, (const bf16*)p.dout,
               EW * p.do_st, EW * (int64_t)h * p.do_sh, roff);
      auto issue = [&](int c) {
        dma_rows(lds + (c % R) * G::SLOT, kb0 + kChunk * c, k2, k_st, k_g, v2, v_st, v_g, koff);
      };
#pragma unroll
      for (int e = 0; e < P; ++e) issue(e);
      wait_vmcnt<P * NI>();
      block_barrier();
      const int srow = qo + n;  // row of query t in the row slot
      // kslot row w holds the k1 (v1: row NW + w) row of key j0 + w / NH, i.e. this wave's key
      if constexpr (F32) {
        OPK::form_hl_lds(rslot + srow * G::RSK, kslot + wid * G::RSK, row_ok, half, ra.a, ra.al);
        if constexpr (kDK)
          OPV::form_hl_lds(rslot + G::VOFF + srow * G::RSV, kslot + NW * G::RSK + wid * G::RSV, row_ok, half,
                           rbv.a, rbv.al);
      } else {
        ra.form_a_lds(rslot + srow * G::RSK, kslot + wid * G::RSK, row_ok, half, false);
        if constexpr (kDK) rbv.form_a_lds(rslot + G::VOFF + srow * G::RSV, kslot + NW * G::RSK + wid * G::RSV, row_ok, half, false);
      }

      floatx16 acc[XW / 32];  // G^T (MODE 1) or O''^T (MODE 2)
#pragma unroll
      for (int i = 0; i < XW / 32; ++i) acc[i] = floatx16{};
      for (int c = 0; c < nc; ++c) {
        wait_tiles<NI, P>(min(P - 1, nc - 1 - c));
        block_barrier();
        if (c + P < nc) issue(c + P);
        const int kfirst = j + 32 * r - p.wl + 1 + kChunk * c;  // key of this wave's chunk row 0
        // per-row key range: max(s0, t - wl + 1) <= k <= t
        const int klo = max(max(s0 - kfirst, n - kChunk * c), 0);
        const int khi = min(n + p.wl - 1 - kChunk * c, kChunk - 1);
        const char* slot = lds + (c % R) * G::SLOT;
        // dv1 launch (registers to spare): reads two MFMAs ahead
        constexpr int kPF = kDV ? 2 : kDk1PF;
        floatx16 sv, dp;
        if constexpr (F32) {
          sv = OPK::template rows_x_hl<G::RSK>(slot, qo, lane, ra.a, ra.al);
          if constexpr (kDK) dp = OPV::template rows_x_hl<G::RSV>(slot + G::VOFF, qo, lane, rbv.a, rbv.al);
        } else {
          sv = OPK::template rows_x<G::RSK, kPF>(slot, qo, lane, ra.a);
          if constexpr (kDK) dp = OPV::template rows_x<G::RSV>(slot + G::VOFF, qo, lane, rbv.a);
        }
        const int lo_h = klo - 4 * half, hi_h = khi - 4 * half;
        // interior chunk: every key valid for every row of the wave (uniform test)
        const bool interior = s0 <= kfirst && c >= 1 && kChunk * c <= p.wl - kChunk;
        if constexpr (F32) {
          // dS (MODE 1) or P (MODE 2) in fp32, then hi/lo B operands
          float x[16];
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const int kr = 8 * (e >> 2) + (e & 3);
            const bool ok = interior || (row_ok && kr >= lo_h && kr <= hi_h);
            const float pe = ok ? fast_exp2(fmaf(sv[e], sl2s, -(interior ? lse2r : lse2))) : 0.f;
            if constexpr (kDK) x[e] = pe * fmaf(dp[e], dpm, dsm);
            else x[e] = pe;
          }
          bf16x8 b0, b1, l0, l1;
          OPK::pack_c_hl(x, b0, b1, l0, l1);
          if constexpr (kDK) OPK::template tr_acc_hl<G::RSK>(acc, slot, qo, lane, b0, b1, l0, l1);
          else OPV::template tr_acc_hl<G::RSV>(acc, slot + G::VOFF, qo, lane, b0, b1, l0, l1);
          continue;
        }
        // dS (MODE 1) or P (MODE 2) straight into packed bf16 pairs (B operand)
        uint32_t pk[8];
        if (interior) {  // rows outside the window: exp2(s*c - inf) = 0 with no per-key test
#pragma unroll
          for (int e = 0; e < 16; e += 2) {
            const float p0 = fast_exp2(fmaf(sv[e], sl2s, -lse2r)), p1 = fast_exp2(fmaf(sv[e + 1], sl2s, -lse2r));
            if constexpr (kDK) pk[e >> 1] = pack_bf16(p0 * fmaf(dp[e], dpm, dsm), p1 * fmaf(dp[e + 1], dpm, dsm));
            else pk[e >> 1] = pack_bf16(p0, p1);
          }
        } else {
#pragma unroll
          for (int e = 0; e < 16; e += 2) {
            const int kr0 = 8 * (e >> 2) + (e & 3), kr1 = kr0 + 1;
            const bool ok0 = row_ok && kr0 >= lo_h && kr0 <= hi_h;
            const bool ok1 = row_ok && kr1 >= lo_h && kr1 <= hi_h;
            const float p0 = ok0 ? fast_exp2(fmaf(sv[e], sl2s, -lse2)) : 0.f;
            const float p1 = ok1 ? fast_exp2(fmaf(sv[e + 1], sl2s, -lse2)) : 0.f;
            if constexpr (kDK) pk[e >> 1] = pack_bf16(p0 * fmaf(dp[e], dpm, dsm), p1 * fmaf(dp[e + 1], dpm, dsm));
            else pk[e >> 1] = pack_bf16(p0, p1);
          }
        }
        const bf16x8 b0 = __builtin_bit_cast(bf16x8, u32x4{pk[0], pk[1], pk[2], pk[3]});
        const bf16x8 b1 = __builtin_bit_cast(bf16x8, u32x4{pk[4], pk[5], pk[6], pk[7]});
        if constexpr (kDK) OPK::template tr_acc<G::RSK, 1, kOT>(acc, slot, qo, lane, b0, b1);  // G^T += K2^T · dS^T
        else OPV::template tr_acc<G::RSV, kPF, kOT>(acc, slot + G::VOFF, qo, lane, b0, b1);  // O''^T += V2^T · P^T
      }
      wait_vmcnt<0>();
      block_barrier();  // ring reads done (LDS reused below)

      // dk1[d] += Σ_t G_t[d] q_t[d] (MODE 1), dv1[d] += Σ_t O''_t[d] dout_t[d] (MODE 2)
      if constexpr (kOT) {
        // acc (lane = d): column d = 32 db + lane % 32, register 4 g + e = row
        // n = 8 g + 4 half + e (row-slot row qo + n); the q / dout values read
        // transposed from the row slot; rows past the window dropped (their
        // products are 0, and a stale row need not be finite)
        const int nv = jvalid ? max(0, min(min(32, p.ws - 32 * r), send - (j + 32 * r))) : 0;
        const int lf = fresh_lane();
        const int hf = lf >> 5, g16 = (lf >> 4) & 1, i16 = lf & 15;
        constexpr int RSX = kDK ? G::RSK : G::RSV;
        const uint32_t xp = lds_addr(rslot + (kDK ? 0 : G::VOFF) + (qo + 4 * hf + (i16 >> 2)) * RSX + 32 * g16 +
                                     8 * (i16 & 3));
        static_for<0, XW / 32>([&](auto dd) {
          constexpr int db = decltype(dd)::value;
          shortx4 x[4];
          static_for<0, 4>([&](auto gg) {
            constexpr int gi = decltype(gg)::value;
            x[gi] = ds_read_tr16<8 * gi * RSX + 64 * db>(xp);
          });
          lds_wait(x[0], x[1]);
          lds_wait(x[2], x[3]);
          float sx = 0.f;
          if (nv >= 32) {
#pragma unroll
            for (int g4 = 0; g4 < 4; ++g4)
#pragma unroll
              for (int e = 0; e < 4; ++e) sx = fmaf(bf16_bits_to_f32(x[g4][e]), acc[db][4 * g4 + e], sx);
          } else {
            // an opaque copy of nv keeps the row tests inside this rare branch
            int nvm = nv;
            asm volatile("" : "+s"(nvm));
#pragma unroll
            for (int g4 = 0; g4 < 4; ++g4)
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                const float xv = 8 * g4 + 4 * hf + e < nvm ? bf16_bits_to_f32(x[g4][e]) : 0.f;
                sx = fmaf(xv, acc[db][4 * g4 + e], sx);
              }
          }
          // both halves hold column d's sum; the half of block db's parity keeps it
          const float tot = pair_sum(sx);
          xrun[db >> 1] = hf == (db & 1) ? xrun[db >> 1] + tot : xrun[db >> 1];
        });
      } else {
        float* red = (float*)lds + wid * (64 * 36);
        const char* xs = kDK ? rslot + srow * G::RSK : rslot + G::VOFF + srow * G::RSV;
        floatx4 xv[XW / 64][2][4];
#pragma unroll
        for (int sl = 0; sl < XW / 64; ++sl)
#pragma unroll
          for (int dbl = 0; dbl < 2; ++dbl)
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4) {
              const int dd = 64 * sl + 32 * dbl + 8 * q4 + 4 * half;
              if constexpr (F32) {
                xv[sl][dbl][q4] = *(const floatx4*)(xs + 4 * dd);
              } else {
                const bf16x4 xb = *(const bf16x4*)(xs + 2 * dd);
#pragma unroll
                for (int e = 0; e < 4; ++e) xv[sl][dbl][q4][e] = (float)xb[e];
              }
            }
#pragma unroll
        for (int sl = 0; sl < XW / 64; ++sl) {
#pragma unroll
          for (int dbl = 0; dbl < 2; ++dbl) {
            const int db = 2 * sl + dbl;
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4) {
              const int dd = 32 * dbl + 8 * q4 + 4 * half;
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                const float x = row_ok ? xv[sl][dbl][q4][e] : 0.f;
                red[(dd + e) * 36 + n] = x * acc[db][4 * q4 + e];
              }
            }
          }
          float acc = 0.f;
          const floatx4* row4 = (const floatx4*)(red + lane * 36);
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            floatx4 x = row4[i];
            acc += (x[0] + x[1]) + (x[2] + x[3]);
          }
          xrun[sl] += acc;
        }
      }
    }
  }

  // sum over the NH waves of each key (heads hw), then write
  block_barrier();
  float* sum = (float*)lds;  // [NW][XW]
#pragma unroll
  for (int i = 0; i < XW / 64; ++i) sum[wid * XW + 64 * i + lane] = xrun[i];
  block_barrier();
  if (hw == 0 && jvalid) {
    const int64_t off = kDK ? (int64_t)j * p.dk_st + (int64_t)g * p.dk_sh : (int64_t)j * p.dv_st + (int64_t)g * p.dv_sh;
#pragma unroll
    for (int i = 0; i < XW / 64; ++i) {
      float a = 0.f;
      for (int w = 0; w < NH; ++w) a += sum[(wid + w) * XW + 64 * i + lane];
      if constexpr (F32) ((float*)(kDK ? p.dk1 : p.dv1))[off + 64 * i + lane] = a;
      else ((bf16*)(kDK ? p.dk1 : p.dv1))[off + 64 * i + lane] = (bf16)a;
    }
  }
}

template <int DK, int DV, int NQ, int NH, bool F32 = false>
hipError_t launch_dkv1_t(const BwdParams& p, BwdGeo geo, hipStream_t stream) {
  constexpr int P = 1;  // two workgroups per CU (<= 80 KB of LDS each; fp32: one)
  geo.qblocks = (p.tokens + NQ - 1) / NQ;
  geo.hsub = p.group / NH;
  geo.nblocks = geo.qblocks * p.hk;
  constexpr int NW = NQ * NH;
  constexpr int EW = F32 ? 2 : 1;
  using G = TileGeom<EW * DK, EW * DV, kChunk + NQ - 1, NW, 32, 32>;
  const size_t kslot = ((size_t)NW * (G::RSK + G::RSV) + 1023) / 1024 * 1024;
  const size_t ring = (size_t)(P + 1) * G::SLOT, red = (size_t)NW * 64 * 36 * sizeof(float);
  const size_t lds = (ring > red ? ring : red) + G::SLOT + kslot;
  for (auto kern : {bwd_dkv1_mfma_kernel<DK, DV, NQ, NH, P, 1, F32>, bwd_dkv1_mfma_kernel<DK, DV, NQ, NH, P, 2, F32>}) {
    if (p.dk1p && kern == bwd_dkv1_mfma_kernel<DK, DV, NQ, NH, P, 1, F32>) continue;  // dk1 came from the dq pass
    hipError_t e = set_lds_limit((const void*)kern, lds);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(kern, dim3(geo.nblocks), dim3(64 * NW), lds, stream, p, geo);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

template <int DK, int DV, bool F32 = false>
hipError_t launch_dkv1_d(const BwdParams& p, BwdGeo geo, hipStream_t stream) {
  return launch_dkv1_t<DK, DV, 4, 1, F32>(p, geo, stream);
}

// dk1[j, g] = Σ_{head sub-groups hs of g} Σ_{row groups r} Σ_{query blocks qb}
// partial[g*hsub + hs][qb][r][j - nq qb + 31 + 32 r], over the blocks whose
// group-r rows hold j (nq qb in [j + 32 r - nq + 1, j + 32 r + 31]), in that
// nesting and ascending order.  nq = queries per dq workgroup, hsub = head
// sub-groups per KV group, nr = row groups.  One thread per (j, g, 4 values
// of d).
template <int D>
__global__ __launch_bounds__(256) void bwd_dk1_sum_kernel(BwdParams p, int qblocks, int nq, int hsub, int nr) {
  constexpr int D4 = D / 4;
  const int64_t i = (int64_t)bid_x() * 256 + tid_x();
  const int64_t jg = i / D4;
  if (jg >= (int64_t)p.tokens * p.hk) return;
  const int d4 = (int)(i % D4);
  const int g = (int)(jg % p.hk), j = (int)(jg / p.hk);
  const int rows = 31 + nq;
  floatx4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int hs = 0; hs < hsub; ++hs) {
    const float* base = p.dk1p + (int64_t)(g * hsub + hs) * qblocks * nr * rows * D + 4 * d4;
    for (int r = 0; r < nr; ++r) {
      const int qlo = (j + 32 * r) / nq, qhi = min((j + 32 * r + 31) / nq, qblocks - 1);
      for (int qb = qlo; qb <= qhi; ++qb) {
        const floatx4 x = *(const floatx4*)(base + (((int64_t)qb * nr + r) * rows + (j - nq * qb + 31 + 32 * r)) * D);
        acc += x;
      }
    }
  }
  const int64_t off = (int64_t)j * p.dk_st + (int64_t)g * p.dk_sh + 4 * d4;
  if (p.f32) {
    *(floatx4*)((float*)p.dk1 + off) = acc;
  } else {
    bf16x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = (bf16)acc[e];
    *(bf16x4*)((bf16*)p.dk1 + off) = o;
  }
}


// ---------------------------------------------------------------------------
// dk2, dv2: a workgroup of NWK waves owns 32 * NWK consecutive long keys of
// one KV group; wave w's 32 keys are kw = k0 + 32w + lane % 32.  It walks the
// steps (t, h) for t = k0 .. k0 + 32 NWK - 1 + wl - 1 (every query whose long
// window can reach a key of the block) and h over the group's heads.  Per
// step the waves build, per 32-row group r < NR of short keys, A_t (rows
// j = t - 32r - 31 .. t - 32r: bf16(q_th ⊙ k1_j)) and B_t (bf16(dout_th ⊙
// v1_j)) in LDS, 32 / NWK rows each; tiles are double-buffered, one barrier
// per step.  Wider blocks (NWK = 8 at D = 128) share each step's tile
// formation, barrier and staging among more keys.  The last wave stages each
// step's q, dout, k1_t and v1_t rows with one full-wave DMA two steps ahead; the
// k1 / v1 rows of earlier queries come from a 64·NR-row ring (row j at slot
// j % (64 NR)) into which wave 0 copies each staged k1_t / v1_t.  Covers
// ws <= 32 NR (NR = 1, 2).

// MODE 1: dK2 only, MODE 2: dV2 only (two launches).  Each holds one
// accumulator set, and the dV2 launch neither the V2 fragments nor dP, so
// both fit two waves per SIMD; the S recomputation is paid twice.
// MODE 3 (fp32 inputs, which run one wave per SIMD either way): dK2 and dV2
// in one launch from one S per step and one formation of the A / B rows.
// PH (phased): twice the short-key rows of one launch run as two launches,
// phase 1 (row groups 0 .. NR-1: rows j = t - 32 NR + 1 .. t) writing its fp32
// sums to p.dkv2p and phase 2 (groups NR .. 2NR-1) starting from them and
// writing the gradient; widths of 256 (one group per launch) always run so.
// Without PH, phase is 0 (one launch).
// F32: fp32 inputs (DK == DV <= 128, NR = 1): the K2 / V2 fragments from the
// hi/lo rows (hi and lo fragments), fp32 q / dout / k1 / v1 rows in the
// stage and the ring, A / B tile rows formed as [hi: D | lo: D] from fp32
// products, three term pairs per product, fp32 output.
// splits > 1 (one launch, bf16): the workgroups of a (key block, KV head)
// walk contiguous pieces of its queries and write fp32 sums to p.dkv2s
// ([split][tokens][hk][XW]); bwd_dkv2_sum_kernel adds them in split order.
template <int DK, int DV, int MODE, int NWK, int NR, bool PH, bool F32 = false>
__global__ __launch_bounds__(64 * NWK, (DK > 128 || F32) ? 1 : 2) void bwd_dkv2_mfma_kernel(BwdParams p,
                                                                                           int nblocks, int phase,
                                                                                           int splits) {
  static_assert(!F32 || (DK == DV && DK <= 128 && NR == 1 && !PH), "fp32 inputs: equal widths up to 128, one group");
  constexpr bool kBoth = MODE == 3;  // dK2 and dV2 (fp32)
  static_assert(!kBoth || F32, "both gradients in one launch: fp32 inputs");
  constexpr bool kDK = MODE == 1 || kBoth, kDV = MODE == 2 || kBoth;
  constexpr int EW = F32 ? 2 : 1;  // bf16 units per element of an LDS row
  constexpr int kKvRing = 64 * NR;  // k1 / v1 ring rows (a power of two)
  constexpr int KB = 32 * NWK;    // keys per workgroup
  constexpr int RPW = 32 / NWK;   // A / B rows formed per wave and step
  // LDS reads in flight ahead of their MFMA: with two waves per SIMD, one
  // read ahead leaves each step's three MFMA chains waiting on LDS latency
  constexpr int kPF = DK >= 256 ? kDkv2PFWide : kDkv2PF;
  static_assert(kDK || kDV, "an output per launch");
  constexpr int XW = kDK ? DK : DV;        // width of the gradient accumulated in acc (dK2 when both)
  using OPK = BwdOps<DK>;
  using OPV = BwdOps<DV>;
  // A / B tile row strides (padded: row and transposing reads)
  constexpr int RSA = 2 * EW * DK + 32, RSB = 2 * EW * DV + 32;
  constexpr int TA = 32 * RSA, TAB = TA + 32 * RSB;  // one A tile, one A + B pair
  constexpr int RBK = 2 * EW * DK, RBV = 2 * EW * DV;  // k1 / v1 row bytes (q / dout rows alike)
  constexpr int RKV = RBK + RBV;             // ring row: k1 then v1
  constexpr int SS = (2 * RKV + 1023) / 1024 * 1024, SI = SS / 1024;  // stage slot bytes, DMA instructions
  extern __shared__ __attribute__((aligned(16))) char lds[];
  char* const tiles = lds;                        // [2 buffers][NR groups][A, B]
  char* const ring = tiles + 2 * NR * TAB;        // [64 NR slots][k1 row, v1 row]
  char* const stage = ring + kKvRing * RKV;       // [3][q row, dout row, k1_t row, v1_t row] (SS bytes each)

  const int tid = tid_x(), lane = tid & 63;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half = lane >> 5, n = lane & 31;
  // per wave: the per-step scalars of 64 steps, 16 bytes each
  floatx4* const scal = (floatx4*)(stage + 3 * SS) + 64 * wid;
  constexpr bool kPhased = PH;
  const int r0 = kPhased && phase == 2 ? NR : 0;  // row group offset of this launch (the ring holds 64 NR rows)
  // walk splits: bf16 single launches only (the launcher passes 1 otherwise)
  constexpr bool kSplit = !PH && !F32;
  const int nsplit = kSplit ? splits : 1;
  const int lb = xcd_remap(bid_x(), nblocks);
  const int kblocks = (p.tokens + KB - 1) / KB;
  const int kb = lb % kblocks;
  const int g = kSplit ? lb / kblocks % p.hk : lb / kblocks;
  const int split = kSplit ? lb / kblocks / p.hk : 0;
  const int k0 = kb * KB;
  const int last = p.tokens - 1;
  const int kw = k0 + 32 * wid + n;  // this lane's key (column of the C layout)
  const int kwc = min(kw, last);
  const bool kvalid = kw < p.tokens;
  const int G = p.group;
  const int64_t kvg_k = (int64_t)g * p.k_sh, kvg_v = (int64_t)g * p.v_sh;

  // K2 / V2 rows of the wave's keys as B operands (k = d): lane (n, half)
  // holds d = 16t + 8*half .. +7 of key kw.
  // (fp32: the hi/lo rows [tokens][hk][2 D], hi fragments in kf / vf, lo in kfl / vfl)
  const bf16* k2r = F32 ? p.k2s + ((int64_t)kwc * p.hk + g) * 2 * DK : (const bf16*)p.k2 + (int64_t)kwc * p.k_st + kvg_k;
  const bf16* v2r = F32 ? p.v2s + ((int64_t)kwc * p.hk + g) * 2 * DV : (const bf16*)p.v2 + (int64_t)kwc * p.v_st + kvg_v;
  bf16x8 kf[DK / 16], vf[kDK ? DV / 16 : 1];
  bf16x8 kfl[F32 ? DK / 16 : 1], vfl[F32 && kDK ? DV / 16 : 1];
#pragma unroll
  for (int t = 0; t < DK / 16; ++t) {
    kf[t] = *(const bf16x8*)(k2r + 16 * t + 8 * half);
    if constexpr (F32) kfl[t] = *(const bf16x8*)(k2r + DK + 16 * t + 8 * half);
  }
  if constexpr (kDK) {
#pragma unroll
    for (int t = 0; t < DV / 16; ++t) {
      vf[t] = *(const bf16x8*)(v2r + 16 * t + 8 * half);
      if constexpr (F32) vfl[t] = *(const bf16x8*)(v2r + DV + 16 * t + 8 * half);
    }
  }
  floatx16 acc[XW / 32];  // dK2^T or dV2^T
#pragma unroll
  for (int i = 0; i < XW / 32; ++i) acc[i] = floatx16{};
  floatx16 accv[kBoth ? DV / 32 : 1];  // dV2^T (both gradients)
#pragma unroll
  for (int i = 0; i < (kBoth ? DV / 32 : 1); ++i) accv[i] = floatx16{};
  // fp32 sums of the first row group (phases 1 and 2): [tokens][hk][DK] for
  // dK2, then [tokens][hk][DV] for dV2, each lane's values at its d
  auto part_row = [&]() {
    return p.dkv2p + (kDK ? 0 : (int64_t)p.tokens * p.hk * DK) + ((int64_t)kwc * p.hk + g) * XW;
  };
  if (kPhased && phase == 2 && kvalid) {
    const float* part = part_row();
#pragma unroll
    for (int db = 0; db < XW / 32; ++db)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const floatx4 x = *(const floatx4*)(part + 32 * db + 8 * q4 + 4 * half);
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[db][4 * q4 + e] = x[e];
      }
  }

  // the queries reaching the block's keys, t = k0 .. min(last, k0 + KB + wl - 2),
  // cut into `splits` contiguous pieces; this workgroup walks piece `split`
  const int walk = min(last, k0 + KB - 1 + p.wl - 1) - k0 + 1;
  const int tfirst = k0 + (int)((int64_t)walk * split / nsplit);
  const int tlast = k0 + (int)((int64_t)walk * (split + 1) / nsplit) - 1;
  // step s <-> (t = tfirst + s / G, h = g*G + s % G)
  const int nsteps = (tlast - tfirst + 1) * G;
  // write: acc[db] holds d = 32*db + acc_row(r, half) of key kw
  auto write_out = [&]() {
    if (!kvalid) return;
    if (kSplit && nsplit > 1) {
      float* part = p.dkv2s + (((int64_t)split * p.tokens + kw) * p.hk + g) * XW;
#pragma unroll
      for (int db = 0; db < XW / 32; ++db)
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
          floatx4 x;
#pragma unroll
          for (int e = 0; e < 4; ++e) x[e] = acc[db][4 * q4 + e];
          *(floatx4*)(part + 32 * db + 8 * q4 + 4 * half) = x;
        }
    } else if (kPhased && phase == 1) {
      float* part = part_row();
#pragma unroll
      for (int db = 0; db < XW / 32; ++db)
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
          floatx4 x;
#pragma unroll
          for (int e = 0; e < 4; ++e) x[e] = acc[db][4 * q4 + e];
          *(floatx4*)(part + 32 * db + 8 * q4 + 4 * half) = x;
        }
    } else if (F32) {
      // key and half from a fresh lane id: row addresses formed here, not
      // held (or spilled) through the step loop
      const int lf = fresh_lane();
      const int kwf = k0 + 32 * wid + (lf & 31), hf = lf >> 5;
      float* orow = kDK ? (float*)p.dk2 + (int64_t)kwf * p.dk_st + (int64_t)g * p.dk_sh
                        : (float*)p.dv2 + (int64_t)kwf * p.dv_st + (int64_t)g * p.dv_sh;
#pragma unroll
      for (int db = 0; db < XW / 32; ++db)
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
          floatx4 a;
#pragma unroll
          for (int e = 0; e < 4; ++e) a[e] = acc[db][4 * q4 + e];
          *(floatx4*)(orow + 32 * db + 8 * q4 + 4 * hf) = a;
        }
      if constexpr (kBoth) {
        float* vrow = (float*)p.dv2 + (int64_t)kwf * p.dv_st + (int64_t)g * p.dv_sh;
#pragma unroll
        for (int db = 0; db < DV / 32; ++db)
#pragma unroll
          for (int q4 = 0; q4 < 4; ++q4) {
            floatx4 a;
#pragma unroll
            for (int e = 0; e < 4; ++e) a[e] = accv[db][4 * q4 + e];
            *(floatx4*)(vrow + 32 * db + 8 * q4 + 4 * hf) = a;
          }
      }
    } else {
      bf16* orow = kDK ? (bf16*)p.dk2 + (int64_t)kw * p.dk_st + (int64_t)g * p.dk_sh
                       : (bf16*)p.dv2 + (int64_t)kw * p.dv_st + (int64_t)g * p.dv_sh;
#pragma unroll
      for (int db = 0; db < XW / 32; ++db)
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
          const int d = 32 * db + 8 * q4 + 4 * half;
          bf16x4 a;
#pragma unroll
          for (int e = 0; e < 4; ++e) a[e] = (bf16)acc[db][4 * q4 + e];
          *(bf16x4*)(orow + d) = a;
        }
    }
  };
  // an empty piece (a short last key block): zero sums (uniform, before any
  // barrier); one piece always holds t = k0
  if (kSplit && nsteps <= 0) {
    write_out();
    return;
  }

  // Step st <-> (t = tfirst + st / G, h = g*G + st % G), stage slot st % 3:
  // carried from step to step (no divisions in the step loop).
  struct Step {
    int t, h, slot;
  };
  auto advance = [&](Step x) {
    Step y{x.t, x.h + 1, x.slot == 2 ? 0 : x.slot + 1};
    if (y.h == g * G + G) y.h = g * G, ++y.t;
    return y;
  };
  // The staging wave stages step st: lane -> byte 16 lane of the rows q,
  // dout, k1_t, v1_t laid end to end (lanes past them re-fetch the q row's
  // first segment into the unused tail); every lane active, one instruction
  // per 1 KB.  Every wave waits for the staging wave at the step's barrier, so
  // its addresses are selected per lane without branches (a lane's tensor is
  // fixed by its byte offset b), the row offsets formed once per step in
  // scalars.  Four-wave workgroups stage from the last wave (wave 0 copies
  // rows into the ring): dk2 / dv2 3-4 % faster at the adapter shape and at
  // width 256 than from wave 0; eight-wave ones from wave 0 (the last wave
  // measured 4 % slower there).
  constexpr int kDmaWave = NWK >= 8 ? 0 : NWK - 1;
  auto dma_step = [&](int st, Step x) {
    if (wid != kDmaWave || st >= nsteps) return;
    // element offsets of the step's rows (uniform)
    const int64_t oq = (int64_t)x.t * p.q_st + (int64_t)x.h * p.q_sh;
    const int64_t og = (int64_t)x.t * p.do_st + (int64_t)x.h * p.do_sh;
    const int64_t ok = (int64_t)x.t * p.k_st + kvg_k, ov = (int64_t)x.t * p.v_st + kvg_v;
#pragma unroll
    for (int k = 0; k < SI; ++k) {
      // byte offset from a fresh lane id: not hoisted into registers held through the step loop
      int b = 1024 * k + 16 * fresh_lane();
      if (b >= 2 * RKV) b = 0;
      const bool isq = b < RBK, isg = b < RKV, isk = b < RKV + RBK;
      const bf16* base = isq ? (const bf16*)p.q : isg ? (const bf16*)p.dout : isk ? (const bf16*)p.k1 : (const bf16*)p.v1;
      const int64_t oe = isq ? oq : isg ? og : isk ? ok : ov;
      const int inrow = b - (isq ? 0 : isg ? RBK : isk ? RKV : RKV + RBK);  // bytes
      // (element offsets scaled by EW: fp32 rows viewed as bf16 units)
      dma16(base + EW * oe + inrow / 2, stage + x.slot * SS + 1024 * k);
    }
  };
  // wave 0 copies the staged k1_t / v1_t rows of step st into ring slot t % (64 NR)
  auto to_ring = [&](int st, Step x) {
    if (wid != 0 || st >= nsteps) return;
    if (lane < RKV / 16) {
      const uint4 v = *(const uint4*)(stage + x.slot * SS + RKV + 16 * lane);
      *(uint4*)(ring + (x.t % kKvRing) * RKV + 16 * lane) = v;
    }
  };

  Step s_cur{tfirst, g * G, 0};
  Step s_nx1 = advance(s_cur), s_nx2 = advance(s_nx1);
  dma_step(0, s_cur);
  dma_step(1, s_nx1);
  // the k1 / v1 rows before the first query (j = tfirst - 32 NR + 1 .. tfirst - 1) into the ring
  for (int idx = tid; idx < (32 * (NR + r0) - 1) * (RKV / 16); idx += 64 * NWK) {
    const int jj = idx / (RKV / 16), w = idx % (RKV / 16);  // w: 16-byte segment of the ring row
    const int j = tfirst - (32 * (NR + r0) - 1) + jj;
    if (j >= 0) {
      const bf16* src = w < RBK / 16 ? (const bf16*)p.k1 + EW * ((int64_t)j * p.k_st + kvg_k) + 8 * w
                                     : (const bf16*)p.v1 + EW * ((int64_t)j * p.v_st + kvg_v) + 8 * (w - RBK / 16);
      *(uint4*)(ring + (j % kKvRing) * RKV + 16 * w) = *(const uint4*)src;
    }
  }
  wait_vmcnt<0>();
  block_barrier();

  // form A / B rows of step st into tile buffer b: wave w builds rows
  // RPW w .. RPW w + RPW - 1 of each group; row 31 of group 0 (j = t) comes
  // from the stage, earlier rows from the ring
  auto form = [&](Step x, int b) {
    const int t = x.t;
    const char* sg_row = stage + x.slot * SS;
    if constexpr (F32) {
      // fp32 rows: one row and 4 elements (16 source bytes) per lane; the
      // products q ⊙ k1 and dout ⊙ v1 split into hi (row elements 4 sg ..)
      // and lo (elements D + 4 sg ..) bf16 terms.  A lane's 4-element group sg
      // = lane % SEGS is the same in every row block: its q and dout values
      // are read once, and the k1 / v1 reads of kB blocks at a time are
      // issued before their products.
      constexpr int SEGS = DK / 4;
      static_assert(RPW * SEGS % 64 == 0 && 64 % SEGS == 0, "whole lanes per formed row block");
      constexpr int NU = RPW * SEGS / 64, kB = NU < 2 ? NU : 2;
      const int sg = lane % SEGS;
      const floatx4 qv = *(const floatx4*)(sg_row + 16 * sg);
      const floatx4 gv = *(const floatx4*)(sg_row + RBK + 16 * sg);
      char* At = tiles + b * TAB;
      char* Bt = At + TA;
#pragma unroll
      for (int u0 = 0; u0 < NU; u0 += kB) {
        floatx4 kv[kB], vv[kB];
#pragma unroll
        for (int u = 0; u < kB; ++u) {
          const int i = RPW * wid + ((u0 + u) * 64 + lane) / SEGS;  // tile row
          const int j = max(t - 31 + i, 0);
          const char* kvrow = j == t ? sg_row + RKV : ring + (j % kKvRing) * RKV;
          kv[u] = *(const floatx4*)(kvrow + 16 * sg);
          vv[u] = *(const floatx4*)(kvrow + RBK + 16 * sg);
        }
#pragma unroll
        for (int u = 0; u < kB; ++u) {
          const int i = RPW * wid + ((u0 + u) * 64 + lane) / SEGS;
          bf16x4 ah, al, bh, bl;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            bf16 h_, l_;
            split_bf16(qv[e] * kv[u][e], h_, l_);
            ah[e] = h_;
            al[e] = l_;
            split_bf16(gv[e] * vv[u][e], h_, l_);
            bh[e] = h_;
            bl[e] = l_;
          }
          *(bf16x4*)(At + i * RSA + 8 * sg) = ah;
          *(bf16x4*)(At + i * RSA + 2 * DK + 8 * sg) = al;
          *(bf16x4*)(Bt + i * RSB + 8 * sg) = bh;
          *(bf16x4*)(Bt + i * RSB + 2 * DV + 8 * sg) = bl;
        }
      }
    } else if constexpr (DK == DV) {  // A and B rows side by side: one row and segment per lane
      constexpr int SEGS = DK / 8;  // 16-byte segments per row
      static_assert(RPW * SEGS % 64 == 0 && 64 % SEGS == 0, "whole lanes per formed row block");
      constexpr int NU = NR * RPW * SEGS / 64;  // row blocks formed by each lane
      // A lane forms segment sg = lane % SEGS of every row block, so its q and
      // dout segments are read once; every k1 / v1 read is issued before the
      // first product (the tile writes would otherwise keep each block's reads
      // behind the previous block's writes: one LDS latency per block).
      const int sg = lane % SEGS;
      const u32x4 q4 = __builtin_bit_cast(u32x4, *(const bf16x8*)(sg_row + 16 * sg));
      const u32x4 g4 = __builtin_bit_cast(u32x4, *(const bf16x8*)(sg_row + RBK + 16 * sg));
      u32x4 k4[NU], v4[NU];
#pragma unroll
      for (int u = 0; u < NU; ++u) {
        const int r = u / (RPW * SEGS / 64);  // row group
        const int i = RPW * wid + ((u % (RPW * SEGS / 64)) * 64 + lane) / SEGS;  // tile row
        const int j = max(t - 32 * (r + r0) - 31 + i, 0);
        const char* kvrow = j == t ? sg_row + RKV : ring + (j % kKvRing) * RKV;
        k4[u] = __builtin_bit_cast(u32x4, *(const bf16x8*)(kvrow + 16 * sg));
        v4[u] = __builtin_bit_cast(u32x4, *(const bf16x8*)(kvrow + RBK + 16 * sg));
      }
#pragma unroll
      for (int u = 0; u < NU; ++u) {
        const int r = u / (RPW * SEGS / 64);
        char* At = tiles + (b * NR + r) * TAB;
        char* Bt = At + TA;
        const int i = RPW * wid + ((u % (RPW * SEGS / 64)) * 64 + lane) / SEGS;
        u32x4 a, bb;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          a[e] = mul_bf16_pair(q4[e], k4[u][e]);
          bb[e] = mul_bf16_pair(g4[e], v4[u][e]);
        }
        *(u32x4*)(At + i * RSA + 16 * sg) = a;
        *(u32x4*)(Bt + i * RSB + 16 * sg) = bb;
      }
    } else {  // A rows (DK / 8 segments), then B rows (DV / 8)
      constexpr int SK = DK / 8, SV = DV / 8;
      static_assert(RPW * SK % 64 == 0 && RPW * SV % 64 == 0 && 64 % SK == 0 && 64 % SV == 0,
                    "whole lanes per formed row block");
      constexpr int UA = RPW * SK / 64, UB = RPW * SV / 64, NU = NR * (UA + UB);
      // as above: a lane's q (dout) segment lane % SK (lane % SV) is the same
      // in every A (B) block, read once; every k1 / v1 read is issued first
      const u32x4 q4 = __builtin_bit_cast(u32x4, *(const bf16x8*)(sg_row + 16 * (lane % SK)));
      const u32x4 g4 = __builtin_bit_cast(u32x4, *(const bf16x8*)(sg_row + RBK + 16 * (lane % SV)));
      u32x4 y4[NU];
#pragma unroll
      for (int u = 0; u < NU; ++u) {
        const int r = u / (UA + UB), v = u % (UA + UB);  // row group, instruction within it
        const bool isb = v >= UA;
        const int segs = isb ? SV : SK, off = isb ? RBK : 0;
        const int idx = (isb ? v - UA : v) * 64 + lane;
        const int i = RPW * wid + idx / segs, sg = idx % segs;  // tile row, segment
        const int j = max(t - 32 * (r + r0) - 31 + i, 0);
        const char* kvrow = j == t ? sg_row + RKV : ring + (j % kKvRing) * RKV;
        y4[u] = __builtin_bit_cast(u32x4, *(const bf16x8*)(kvrow + off + 16 * sg));
      }
#pragma unroll
      for (int u = 0; u < NU; ++u) {
        const int r = u / (UA + UB), v = u % (UA + UB);
        const bool isb = v >= UA;
        const int segs = isb ? SV : SK;
        const int idx = (isb ? v - UA : v) * 64 + lane;
        const int i = RPW * wid + idx / segs, sg = idx % segs;
        const u32x4 x4 = isb ? g4 : q4;
        u32x4 a;
#pragma unroll
        for (int e = 0; e < 4; ++e) a[e] = mul_bf16_pair(x4[e], y4[u][e]);
        char* At = tiles + (b * NR + r) * TAB;
        *(u32x4*)(isb ? At + TA + i * RSB + 16 * sg : At + i * RSA + 16 * sg) = a;
      }
    }
  };

  const float sl2s = p.scale * kLog2e;
  // Sequence of t, tracked as the start s0 of t's sequence and the first
  // token past it (dense: a boundary every seqlen; packed: the cu walk, one
  // load per boundary crossed).
  int seq = 0, s0 = 0, snext = 0;
  if (p.cu != nullptr) {
    int lo = 0, hi = p.num_seqs - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (p.cu[mid] <= tfirst) lo = mid;
      else hi = mid - 1;
    }
    seq = lo;
    snext = tfirst;  // first step loads the start and the next boundary
  } else {
    s0 = (tfirst / p.seqlen) * p.seqlen;
    snext = s0 + p.seqlen;
  }
  // Per-step scalars (lse, and for dK2 dl and delta of (t, h)): loaded one
  // lane per step, 64 steps at a time and one block ahead, and kept in a
  // wave-private LDS table, so that a step reads them from LDS instead of
  // waiting on a global load.
  floatx4 nx{};  // this lane's step of the next block (loads in flight)
  auto load_block = [&](int blk) {
    const int si = min(64 * blk + lane, nsteps - 1);
    const int tq = tfirst + si / G, hq = g * G + si % G;
    const int64_t thq = (int64_t)tq * p.hq + hq;
    nx[0] = p.lse[(int64_t)tq * p.lse_st + hq];
    if constexpr (kDK) {
      nx[1] = p.dl[thq];
      nx[2] = p.delta[thq];
    }
  };
  auto store_block = [&]() {
    // the wait is tied to these registers: later steps need none
    asm volatile("s_waitcnt vmcnt(0)" : "+v"(nx));
    scal[lane] = nx;
  };
  load_block(0);
  store_block();
  if (nsteps > 64) load_block(1);
  to_ring(0, s_cur);
  form(s_cur, 0);
  for (int st = 0; st < nsteps; ++st) {
    const int sl = st & 63;
    if (sl == 0 && st > 0) {  // next block: its values into the table, load the one after
      store_block();
      if (st + 64 < nsteps) load_block((st >> 6) + 1);
    }
    // staging wave: the rows of step st+1 have landed (step st+2's may be in flight)
    if (wid == kDmaWave) {
      dma_step(st + 2, s_nx2);
      if (st + 2 < nsteps) wait_vmcnt<SI>();
      else wait_vmcnt<0>();
    }
    block_barrier();  // tiles of st formed, ring rows up to t(st) copied; rows of st+1 staged; buffer (st+1)%2 free
    const Step s_now = s_cur, s_form = s_nx1;
    s_cur = s_nx1, s_nx1 = s_nx2, s_nx2 = advance(s_nx2);

    const int t = s_now.t;
    if (t >= snext) {  // crossed into another sequence (uniform, rare)
      if (p.cu == nullptr) {
        s0 = (t / p.seqlen) * p.seqlen;
        snext = s0 + p.seqlen;
      } else {
        while (seq + 1 < p.num_seqs && p.cu[seq + 1] <= t) ++seq;
        const int c = p.cu[seq];
        s0 = min(max(c, 0), t);
        // well formed (cu[seq] <= t): the start holds up to the next boundary
        snext = c > t ? t + 1 : (seq + 1 < p.num_seqs ? p.cu[seq + 1] : 0x7fffffff);
      }
      s0 = __builtin_amdgcn_readfirstlane(s0);
      snext = __builtin_amdgcn_readfirstlane(snext);
    }
    const floatx4 sv4 = scal[sl];  // wave-private: this wave's table writes are ordered before
    const float lse2 = sv4[0] * kLog2e;
    const bool single = t == s0 || (p.ws == 1 && p.wl == 1);
    const float dpm = single ? 0.f : p.scale;
    const float dsm = kDK ? (single ? sv4[1] * p.scale : -sv4[2] * p.scale) : 0.f;
    // validity: key kw in [max(s0, t - wl + 1), t]; row i (j = t - 31 + i) in [max(s0, t - ws + 1), t]
    const bool kok = kvalid && kw <= t && kw >= max(s0, t - p.wl + 1);
    const int ilo = max(s0, t - p.ws + 1) - (t - 31 - 32 * r0);
    // a wave none of whose 32 keys lies in t's long window skips the step
    // (about a fifth of the steps at the block's ends)
    const int kw0 = k0 + 32 * wid;
    const bool skip = kw0 > t || kw0 + 31 < max(s0, t - p.wl + 1) || kw0 >= p.tokens;
    const char* At = tiles + (st & 1) * NR * TAB;  // group 0
    const char* Bt = At + TA;
    floatx16 sv, dp;
    if (!skip) {
      if constexpr (F32) {
        sv = OPK::template rows_x_hl<RSA>(At, 0, lane, kf, kfl);  // C[j][key]
        if constexpr (kDK) dp = OPV::template rows_x_hl<RSB>(Bt, 0, lane, vf, vfl);
      } else {
        sv = OPK::template rows_x<RSA, kPF>(At, 0, lane, kf);  // C[j][key]
        if constexpr (kDK) dp = OPV::template rows_x<RSB, kPF>(Bt, 0, lane, vf);
      }
    }
    // the next step's rows are formed after this step's S (and dP) MFMAs are
    // issued: the VALU work runs while the matrix cores work (the two waves
    // of a SIMD are in step with each other through the barrier, so their
    // VALU phases would otherwise coincide with an idle matrix pipe)
    if (st + 1 < nsteps) {
      to_ring(st + 1, s_form);  // slot t(st+1) % 64 is read only from the next iteration on
      form(s_form, (st + 1) & 1);
    }
    if (skip) continue;
    // group r: the probabilities (dS or P) from its scores, then
    // dK2^T += A_t^T · dS^T, or dV2^T += B_t^T · P^T
    auto accumulate = [&](const floatx16& s_, const floatx16& dp_, int ilo_r, const char* At_r, const char* Bt_r) {
      if constexpr (F32) {
        // dS (dK2) and / or P (dV2) in fp32, as hi/lo B operands
        float x[16], pv[kBoth ? 16 : 1];
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int ie = 8 * (e >> 2) + 4 * half + (e & 3);
          const bool ok = kok && ie >= ilo_r;
          const float pe = ok ? fast_exp2(fmaf(s_[e], sl2s, -lse2)) : 0.f;
          if constexpr (kDK) x[e] = pe * fmaf(dp_[e], dpm, dsm);
          else x[e] = pe;
          if constexpr (kBoth) pv[e] = pe;
        }
        bf16x8 b0, b1, l0, l1;
        OPK::pack_c_hl(x, b0, b1, l0, l1);
        if constexpr (kDK) OPK::template tr_acc_hl<RSA>(acc, At_r, 0, lane, b0, b1, l0, l1);
        else OPV::template tr_acc_hl<RSB>(acc, Bt_r, 0, lane, b0, b1, l0, l1);
        if constexpr (kBoth) {
          OPK::pack_c_hl(pv, b0, b1, l0, l1);
          OPV::template tr_acc_hl<RSB>(accv, Bt_r, 0, lane, b0, b1, l0, l1);
        }
        return;
      }
      uint32_t pk[8];  // bf16(dS) (dK2 launch) or bf16(P) (dV2 launch)
      if (ilo_r <= 0) {  // every row valid (uniform test); keys outside: exp2(s*c - inf) = 0
        const float lse2k = kok ? lse2 : INFINITY;
#pragma unroll
        for (int e = 0; e < 16; e += 2) {
          const float p0 = fast_exp2(fmaf(s_[e], sl2s, -lse2k)), p1 = fast_exp2(fmaf(s_[e + 1], sl2s, -lse2k));
          if constexpr (kDK) pk[e >> 1] = pack_bf16(p0 * fmaf(dp_[e], dpm, dsm), p1 * fmaf(dp_[e + 1], dpm, dsm));
          else pk[e >> 1] = pack_bf16(p0, p1);
        }
      } else {
#pragma unroll
        for (int e = 0; e < 16; e += 2) {
          const int i0 = 8 * (e >> 2) + 4 * half + (e & 3), i1 = i0 + 1;
          const bool ok0 = kok && i0 >= ilo_r, ok1 = kok && i1 >= ilo_r;
          const float p0 = ok0 ? fast_exp2(fmaf(s_[e], sl2s, -lse2)) : 0.f;
          const float p1 = ok1 ? fast_exp2(fmaf(s_[e + 1], sl2s, -lse2)) : 0.f;
          if constexpr (kDK) pk[e >> 1] = pack_bf16(p0 * fmaf(dp_[e], dpm, dsm), p1 * fmaf(dp_[e + 1], dpm, dsm));
          else pk[e >> 1] = pack_bf16(p0, p1);
        }
      }
      const bf16x8 b0 = __builtin_bit_cast(bf16x8, u32x4{pk[0], pk[1], pk[2], pk[3]});
      const bf16x8 b1 = __builtin_bit_cast(bf16x8, u32x4{pk[4], pk[5], pk[6], pk[7]});
      if constexpr (kDK) OPK::template tr_acc<RSA, kPF>(acc, At_r, 0, lane, b0, b1);
      else OPV::template tr_acc<RSB, kPF>(acc, Bt_r, 0, lane, b0, b1);
    };
    accumulate(sv, dp, ilo, At, Bt);
#pragma unroll
    for (int r = 1; r < NR; ++r) {
      const int ilo_r = ilo + 32 * r;  // first valid row of group r (rows j = t - 32r - 31 + i)
      if (ilo_r >= 32) break;          // group r lies before the short window (uniform)
      const char* Ar = At + r * TAB;
      const floatx16 sr = OPK::template rows_x<RSA, kPF>(Ar, 0, lane, kf);
      floatx16 dr;
      if constexpr (kDK) dr = OPV::template rows_x<RSB, kPF>(Ar + TA, 0, lane, vf);
      accumulate(sr, dr, ilo_r, Ar, Ar + TA);
    }
  }

  write_out();
}

// dk2 or dv2 (mode 1 / 2) = the sum of the walk splits' fp32 sums in split
// order; 4 values per thread
template <int XW>
__global__ __launch_bounds__(256) void bwd_dkv2_sum_kernel(BwdParams p, int splits, int mode) {
  const int64_t i = (int64_t)bid_x() * 256 + tid_x();
  const int64_t rows = (int64_t)p.tokens * p.hk;
  if (i >= rows * (XW / 4)) return;
  const int64_t row = i / (XW / 4);
  const int c = (int)(i % (XW / 4)) * 4;
  const float* src = p.dkv2s + row * XW + c;
  floatx4 acc = *(const floatx4*)src;
  for (int k = 1; k < splits; ++k) {
    const floatx4 x = *(const floatx4*)(src + (int64_t)k * rows * XW);
#pragma unroll
    for (int e = 0; e < 4; ++e) acc[e] += x[e];
  }
  const int64_t t = row / p.hk, g = row % p.hk;
  bf16* o = mode == 1 ? (bf16*)p.dk2 + t * p.dk_st + g * p.dk_sh : (bf16*)p.dv2 + t * p.dv_st + g * p.dv_sh;
  bf16x4 b;
#pragma unroll
  for (int e = 0; e < 4; ++e) b[e] = (bf16)acc[e];
  *(bf16x4*)(o + c) = b;
}

// LDS bytes of a dk2 / dv2 workgroup (EW: bf16 units per row element)
constexpr size_t dkv2_lds_bytes(int dk, int dv, int nr, int nwk, int ew) {
  const size_t rsa = 2 * ew * dk + 32, rsb = 2 * ew * dv + 32, rkv = 2 * ew * (dk + dv);
  const size_t ss = (2 * rkv + 1023) / 1024 * 1024;  // stage slot
  return 2 * nr * 32 * (rsa + rsb) + 64 * nr * rkv + 3 * ss + (size_t)nwk * 64 * 16;
}

template <int DK, int DV, int NR, bool PH, bool F32, int NWK>
hipError_t launch_dkv2_t(const BwdParams& p, int splits, hipStream_t stream) {
  constexpr size_t lds = dkv2_lds_bytes(DK, DV, NR, NWK, F32 ? 2 : 1);
  // more short-key rows than one launch's LDS holds: two launches (phases 1, 2)
  const bool two = PH && p.ws > 32 * NR;
  if (two || F32 || !p.dkv2s) splits = 1;
  const int nblocks = (p.tokens + 32 * NWK - 1) / (32 * NWK) * p.hk * splits;
  // fp32: one launch for both gradients (mode 3); bf16: dK2, then dV2
  for (int mode = F32 ? 3 : 1; mode <= (F32 ? 3 : 2); ++mode) {
    auto kern = [&]() {
      if constexpr (F32) return bwd_dkv2_mfma_kernel<DK, DV, 3, NWK, NR, PH, true>;
      else return mode == 1 ? bwd_dkv2_mfma_kernel<DK, DV, 1, NWK, NR, PH, false>
                            : bwd_dkv2_mfma_kernel<DK, DV, 2, NWK, NR, PH, false>;
    }();
    hipError_t e = set_lds_limit((const void*)kern, lds);
    if (e != hipSuccess) return e;
    for (int phase = two ? 1 : 0; phase <= (two ? 2 : 0); ++phase) {
      hipLaunchKernelGGL(kern, dim3(nblocks), dim3(64 * NWK), lds, stream, p, nblocks, phase, splits);
      e = hipGetLastError();
      if (e != hipSuccess) return e;
    }
    if (splits > 1) {
      const int xw = mode == 1 ? DK : DV;
      const dim3 grid((unsigned)(((int64_t)p.tokens * p.hk * (xw / 4) + 255) / 256));
      if (xw == 64) hipLaunchKernelGGL(bwd_dkv2_sum_kernel<64>, grid, dim3(256), 0, stream, p, splits, mode);
      else hipLaunchKernelGGL(bwd_dkv2_sum_kernel<128>, grid, dim3(256), 0, stream, p, splits, mode);
      e = hipGetLastError();
      if (e != hipSuccess) return e;
    }
  }
  return hipSuccess;
}

template <int DK, int DV, int NR, bool PH, bool F32 = false>
hipError_t launch_dkv2_w(const BwdParams& p, hipStream_t stream) {
  const Dkv2Plan pl = bwd_dkv2_plan(p.tokens, p.hk, DK, DV, p.ws, p.wl, F32, device_cu_count());
  if constexpr (DK == 128 && DV == 128 && !F32) {
    if (pl.nwk == 8) return launch_dkv2_t<DK, DV, NR, PH, F32, 8>(p, pl.splits, stream);
  }
  return launch_dkv2_t<DK, DV, NR, PH, F32, 4>(p, pl.splits, stream);
}

template <int DK, int DV>
hipError_t launch_dkv2_d(const BwdParams& p, hipStream_t stream) {
  if constexpr (DK > 128) {
    return launch_dkv2_w<DK, DV, 1, true>(p, stream);  // LDS for one row group per launch
  } else {
    if (p.ws <= 32) return launch_dkv2_w<DK, DV, 1, false>(p, stream);
    if (p.ws <= 64) return launch_dkv2_w<DK, DV, 2, false>(p, stream);
    return launch_dkv2_w<DK, DV, 2, true>(p, stream);  // two launches of two row groups
  }
}

// bf16, score width DK and value width DV each 64 or 128, or DK = 256 over
// DV = 128 or 256 (the dq and dk1 / dv1 passes only), 16-byte aligned rows;
// fp32 inputs (p.f32, with the hi/lo rows of k2 and v2): DK == DV in {64, 128}.
bool bwd_mfma_ok(const BwdParams& p) {
  if (!p.mfma) return false;
  if (p.f32 && (p.d != p.dv || (p.d != 64 && p.d != 128) || !p.k2s || !p.v2s)) return false;
  const bool narrow = (p.d == 64 || p.d == 128) && (p.dv == 64 || p.dv == 128);
  if (!narrow && !(p.d == 256 && (p.dv == 128 || p.dv == 256))) return false;
  const int64_t st[] = {p.q_st, p.q_sh, p.k_st, p.k_sh, p.v_st, p.v_sh, p.do_st, p.do_sh};
  for (int64_t s : st)
    if (s % 8) return false;
  const uintptr_t ptrs = (uintptr_t)p.q | (uintptr_t)p.k1 | (uintptr_t)p.k2 | (uintptr_t)p.v1 |
                         (uintptr_t)p.v2 | (uintptr_t)p.dout;
  // gradients are written 4 elements at a time
  const int64_t ost[] = {p.dq_st, p.dq_sh, p.dk_st, p.dk_sh, p.dv_st, p.dv_sh};
  for (int64_t s : ost)
    if (s % 4) return false;
  const uintptr_t optrs = (uintptr_t)p.dq | (uintptr_t)p.dk1 | (uintptr_t)p.dk2 | (uintptr_t)p.dv1 | (uintptr_t)p.dv2;
  return (ptrs & 15) == 0 && (optrs & 15) == 0;
}

// fn(DK, DV) with the widths as integral constants; WIDE: DK = 256 as well
template <bool WIDE, typename Fn>
hipError_t by_widths(const BwdParams& p, Fn&& fn) {
  using W64 = std::integral_constant<int, 64>;
  using W128 = std::integral_constant<int, 128>;
  using W256 = std::integral_constant<int, 256>;
  if constexpr (WIDE) {
    if (p.d == 256) return p.dv == 256 ? fn(W256{}, W256{}) : fn(W256{}, W128{});
  }
  if (p.d == 64) return p.dv == 64 ? fn(W64{}, W64{}) : fn(W64{}, W128{});
  return p.dv == 64 ? fn(W128{}, W64{}) : fn(W128{}, W128{});
}

BwdGeo base_geo(const BwdParams& p) {
  BwdGeo geo{};
  geo.nc = (p.wl + kChunk - 1) / kChunk;
  geo.nr = (p.ws + 31) / 32;
  return geo;
}

}  // namespace

// Keys per workgroup (32 per wave, NWK waves): 8 waves when both widths are
// 128 (bf16), 4 otherwise (at DK = 256 and for fp32 the 4 waves fill a CU's
// LDS or registers).  When 8-wave workgroups would leave CUs without work --
// few KV heads over few tokens, e.g. the reference adapter's 2 KV heads x
// 16K tokens: 128 workgroups of 256 keys for 256 CUs -- 4-wave ones run, and
// at bf16 widths <= 128 with one launch (short window <= 64) each (key block,
// KV head) walk is cut into as many pieces as fill the CUs' resident
// workgroup slots (two waves per SIMD, or what the LDS allows), up to 8 and
// at least 128 queries per piece: the pieces' fp32 sums are added in a fixed
// order.  Narrower workgroups alone measured slower (every workgroup forms
// all 32 A / B rows of each step, so that work grows with the workgroup
// count); a split walk forms each step's rows once, as before.
Dkv2Plan bwd_dkv2_plan(int tokens, int hk, int d, int dv, int ws, int wl, bool f32, int cus) {
  const int nr = ws <= 32 ? 1 : 2;  // row groups per launch at widths <= 128
  const int64_t blocks8 = (int64_t)(tokens + 255) / 256 * hk;
  if (!f32 && d == 128 && dv == 128 && blocks8 >= (nr == 1 ? 2 : 1) * (int64_t)cus) return {8, 1};
  constexpr int nwk = 4;
  if (f32 || d > 128 || dv > 128 || ws > 64 || tokens <= 0 || hk <= 0) return {nwk, 1};
  const int64_t blocks = (int64_t)(tokens + 32 * nwk - 1) / (32 * nwk) * hk;
  const int64_t by_lds = (int64_t)kLdsPerCu / dkv2_lds_bytes(d, dv, nr, nwk, 1);
  const int64_t per_cu = std::max<int64_t>(1, std::min<int64_t>(by_lds, 8 / nwk));
  int64_t splits = ((int64_t)cus * per_cu + blocks - 1) / blocks;
  splits = std::min<int64_t>(splits, kMaxWalkSplits);
  splits = std::min<int64_t>(splits, ((int64_t)32 * nwk + wl - 1) / 128);  // pieces of >= 128 queries
  return {nwk, (int)std::max<int64_t>(splits, 1)};
}

hipError_t launch_bwd_dq_mfma(const BwdParams& p, hipStream_t stream) {
  if (!bwd_mfma_ok(p)) return hipErrorNotSupported;
  const BwdGeo geo = base_geo(p);
  if (p.f32) {
    if (p.ws > 32) return hipErrorNotSupported;  // fp32: one 32-row group of short keys
    return p.d == 64 ? launch_dq_d<64, 64, true>(p, geo, stream) : launch_dq_d<128, 128, true>(p, geo, stream);
  }
  return by_widths<true>(p, [&](auto dk, auto dv) { return launch_dq_d<decltype(dk)::value, decltype(dv)::value>(p, geo, stream); });
}

hipError_t launch_bwd_dkv1_mfma(const BwdParams& p, hipStream_t stream) {
  if (!bwd_mfma_ok(p)) return hipErrorNotSupported;
  const BwdGeo geo = base_geo(p);
  if (p.f32) {
    if (p.ws > 32) return hipErrorNotSupported;  // fp32: one 32-row group of short keys
    return p.d == 64 ? launch_dkv1_d<64, 64, true>(p, geo, stream) : launch_dkv1_d<128, 128, true>(p, geo, stream);
  }
  return by_widths<true>(p, [&](auto dk, auto dv) { return launch_dkv1_d<decltype(dk)::value, decltype(dv)::value>(p, geo, stream); });
}
bool bwd_dk1_fused_ok(const BwdParams& p) {
  return bwd_mfma_ok(p) && p.ws <= (p.f32 ? 32 : 64);
}

hipError_t launch_bwd_dk1_sum(const BwdParams& p, hipStream_t stream) {
  const int nq = dq_queries_per_block(p.group), hsub = p.group / (4 / nq);
  const int qblocks = (p.tokens + nq - 1) / nq;
  const int nr = (p.ws + 31) / 32;
  const int64_t threads = (int64_t)p.tokens * p.hk * (p.d / 4);
  const dim3 grid((unsigned)((threads + 255) / 256));
  if (p.d == 64) hipLaunchKernelGGL(bwd_dk1_sum_kernel<64>, grid, dim3(256), 0, stream, p, qblocks, nq, hsub, nr);
  else if (p.d == 128) hipLaunchKernelGGL(bwd_dk1_sum_kernel<128>, grid, dim3(256), 0, stream, p, qblocks, nq, hsub, nr);
  else hipLaunchKernelGGL(bwd_dk1_sum_kernel<256>, grid, dim3(256), 0, stream, p, qblocks, nq, hsub, nr);
  return hipGetLastError();
}

hipError_t launch_bwd_dv1_sum(const BwdParams& p, hipStream_t stream) {
  // the dk1 sum over the dv1 partials, into dv1 (value width and strides)
  BwdParams q = p;
  q.dk1p = p.dv1p;
  q.dk1 = p.dv1;
  q.dk_st = p.dv_st;
  q.dk_sh = p.dv_sh;
  q.d = p.dv;
  return launch_bwd_dk1_sum(q, stream);
}

hipError_t launch_bwd_dkv2_mfma(const BwdParams& p, hipStream_t stream) {
  if (p.f32) {  // fp32: one 32-row group of short keys
    if (!bwd_mfma_ok(p) || p.ws > 32) return hipErrorNotSupported;
    return p.d == 64 ? launch_dkv2_w<64, 64, 1, false, true>(p, stream) : launch_dkv2_w<128, 128, 1, false, true>(p, stream);
  }
  // one launch covers 64 short keys (32 at DK = 256); two launches over the fp32 partial twice that
  const int one = p.d > 128 ? 32 : 64;
  if (!bwd_mfma_ok(p) || p.ws > 2 * one || (p.ws > one && !p.dkv2p)) return hipErrorNotSupported;
  return by_widths<true>(p, [&](auto dk, auto dv) { return launch_dkv2_d<decltype(dk)::value, decltype(dv)::value>(p, stream); });
}

}  // namespace sa
