// Wave-level MFMA core shared by the bf16 prefill and paged kernels.
//
// A wave owns 32 "A rows" (one query token x one head x up to 32 short-axis
// keys j).  Lane l holds row n = l % 32 and half h = l / 32.  Per 32-key chunk
// of the long axis staged in LDS:
//
//   S^T = K_chunk · A^T     DK/16 v_mfma_f32_32x32x16_bf16, K rows from LDS
//   P^T = exp2(S^T*c - m)   per-row online softmax, lazy rescale
//   O^T += V^T · P^T        DV/32 x 2 MFMAs; the V^T operand is read from the
//                           natural [key][d] tile with ds_read_b64_tr_b16
//
// DK is the score width (q, k1, k2) and DV the value width (v1, v2, out); the
// reference's determinant scores use DK = 2 * DV.  LDS tiles: K [rows][DK]
// and V [rows][DV] bf16, row-major with a pad per row (see TileGeom).
//
// Tiles are filled with global_load_lds_dwordx4 (16 bytes per lane straight
// into LDS, no staging registers); one instruction fills 1 KB of LDS.
// The compiler does not order these DMA writes against later LDS reads, so
// the kernels wait explicitly (vmcnt) before the barrier that publishes a tile.
#pragma once

#include <type_traits>

#include "sa_common.h"

namespace sa {

typedef short shortx4 __attribute__((ext_vector_type(4)));
typedef short shortx8 __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(3))) shortx4 lds_shortx4;

// The bf16 held in the low 16 bits of x, widened to fp32 (exact).
__device__ __forceinline__ float bf16_bits_to_f32(short x) { return __uint_as_float((uint32_t)(uint16_t)x << 16); }

// LDS tile geometry.  The K tile is [rows][DK] bf16 with a row stride of
// 2DK + PADK bytes, the V tile [rows][DV] with 2DV + PADV.  LDS has 64 banks
// of 4 bytes; a ds_read_b128 serves 16 lanes per cycle and a
// ds_read_b64_tr_b16 32 lanes (measured with SQ_LDS_BANK_CONFLICT on this
// GPU).  The K reads put 16 consecutive rows (16 bytes each) in one cycle: a
// 16-byte pad moves consecutive rows by 4 banks, so the 16 rows cover all 64
// banks once.  The transposing V reads put 4 rows x 64 bytes in one cycle: a
// 64-byte pad moves consecutive rows by 16 banks, again 64 distinct banks.
// (A 32-byte pad on both gave 2-way conflicts on both.)  Every read address
// is a per-lane base plus an immediate.
template <int DK, int DV, int ROWS_T, int NW, int PADK = 16, int PADV = 64>
struct TileGeom {
  static constexpr int kSegsK = DK / 8;                       // 16-byte segments per K row
  static constexpr int kSegsV = DV / 8;                       // ... per V row
  static constexpr int RSK = 2 * DK + PADK;                   // LDS row strides (bytes)
  static constexpr int RSV = 2 * DV + PADV;
  static constexpr int TBK = ROWS_T * RSK;                    // one K tile (bytes)
  static constexpr int TBV = ROWS_T * RSV;                    // one V tile
  static constexpr int kInstrK = (TBK + 1023) / 1024;         // DMA instructions per K tile
  static constexpr int kInstrV = (TBV + 1023) / 1024;         // ... per V tile
  static constexpr int kInstr = (kInstrK + kInstrV + NW - 1) / NW * NW;
  static constexpr int NI = kInstr / NW;                      // DMA instructions per wave per tile
  static constexpr int VOFF = kInstrK * 1024;                 // V tile offset inside a slot
  static constexpr int SLOT = kInstr * 1024;                  // bytes of one ring slot

  // DMA instruction k of wave `wid` fills LDS bytes [1024*(wid*NI + k), +1024)
  // of the slot; instructions 0..kInstrK-1 fill the K tile, the next kInstrV
  // the V tile, any further ones are idle (they re-fetch row 0 into the
  // unused tail).  Lane `lane` fetches row `row`, segment `seg` of tensor
  // is_v.  Pad bytes fetch segment 0 of their row (never read).
  __device__ static __forceinline__ void decode(int wid, int k, int lane, int& is_v, int& row, int& seg) {
    const int i = wid * NI + k;
    is_v = i >= kInstrK;
    const int tb = is_v ? TBV : TBK, rs = is_v ? RSV : RSK, segs = is_v ? kSegsV : kSegsK;
    int b = (is_v ? i - kInstrK : i) * 1024 + lane * 16;
    if (i >= kInstrK + kInstrV || b >= tb) b = 0;
    row = b / rs;
    seg = (b % rs) >> 4;
    if (seg >= segs) seg = 0;
  }
  __device__ static __forceinline__ bool instr_is_v(int wid, int k) { return wid * NI + k >= kInstrK; }
  __device__ static __forceinline__ char* dst(char* slot, int wid, int k) { return slot + (wid * NI + k) * 1024; }
};

// Tile geometry of the forward kernels.  Widths of 256 keep 32-byte pads on
// both tiles (measured faster there with one wave per SIMD).  Smaller widths
// take the conflict-free 16-byte K pad; the V pad is 64 bytes (conflict-free
// transposing reads) unless that costs each wave one more DMA instruction per
// tile than a 32-byte pad (2-way conflicts on the V reads), as for the 35-row
// tiles of 4-query blocks: there the fewer DMA instructions and registers
// measured 3-4 % faster on NS and C2.
template <int DK, int DV, int ROWS_T, int NW>
using FwdGeom = std::conditional_t<
    (DK >= 256 || DV >= 256), TileGeom<DK, DV, ROWS_T, NW, 32, 32>,
    std::conditional_t<(TileGeom<DK, DV, ROWS_T, NW, 16, 64>::NI > TileGeom<DK, DV, ROWS_T, NW, 16, 32>::NI),
                       TileGeom<DK, DV, ROWS_T, NW, 16, 32>, TileGeom<DK, DV, ROWS_T, NW, 16, 64>>>;

// s_waitcnt vmcnt(n) with the other counters left alone (gfx9 encoding:
// vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt[5:4] << 14).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// Wait until at most k later tiles (NI DMA instructions each) are in flight.
template <int NI, int P>
__device__ __forceinline__ void wait_tiles(int k) {
  if constexpr (P >= 4) {
    if (k >= 3) { wait_vmcnt<NI * 3>(); return; }
  }
  if constexpr (P >= 3) {
    if (k >= 2) { wait_vmcnt<NI * 2>(); return; }
  }
  if constexpr (P >= 2) {
    if (k >= 1) { wait_vmcnt<NI>(); return; }
  }
  wait_vmcnt<0>();
}

// Barrier without the memory fences of __syncthreads.  Ordering of the DMA
// writes comes from the explicit vmcnt waits; the waves' own LDS accesses are
// ordered by the lgkmcnt(0) wait issued here before s_barrier.
__device__ __forceinline__ void block_barrier() {
  __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (0 << 8) | (3 << 14));  // lgkmcnt(0) only
  __builtin_amdgcn_s_barrier();
}

// A wave-uniform pointer pinned to SGPRs, so that DMA addresses take the
// scalar-base + 32-bit lane-offset form (no per-lane 64-bit adds).
template <typename T>
__device__ __forceinline__ const T* uniform_ptr(const T* p) {
  const uint64_t v = (uint64_t)(uintptr_t)p;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return (const T*)(uintptr_t)(((uint64_t)hi << 32) | lo);
}

__device__ __forceinline__ void dma16(const void* src, char* dst) {
  __builtin_amdgcn_global_load_lds(src, (lds_void*)dst, 16, 0, 0);
}
// Raw buffer descriptor over `base` (untyped 32-bit data format, no range
// limit in practice) for the buffer form of the same DMA.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t raw_rsrc(const void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, 0x7fffffff, 0x00020000);
}
// 16 bytes per lane from descriptor `r` at byte offset `voff` into LDS, the
// same lane layout as dma16.
__device__ __forceinline__ void dma16_buf(__amdgpu_buffer_rsrc_t r, uint32_t voff, char* dst) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void*)dst, 16, voff, 0, 0, 0);
}

// Compile-time loop: f(std::integral_constant<int, I>) for I in [B, E).
template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
}

// 32-bit LDS address of a pointer into the workgroup's LDS.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char*)p;
}

// ds_read_b64_tr_b16 issued through inline asm.  The compiler builtin makes
// the backend wait for every outstanding global->LDS DMA (vmcnt(0)) before
// each transposing read, which would drain the tile prefetch queue; the DMA
// ordering is already enforced explicitly (vmcnt wait + barrier per tile).
// The result is only valid after lds_wait() on it.
template <int OFF>
__device__ __forceinline__ shortx4 ds_read_tr16(uint32_t addr) {
  shortx4 r;
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF));
  return r;
}

// Wait for this wave's LDS reads; the operands tie the wait to the registers
// those reads fill, so no use of them can be scheduled before it.
__device__ __forceinline__ void lds_wait(shortx4& a, shortx4& b) {
  asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(a), "+v"(b));
}

// Wait until at most N of this wave's LDS operations are outstanding.  LDS
// operations complete in order, so with N issued after the reads that fill a
// and b, those reads are done (SMEM loads in flight only make it stricter).
template <int N>
__device__ __forceinline__ void lds_wait_n(shortx4& a, shortx4& b) {
  static_assert(N >= 0 && N < 16, "lgkmcnt is 4 bits");
  asm volatile("s_waitcnt lgkmcnt(%2)" : "+v"(a), "+v"(b) : "i"(N));
}

// ds_read_b128 issued through inline asm, for fragment chains that read ahead
// of their MFMAs: for the compiler's own reads in such a chain the backend
// emits lgkmcnt(0) before every few MFMAs, which also waits for the reads
// issued ahead (one MFMA earlier), so the chain stalls on LDS latency.  The
// result is only valid after lds_wait_k on it, with the exact count of LDS
// operations issued after it.
template <int OFF>
__device__ __forceinline__ bf16x8 ds_read_b128_at(uint32_t addr) {
  static_assert(OFF >= 0 && OFF < 65536, "16-bit LDS offset");
  bf16x8 r;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF));
  return r;
}
template <int N>
__device__ __forceinline__ void lds_wait_k(bf16x8& a) {
  static_assert(N >= 0 && N < 16, "lgkmcnt is 4 bits");
  asm volatile("s_waitcnt lgkmcnt(%1)" : "+v"(a) : "i"(N));
}

// Row sum of one chunk's probabilities beyond which the chunk loop moves the
// reference max (see RowBlock::chunk): probabilities stay below 2^24, far
// inside the fp32 range of the accumulators, and bf16 rounding is relative.
constexpr float kLazyBound = 16777216.0f;

// Initial running max: finite, so that exp2(s*c - m) of a masked score
// (s = -inf) is exactly 0 even before a row has seen a valid key; the first
// valid chunk always triggers a rescale (by exp2(kMInit - m') = 0).
constexpr float kMInit = -1e30f;

// Two fp32 values rounded to a packed bf16 pair (one v_cvt_pk_bf16_f32).
typedef float floatx2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
  const floatx2 f = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2));
}

// fp32 value split into two bf16 terms: hi = bf16(x), lo = bf16(x - hi).
// hi + lo carries 16 significant bits (|x - hi - lo| <= 2^-17 |x|), so a bf16
// MFMA against an exact bf16 operand, run on both terms, gives fp32-level
// products (the hi/lo form of fp32 GEMM emulation on bf16 matrix cores).
__device__ __forceinline__ void split_bf16(float x, bf16& hi, bf16& lo) {
  hi = (bf16)x;
  lo = (bf16)(x - (float)hi);
}

// Product of two packed bf16 pairs, rounded to a packed bf16 pair: each half
// widened by a shift or a mask, multiplied in fp32 (exact for bf16 inputs)
// and rounded to nearest-even once -- bf16(float(a) * float(b)) per half.
__device__ __forceinline__ uint32_t mul_bf16_pair(uint32_t a2, uint32_t b2) {
  const float lo = __uint_as_float(a2 << 16) * __uint_as_float(b2 << 16);
  const float hi = __uint_as_float(a2 & 0xffff0000u) * __uint_as_float(b2 & 0xffff0000u);
  return pack_bf16(lo, hi);
}

// Packed probability pair and its low-order remainder: (p0, p1) -> bf16
// pairs hi and lo with p = hi + lo to 2^-17 relative.
__device__ __forceinline__ void pack_bf16_split(float p0, float p1, uint32_t& hi, uint32_t& lo) {
  hi = pack_bf16(p0, p1);
  const float h0 = __uint_as_float(hi << 16), h1 = __uint_as_float(hi & 0xffff0000u);
  lo = pack_bf16(p0 - h0, p1 - h1);
}

// Per-wave state for 32 A rows.  HL (fp32 queries over bf16 keys, the
// reference's fp32 rounding points: a = q ⊙ k1 kept in fp32,
// simplicial_paged.py:45, and P kept in fp32 for P·V2): A and P carry a
// low-order bf16 term and every score and output MFMA runs on both terms.
//
// The softmax keeps ONE running reference max for the wave's 32 rows (the
// joint softmax of the reference has one max per query and head, and every
// row of the wave belongs to the same query and head), moved lazily, by a
// two-level rule.  The chunk loop (chunk) computes probabilities against the
// current reference without a chunk maximum, except in the wave's first chunk
// with a valid key (the reference is still kMInit there); only when some
// row's chunk sum passes kLazyBound = 2^24 (a score far above the reference,
// an overflow) does it take the chunk maxima and call rescale,
// which moves the reference only when a row's maximum exceeds it by more than
// 8 in the log2 domain (a factor 2^8), and then to the largest such maximum,
// and recomputes the chunk.  The pipelined step (step) calls rescale with
// every chunk's maximum.  Rows outside the query's short window get p = 0
// through an infinite exponent bias.
//
// OT selects the output layout.  !OT: O^T = V^T · P^T, lane = A row n,
// registers = d (32*db + acc_row(r, half)).  OT: O = P · V (the same two
// operand registers, swapped), lane = d (32*db + lane % 32), registers =
// rows n (acc_row(r, half)): the epilogue's sum over rows then runs inside
// each lane.
//
// KL (fp32 keys and values): every K and V tile row holds the row's hi terms
// followed by its lo terms ([hi: DK | lo: DK] and [hi: DV | lo: DV] bf16, the
// fp32 row split by split_bf16), and each product runs on three term pairs
// (hi*hi + hi*lo + lo*hi); requires HL.
// A load through the global address space.  From a pointer the compiler
// cannot place (e.g. a select between a tensor row and a static table) it
// would emit a flat load, which also counts against the LDS/scalar wait
// counter, so that unrelated LDS waits then wait for it.
template <typename T>
__device__ __forceinline__ T load_global(const void* p) {
  return *(const __attribute__((address_space(1))) T*)p;
}

template <int DK, int DV, bool HL = false, bool OT = false, bool KL = false>
struct RowBlock {
  static_assert(!KL || HL, "fp32 keys and values need the low-order A and P terms");
  bf16x8 a[DK / 16];    // A^T fragments (B operand of S^T = K·A^T)
  bf16x8 al[HL ? DK / 16 : 1];  // HL: low-order terms of the A^T fragments
  floatx16 o[DV / 32];  // output accumulators (layout: see OT)
  float m;              // reference max of the joint softmax (log2 domain), wave-uniform
  float mb;             // exponent bias of this lane's row: m inside the window, +inf outside
  bool valid;           // this lane's row lies inside the short window (a lane mask)
  float z;              // running sum of this lane's 16 keys per chunk (halves added at the end)

  // S^T += K_frag · A_t^T (both terms under HL)
  __device__ __forceinline__ floatx16 qk_mfma(const bf16x8& kf, int t, const floatx16& s) const {
    floatx16 r = mfma32x32x16(kf, a[t], s);
    if constexpr (HL) r = mfma32x32x16(kf, al[t], r);
    return r;
  }

  // O += P · V (OT) or O^T += V^T · P^T (!OT) for one 16-key step
  __device__ __forceinline__ floatx16 pv_mfma(const bf16x8& vf, const bf16x8& pb, const floatx16& acc) const {
    if constexpr (OT) return mfma32x32x16(pb, vf, acc);
    else return mfma32x32x16(vf, pb, acc);
  }

  // valid: this lane's A row lies inside the query's short window
  __device__ __forceinline__ void reset(bool row_valid) {
#pragma unroll
    for (int i = 0; i < DV / 32; ++i) o[i] = floatx16{};
    m = kMInit;
    valid = row_valid;
    mb = valid ? m : INFINITY;
    z = 0.f;
  }

  // A rows of this wave: a_j = bf16(q ⊙ k1_j) for the lane's short-axis key,
  // zero where `valid` is false (q_neg flips the sign of q, which keeps the
  // softmax scale non-negative).  Split in two so that callers can issue
  // other loads between the fragment loads and their first use: load_a
  // reads the 2*DK/16 fragments (q and k1 must point at readable rows in
  // every lane), make_a forms the bf16 products.
  struct AInputs {
    bf16x8 q[DK / 16], k[DK / 16];
  };
  __device__ static __forceinline__ AInputs load_a(const bf16* __restrict__ q, const bf16* __restrict__ k1,
                                                   int half) {
    AInputs in;
#pragma unroll
    for (int t = 0; t < DK / 16; ++t) {
      const int d0 = 16 * t + 8 * half;
      in.q[t] = load_global<bf16x8>(q + d0);
      in.k[t] = load_global<bf16x8>(k1 + d0);
    }
    return in;
  }
  // The sign flip and the row mask act on the packed product
  // (bf16(-x) == -bf16(x)): no per-element selects.
  __device__ static __forceinline__ uint32_t mul_pair(uint32_t q2, uint32_t k2, uint32_t sgn, uint32_t keep) {
    return (mul_bf16_pair(q2, k2) ^ sgn) & keep;
  }
  __device__ __forceinline__ void make_a(const AInputs& in, bool valid, bool q_neg) {
    const uint32_t sgn = q_neg ? 0x80008000u : 0u, keep = valid ? 0xffffffffu : 0u;
#pragma unroll
    for (int t = 0; t < DK / 16; ++t) {
      const u32x4 qw = __builtin_bit_cast(u32x4, in.q[t]), kw = __builtin_bit_cast(u32x4, in.k[t]);
      u32x4 r;
#pragma unroll
      for (int e = 0; e < 4; ++e) r[e] = mul_pair(qw[e], kw[e], sgn, keep);
      a[t] = __builtin_bit_cast(bf16x8, r);
    }
  }
  // The same for callers whose lanes outside the window read a row of zeros
  // (no row mask), with the sign flip a compile-time choice.
  template <bool NEG>
  __device__ __forceinline__ void make_a_unmasked(const AInputs& in) {
#pragma unroll
    for (int t = 0; t < DK / 16; ++t) {
      const u32x4 qw = __builtin_bit_cast(u32x4, in.q[t]), kw = __builtin_bit_cast(u32x4, in.k[t]);
      u32x4 r;
#pragma unroll
      for (int e = 0; e < 4; ++e) r[e] = mul_pair(qw[e], kw[e], NEG ? 0x80008000u : 0u, 0xffffffffu);
      a[t] = __builtin_bit_cast(bf16x8, r);
    }
  }
  __device__ __forceinline__ void form_a(const bf16* __restrict__ q, const bf16* __restrict__ k1, bool valid,
                                         int half, bool q_neg) {
    make_a(load_a(q, k1, half), valid, q_neg);
  }
  // HL: a_j = q ⊙ k1_j with an fp32 query, split into hi + lo terms.
  // K1 = bf16 (paged caches) or float (fp32 prefill)
  template <typename K1>
  __device__ __forceinline__ void form_a_f32(const float* __restrict__ q, const K1* __restrict__ k1, bool valid,
                                             int half, bool q_neg) {
    static_assert(HL, "fp32 A rows need the low-order terms");
    floatx4 qv[DK / 16][2];
    float kv[DK / 16][8];
#pragma unroll
    for (int t = 0; t < DK / 16; ++t) {
      const int d0 = 16 * t + 8 * half;
      qv[t][0] = *(const floatx4*)(q + d0);
      qv[t][1] = *(const floatx4*)(q + d0 + 4);
      if constexpr (std::is_same_v<K1, float>) {
        const floatx4 k0 = *(const floatx4*)(k1 + d0), k4 = *(const floatx4*)(k1 + d0 + 4);
#pragma unroll
        for (int u = 0; u < 4; ++u) kv[t][u] = k0[u], kv[t][u + 4] = k4[u];
      } else {
        const bf16x8 kb = *(const bf16x8*)(k1 + d0);
#pragma unroll
        for (int u = 0; u < 8; ++u) kv[t][u] = (float)kb[u];
      }
    }
#pragma unroll
    for (int t = 0; t < DK / 16; ++t) {
      bf16x8 h, l;
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        float x = qv[t][u >> 2][u & 3] * kv[t][u];
        if (q_neg) x = -x;
        bf16 xh, xl;
        split_bf16(valid ? x : 0.f, xh, xl);
        h[u] = xh;
        l[u] = xl;
      }
      a[t] = h;
      al[t] = l;
    }
  }
  // The wave's q row (DK bf16 at qrow, in LDS) widened to DK fp32 values at
  // qf (LDS), negated when q_neg; each lane widens DK / 64 of them.  A wave's
  // LDS accesses execute in order, so its lanes may read qf right after (no
  // barrier), and form_a_qf then multiplies without unpacking q per lane.
  __device__ static __forceinline__ void widen_q(const char* qrow, char* qf, int lane, bool q_neg) {
    constexpr int W = DK >= 128 ? DK / 128 : 1;  // packed words per lane
    constexpr int LANES = DK / 2 / W;            // lanes with words (all but DK = 64)
    static_assert(W == 1 || W == 2 || W == 4, "widths 64 .. 512");
    const uint32_t sgn = q_neg ? 0x80000000u : 0u;
    if (LANES == 64 || lane < LANES) {
      uint32_t w[W];
      if constexpr (W == 4) {
        const u32x4 x = *(const u32x4*)(qrow + 16 * lane);
#pragma unroll
        for (int e = 0; e < 4; ++e) w[e] = x[e];
      } else if constexpr (W == 2) {
        const uint2 x = *(const uint2*)(qrow + 8 * lane);
        w[0] = x.x, w[1] = x.y;
      } else {
        w[0] = *(const uint32_t*)(qrow + 4 * lane);
      }
      float f[2 * W];
#pragma unroll
      for (int e = 0; e < W; ++e) {
        f[2 * e] = __uint_as_float((w[e] << 16) ^ sgn);
        f[2 * e + 1] = __uint_as_float((w[e] & 0xffff0000u) ^ sgn);
      }
      float* dst = (float*)qf + 2 * W * lane;
      if constexpr (W == 1) {
        *(floatx2*)dst = floatx2{f[0], f[1]};
      } else {
#pragma unroll
        for (int e = 0; e < W / 2; ++e) *(floatx4*)(dst + 4 * e) = floatx4{f[4 * e], f[4 * e + 1], f[4 * e + 2], f[4 * e + 3]};
      }
    }
  }
  // A rows from the lane's staged k1 row (krow, DK bf16) and the wave's
  // widened q row (qf, DK fp32 with the sign of q_neg applied): the products
  // of the same operands as form_a_lds, so the same bits.  Fragments are read
  // in groups (bounded register footprint).
  __device__ __forceinline__ void form_a_qf(const char* krow, const char* qf, bool valid, int half) {
    constexpr int GRP = DK / 16 < 4 ? DK / 16 : 4;
    const uint32_t keep = valid ? 0xffffffffu : 0u;
#pragma unroll
    for (int t0 = 0; t0 < DK / 16; t0 += GRP) {
      floatx4 qv[GRP][2];
      u32x4 kv[GRP];
#pragma unroll
      for (int u = 0; u < GRP; ++u) {
        const char* qp = qf + 4 * (16 * (t0 + u) + 8 * half);
        qv[u][0] = *(const floatx4*)qp;
        qv[u][1] = *(const floatx4*)(qp + 16);
        kv[u] = *(const u32x4*)(krow + 32 * (t0 + u) + 16 * half);
      }
#pragma unroll
      for (int u = 0; u < GRP; ++u) {
        u32x4 r;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float lo = qv[u][e >> 1][2 * (e & 1)] * __uint_as_float(kv[u][e] << 16);
          const float hi = qv[u][e >> 1][2 * (e & 1) + 1] * __uint_as_float(kv[u][e] & 0xffff0000u);
          r[e] = pack_bf16(lo, hi) & keep;
        }
        a[t0 + u] = __builtin_bit_cast(bf16x8, r);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  // The same from rows staged in LDS: krow = the lane's k1 row, qrow = the
  // wave's q row (both DK contiguous bf16).
  // Fragments are read in groups of 4 (bounded register footprint).
  __device__ __forceinline__ void form_a_lds(const char* krow, const char* qrow, bool valid, int half, bool q_neg) {
    constexpr int GRP = DK / 16 < 4 ? DK / 16 : 4;
#pragma unroll
    for (int t0 = 0; t0 < DK / 16; t0 += GRP) {
      bf16x8 qv[GRP], kv[GRP];
#pragma unroll
      for (int u = 0; u < GRP; ++u) {
        qv[u] = *(const bf16x8*)(qrow + 32 * (t0 + u) + 16 * half);
        kv[u] = *(const bf16x8*)(krow + 32 * (t0 + u) + 16 * half);
      }
      const uint32_t sgn = q_neg ? 0x80008000u : 0u, keep = valid ? 0xffffffffu : 0u;
#pragma unroll
      for (int u = 0; u < GRP; ++u) {
        const u32x4 qw = __builtin_bit_cast(u32x4, qv[u]), kw = __builtin_bit_cast(u32x4, kv[u]);
        u32x4 r;
#pragma unroll
        for (int e = 0; e < 4; ++e) r[e] = mul_pair(qw[e], kw[e], sgn, keep);
        a[t0 + u] = __builtin_bit_cast(bf16x8, r);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  // The two transposing reads of V fragment `step` (t = step / (DV/32) selects
  // keys 16t.., db = step % (DV/32) the 32-wide d block).
  template <int RS, int STEP, int XB = 0>
  __device__ static __forceinline__ void vread(uint32_t vp, shortx4& v1, shortx4& v2) {
    constexpr int t = STEP / (DV / 32), db = STEP % (DV / 32);
    constexpr int off = 16 * t * RS + 64 * db + XB;  // XB: extra bytes into the row (KL: the lo terms)
    v1 = ds_read_tr16<off>(vp);
    v2 = ds_read_tr16<off + 8 * RS>(vp);
  }

  // One 32-key chunk: tile rows row0 .. row0+31 of the K tile at `ktile` (row
  // stride RSK bytes) and the V tile at `vtile` (row stride RSV).  sl2 = |scale|*log2(e) >= 0.
  // key_lo/key_hi: range of valid chunk keys (0..31) for this wave's query;
  // masking is applied only when the chunk is not fully valid.
  // PF: V fragments read that many PV MFMAs ahead (1: each read is waited
  // for right after the MFMA before it).
  template <int RSK, int RSV, int PF = 1>
  __device__ __forceinline__ void chunk(const char* ktile, const char* vtile, int row0, int lane, float sl2,
                                        int key_lo, int key_hi, bool first = false) {
    const int n = lane & 31, half = lane >> 5;
    floatx16 s = floatx16{};
    {
      // K fragments are read two steps ahead of their MFMA (one ahead measured
      // 0.5-0.9 % slower at widths of 128; four at score width 512, one wave
      // per SIMD with accumulation registers to spare: DS 512 6.20 -> 6.14
      // ms); the scheduling barriers stop the compiler from hoisting all DK/16
      // reads (which would hold DK/4 extra VGPRs live).
      const char* kp = ktile + (row0 + n) * RSK + 16 * half;
      if constexpr (KL) {
#pragma unroll
        for (int t = 0; t < DK / 16; ++t) {
          const bf16x8 kh = *(const bf16x8*)(kp + 32 * t), kl = *(const bf16x8*)(kp + 2 * DK + 32 * t);
          __builtin_amdgcn_sched_barrier(0);
          s = mfma32x32x16(kh, a[t], s);
          s = mfma32x32x16(kh, al[t], s);
          s = mfma32x32x16(kl, a[t], s);
          __builtin_amdgcn_sched_barrier(0);
        }
      } else {
        bf16x8 kq[DK / 16];
        constexpr int KA = DK >= 512 ? 4 : 2;  // fragments read ahead
        // explicit reads and counted waits (ds_read_b128_at)
        const uint32_t ka = lds_addr(kp);
        static_for<0, (KA < DK / 16 ? KA : DK / 16)>(
            [&](auto tt) { kq[tt] = ds_read_b128_at<32 * decltype(tt)::value>(ka); });
        static_for<0, DK / 16>([&](auto tt) {
          constexpr int t = decltype(tt)::value;
          if constexpr (t + KA < DK / 16) kq[t + KA] = ds_read_b128_at<32 * (t + KA)>(ka);
          lds_wait_k<(t + KA < DK / 16 ? t + KA : DK / 16 - 1) - t>(kq[t]);
          __builtin_amdgcn_sched_barrier(0);
          s = qk_mfma(kq[t], t, s);
          __builtin_amdgcn_sched_barrier(0);
        });
      }
    }
    const bool masked = key_lo > 0 || key_hi < kChunk - 1;
    // register r holds chunk key 8*(r/4) + r%4 + 4*half: compare the
    // compile-time part against bounds shifted by 4*half
    const int lo_h = key_lo - 4 * half, hi_h = key_hi - 4 * half;
    if (masked) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int kr = 8 * (r >> 2) + (r & 3);
        if (kr < lo_h || kr > hi_h) s[r] = -INFINITY;
      }
    }
    // Probabilities against the current reference max, with no chunk maximum:
    // masked scores are -inf and give exactly 0 (sl2 > 0).  Only when a row's
    // sum passes kLazyBound (a score above the reference by about 2^20, the
    // first valid chunk of a row, or an overflow to inf) does the wave take
    // the chunk maxima, move the reference (rescale) and recompute the chunk.
    float zs;
    uint32_t pk[8], pkl[HL ? 8 : 1];
    auto probs = [&]() {
#pragma unroll
      for (int r = 0; r < 16; r += 2) {
        const float p0 = fast_exp2(fmaf(s[r], sl2, -mb)), p1 = fast_exp2(fmaf(s[r + 1], sl2, -mb));
        zs = r == 0 ? p0 + p1 : zs + (p0 + p1);
        if constexpr (HL) pack_bf16_split(p0, p1, pk[r >> 1], pkl[r >> 1]);
        else pk[r >> 1] = pack_bf16(p0, p1);
      }
    };
    auto move_reference = [&]() {
      float rmax = -INFINITY;
#pragma unroll
      for (int r = 0; r < 16; ++r) rmax = fmaxf(rmax, s[r]);
      rescale(pair_max(rmax) * sl2);
    };
    // Until the wave's first chunk with a valid key the reference is kMInit,
    // against which every valid probability overflows: in that chunk (`first`,
    // a uniform flag from the caller's chunk index) take the maxima before the
    // probabilities instead of after -- the same reference, one pass of
    // exponentials instead of two.
    if (first) move_reference();
    probs();
    if (__builtin_amdgcn_ballot_w64(!(zs <= kLazyBound)) != 0ull) {
      move_reference();
      probs();
    }
    z += zs;
    const bf16x8 pb[2] = {__builtin_bit_cast(bf16x8, u32x4{pk[0], pk[1], pk[2], pk[3]}),
                          __builtin_bit_cast(bf16x8, u32x4{pk[4], pk[5], pk[6], pk[7]})};
    bf16x8 pbl[2];
    if constexpr (HL) {
      pbl[0] = __builtin_bit_cast(bf16x8, u32x4{pkl[0], pkl[1], pkl[2], pkl[3]});
      pbl[1] = __builtin_bit_cast(bf16x8, u32x4{pkl[4], pkl[5], pkl[6], pkl[7]});
    }

    // V^T operand through the transposing read: within each 16-lane group,
    // source lane (4e + q) fetches 4 consecutive d of row (key e); output lane
    // i then holds d = d0 + i for the 4 keys.  Lane l ends with d = 32*db + l%32
    // and keys 16t + 4*half + {0..3} (+8 for the second read).
    const int g16 = (lane >> 4) & 1, i16 = lane & 15;
    const int e_src = i16 >> 2, q_src = i16 & 3;
    const uint32_t vp = lds_addr(vtile + (row0 + 4 * half + e_src) * RSV + 32 * g16 + 8 * q_src);
    constexpr int kSteps = 2 * (DV / 32);
    if constexpr (KL) {
      // three term pairs per step: P_hi*V_hi + P_lo*V_hi + P_hi*V_lo
      static_for<0, kSteps>([&](auto st) {
        constexpr int step = decltype(st)::value;
        shortx4 h1, h2, l1, l2;
        vread<RSV, step>(vp, h1, h2);
        vread<RSV, step, 2 * DV>(vp, l1, l2);
        lds_wait(h1, h2);
        lds_wait(l1, l2);
        const bf16x8 vh = __builtin_bit_cast(bf16x8, shortx8{h1[0], h1[1], h1[2], h1[3], h2[0], h2[1], h2[2], h2[3]});
        const bf16x8 vl = __builtin_bit_cast(bf16x8, shortx8{l1[0], l1[1], l1[2], l1[3], l2[0], l2[1], l2[2], l2[3]});
        __builtin_amdgcn_sched_barrier(0);
        o[step % (DV / 32)] = pv_mfma(vh, pb[step / (DV / 32)], o[step % (DV / 32)]);
        o[step % (DV / 32)] = pv_mfma(vh, pbl[step / (DV / 32)], o[step % (DV / 32)]);
        o[step % (DV / 32)] = pv_mfma(vl, pb[step / (DV / 32)], o[step % (DV / 32)]);
        __builtin_amdgcn_sched_barrier(0);
      });
      return;
    }
    if constexpr (PF > 1) {
      shortx4 va[kSteps], vb[kSteps];
      static_for<0, (PF < kSteps ? PF : kSteps)>([&](auto q) { vread<RSV, decltype(q)::value>(vp, va[q], vb[q]); });
      static_for<0, kSteps>([&](auto st) {
        constexpr int step = decltype(st)::value;
        if constexpr (step + PF < kSteps) vread<RSV, step + PF>(vp, va[step + PF], vb[step + PF]);
        constexpr int later = (step + PF < kSteps ? step + PF : kSteps - 1) - step;  // read pairs issued after
        lds_wait_n<2 * later>(va[step], vb[step]);
        shortx8 vv = {va[step][0], va[step][1], va[step][2], va[step][3],
                      vb[step][0], vb[step][1], vb[step][2], vb[step][3]};
        const bf16x8 vf = __builtin_bit_cast(bf16x8, vv);
        __builtin_amdgcn_sched_barrier(0);
        o[step % (DV / 32)] = pv_mfma(vf, pb[step / (DV / 32)], o[step % (DV / 32)]);
        if constexpr (HL) o[step % (DV / 32)] = pv_mfma(vf, pbl[step / (DV / 32)], o[step % (DV / 32)]);
        __builtin_amdgcn_sched_barrier(0);
      });
      return;
    }
    // V fragments are read one step ahead of their MFMA
    shortx4 v1, v2;
    vread<RSV, 0>(vp, v1, v2);
    lds_wait(v1, v2);
    static_for<0, kSteps>([&](auto st) {
      constexpr int step = decltype(st)::value;
      shortx8 vv = {v1[0], v1[1], v1[2], v1[3], v2[0], v2[1], v2[2], v2[3]};
      const bf16x8 vf = __builtin_bit_cast(bf16x8, vv);
      shortx4 n1, n2;
      if constexpr (step + 1 < kSteps) vread<RSV, step + 1>(vp, n1, n2);
      __builtin_amdgcn_sched_barrier(0);
      o[step % (DV / 32)] = pv_mfma(vf, pb[step / (DV / 32)], o[step % (DV / 32)]);
      if constexpr (HL) o[step % (DV / 32)] = pv_mfma(vf, pbl[step / (DV / 32)], o[step % (DV / 32)]);
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (step + 1 < kSteps) {
        lds_wait(n1, n2);
        v1 = n1;
        v2 = n2;
      }
    });
  }

  // ---- Software-pipelined form -------------------------------------------
  // A key chunk is processed in two phases that each pair one group of
  // MFMAs with VALU work that does not depend on it:
  //   phase 1: QK^T MFMAs of chunk c+1  ||  probabilities of chunk c
  //   phase 2: PV MFMAs of chunk c      ||  row maxima of chunk c+1
  // Scheduling barriers keep the instructions in this order, so the VALU
  // work of a wave issues while its own MFMAs occupy the matrix core.

  // Raw scores of one chunk (pipeline prologue; no interleaving).
  template <int RSK>
  __device__ __forceinline__ floatx16 qk(const char* ktile, int row0, int lane) const {
    const int n = lane & 31, half = lane >> 5;
    const char* kp = ktile + (row0 + n) * RSK + 16 * half;
    floatx16 s = floatx16{};
#pragma unroll
    for (int t = 0; t < DK / 16; ++t) s = qk_mfma(*(const bf16x8*)(kp + 32 * t), t, s);
    return s;
  }

  // Row maximum of a score tile (both halves), unscaled.
  __device__ static __forceinline__ float row_max(const floatx16& s) {
    float r = fmaxf(s[0], s[1]);
#pragma unroll
    for (int i = 2; i < 16; i += 2) r = fmaxf(r, fmaxf(s[i], s[i + 1]));
    return pair_max(r);
  }

  // Scores of keys outside [key_lo, key_hi] (chunk-relative) become -inf.
  __device__ static __forceinline__ void mask(floatx16& s, int lane, int key_lo, int key_hi) {
    const int half = lane >> 5;
    const int lo_h = key_lo - 4 * half, hi_h = key_hi - 4 * half;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int kr = 8 * (r >> 2) + (r & 3);
      if (kr < lo_h || kr > hi_h) s[r] = -INFINITY;
    }
  }

  // Lazy rescale: move the wave's reference max only when some row's scaled
  // chunk max `cmax` (rows outside the window excluded, log2 domain) exceeds
  // it by more than 8 (a factor 2^8); then to the largest such max, and every
  // row is rescaled by the same factor.
  __device__ __forceinline__ void rescale(float cmax) {
    const float cand = valid ? cmax : -INFINITY;
    const bool grow = cand > m + 8.0f;
    if (__builtin_amdgcn_ballot_w64(grow) != 0ull) {
      const float mn = fmaxf(m, uniform_f(wave_max(cand)));
      if (m != kMInit) {  // before the first move nothing has been accumulated: o = 0, z = 0
        const float alpha = fast_exp2(m - mn);
#pragma unroll
        for (int i = 0; i < DV / 32; ++i) o[i] *= alpha;
        z *= alpha;
      }
      m = mn;
      mb = valid ? m : INFINITY;
    }
  }

  // One pipelined chunk.  On entry `s` holds chunk c's scores (masked) and
  // the rescale for chunk c has been applied.  With NEXT, the QK^T of chunk
  // c+1 (K tile `knext`) is computed into `s` and its scaled row max into
  // `cmax`.  `vtile` is chunk c's V tile; both tiles use rows row0.. .
  // PF: V fragments read that many PV MFMAs ahead (the first PF issued before
  // phase 1); 1 waits for each read right after the MFMA before it.
  template <int RSK, int RSV, bool NEXT, int PF = 1>
  __device__ __forceinline__ void step(floatx16& s, float& cmax, const char* knext, const char* vtile, int row0,
                                       int lane, float sl2) {
    const int n = lane & 31, half = lane >> 5;
    constexpr int NT = DK / 16;   // QK^T MFMAs
    floatx16 sn = floatx16{};
    uint32_t pk[8];              // P^T as packed bf16 pairs (B operand of the PV MFMAs)
    uint32_t pkl[HL ? 8 : 1];    // HL: their low-order terms
    float zs = 0.f;

    // V^T operand addresses (see vread); the first pair is issued now
    const int g16 = (lane >> 4) & 1, i16 = lane & 15;
    const int e_src = i16 >> 2, q_src = i16 & 3;
    const uint32_t vp = lds_addr(vtile + (row0 + 4 * half + e_src) * RSV + 32 * g16 + 8 * q_src);
    constexpr int kSteps = 2 * (DV / 32);
    constexpr int kPre = PF < kSteps ? PF : kSteps;
    shortx4 v1, v2, va[kSteps], vb[kSteps];
    if constexpr (PF > 1) static_for<0, kPre>([&](auto q) { vread<RSV, decltype(q)::value>(vp, va[q], vb[q]); });
    else vread<RSV, 0>(vp, v1, v2);

    // phase 1
    const char* kp = knext + (row0 + n) * RSK + 16 * half;
    bf16x8 kf;
    if constexpr (NEXT) kf = *(const bf16x8*)kp;
    static_for<0, NT>([&](auto tt) {
      constexpr int t = decltype(tt)::value;
      bf16x8 kn;
      if constexpr (NEXT) {
        if constexpr (t + 1 < NT) kn = *(const bf16x8*)(kp + 32 * (t + 1));
        __builtin_amdgcn_sched_barrier(0);
        sn = qk_mfma(kf, t, sn);
      }
      __builtin_amdgcn_sched_barrier(0);
      // probability pair pi (scores 2pi, 2pi+1) goes with QK^T MFMA pi * NT / 8
      static_for<0, 8>([&](auto pp) {
        constexpr int pi = decltype(pp)::value;
        if constexpr (pi * NT / 8 == t) {
          const float p0 = fast_exp2(fmaf(s[2 * pi], sl2, -mb)), p1 = fast_exp2(fmaf(s[2 * pi + 1], sl2, -mb));
          zs += p0 + p1;
          if constexpr (HL) pack_bf16_split(p0, p1, pk[pi], pkl[pi]);
          else pk[pi] = pack_bf16(p0, p1);
        }
      });
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (NEXT && t + 1 < NT) kf = kn;
    });
    z += zs;
    const bf16x8 pb0 = __builtin_bit_cast(bf16x8, u32x4{pk[0], pk[1], pk[2], pk[3]});
    const bf16x8 pb1 = __builtin_bit_cast(bf16x8, u32x4{pk[4], pk[5], pk[6], pk[7]});
    bf16x8 pbl0, pbl1;
    if constexpr (HL) {
      pbl0 = __builtin_bit_cast(bf16x8, u32x4{pkl[0], pkl[1], pkl[2], pkl[3]});
      pbl1 = __builtin_bit_cast(bf16x8, u32x4{pkl[4], pkl[5], pkl[6], pkl[7]});
    }

    // phase 2
    float rmax = -INFINITY;
    if constexpr (PF > 1) {
      static_for<0, kSteps>([&](auto st) {
        constexpr int step = decltype(st)::value;
        if constexpr (step + PF < kSteps) vread<RSV, step + PF>(vp, va[step + PF], vb[step + PF]);
        constexpr int later = (step + PF < kSteps ? step + PF : kSteps - 1) - step;  // read pairs issued after
        lds_wait_n<2 * later>(va[step], vb[step]);
        shortx8 vv = {va[step][0], va[step][1], va[step][2], va[step][3],
                      vb[step][0], vb[step][1], vb[step][2], vb[step][3]};
        const bf16x8 vf = __builtin_bit_cast(bf16x8, vv);
        __builtin_amdgcn_sched_barrier(0);
        o[step % (DV / 32)] = pv_mfma(vf, step / (DV / 32) == 0 ? pb0 : pb1, o[step % (DV / 32)]);
        if constexpr (HL)
          o[step % (DV / 32)] = pv_mfma(vf, step / (DV / 32) == 0 ? pbl0 : pbl1, o[step % (DV / 32)]);
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (NEXT) {
          static_for<0, 16>([&](auto vv2) {
            constexpr int v = decltype(vv2)::value;
            if constexpr (v * kSteps / 16 == step) rmax = fmaxf(rmax, sn[v]);
          });
        }
        __builtin_amdgcn_sched_barrier(0);
      });
      if constexpr (NEXT) {
        cmax = pair_max(rmax) * sl2;
        s = sn;
      }
      return;
    }
    lds_wait(v1, v2);
    static_for<0, kSteps>([&](auto st) {
      constexpr int step = decltype(st)::value;
      shortx8 vv = {v1[0], v1[1], v1[2], v1[3], v2[0], v2[1], v2[2], v2[3]};
      const bf16x8 vf = __builtin_bit_cast(bf16x8, vv);
      shortx4 n1, n2;
      if constexpr (step + 1 < kSteps) vread<RSV, step + 1>(vp, n1, n2);
      __builtin_amdgcn_sched_barrier(0);
      o[step % (DV / 32)] = pv_mfma(vf, step / (DV / 32) == 0 ? pb0 : pb1, o[step % (DV / 32)]);
      if constexpr (HL) o[step % (DV / 32)] = pv_mfma(vf, step / (DV / 32) == 0 ? pbl0 : pbl1, o[step % (DV / 32)]);
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (NEXT) {  // score v of the next chunk is folded in at PV MFMA v * kSteps / 16
        static_for<0, 16>([&](auto vv2) {
          constexpr int v = decltype(vv2)::value;
          if constexpr (v * kSteps / 16 == step) rmax = fmaxf(rmax, sn[v]);
        });
      }
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (step + 1 < kSteps) {
        lds_wait(n1, n2);
        v1 = n1;
        v2 = n2;
      }
    });
    if constexpr (NEXT) {
      cmax = pair_max(rmax) * sl2;
      s = sn;
    }
  }
};

}  // namespace sa
