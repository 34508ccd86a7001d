// Wave-level MFMA core shared by the bf16 prefill and paged kernels.
//
// A wave owns 32 "A rows" (one query token x one head x up to 32 short-axis
// keys j).  Lane l holds row n = l % 32 and half h = l / 32.  Per 32-key chunk
// of the long axis staged in LDS:
//
//   S^T = K_chunk · A^T     D/16 v_mfma_f32_32x32x16_bf16, K rows from LDS
//   P^T = exp2(S^T*c - m)   per-row online softmax, lazy rescale
//   O^T += V^T · P^T        D/32 x 2 MFMAs; the V^T operand is read from the
//                           natural [key][d] tile with ds_read_b64_tr_b16
//
// LDS tiles: K and V, each [rows][D] bf16, row-major, no padding.  The
// 16-byte segment s of row r is stored at segment s ^ (r & SWZ) so that the
// 32 lanes reading one segment of 32 consecutive rows hit distinct banks.
//
// Tiles are filled with global_load_lds_dwordx4 (16 bytes per lane straight
// into LDS, no staging registers); each DMA instruction covers 512/D rows.
// The compiler does not order these DMA writes against later LDS reads, so
// the kernels wait explicitly (vmcnt) before the barrier that publishes a tile.
#pragma once

#include "sa_common.h"

namespace sa {

typedef short shortx4 __attribute__((ext_vector_type(4)));
typedef short shortx8 __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(3))) shortx4 lds_shortx4;

template <int D>
struct Tile {
  static constexpr int kSegs = D / 8;                         // 16-byte segments per row
  static constexpr int kSwz = (kSegs < 16 ? kSegs : 16) - 1;  // XOR mask of the segment swizzle
  static constexpr int kRowBytes = 2 * D;
  static constexpr int kRowsPerDma = 512 / D;                 // rows one 64-lane DMA instruction covers
  __device__ static __forceinline__ int swz(int row) { return row & kSwz; }
  __device__ static __forceinline__ int seg_off(int row, int seg) { return row * kRowBytes + ((seg ^ swz(row)) << 4); }
};

// Smallest row count >= need that is a multiple of the DMA row granularity and
// whose K+V instruction count divides evenly over `waves` waves (uniform vmcnt).
template <int D>
__host__ __device__ constexpr int tile_rows(int need, int waves) {
  int rpi = 512 / D;
  int r = (need + rpi - 1) / rpi * rpi;
  while ((2 * r / rpi) % waves) r += rpi;
  return r;
}

// s_waitcnt vmcnt(n) with the other counters left alone (gfx9 encoding:
// vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt[5:4] << 14).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// Barrier without the memory fences of __syncthreads.  Ordering of the DMA
// writes comes from the explicit vmcnt waits; the waves' own LDS accesses are
// ordered by the lgkmcnt(0) wait issued here before s_barrier.
__device__ __forceinline__ void block_barrier() {
  __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (0 << 8) | (3 << 14));  // lgkmcnt(0) only
  __builtin_amdgcn_s_barrier();
}

// Issue the DMA loads of one K/V tile of ROWS rows into `slot` (K tile at
// slot, V tile at slot + ROWS*2D).  row_off(r, is_v) gives the element offset
// of tile row r in kbase / vbase (the caller maps rows outside the tensor to a
// valid row; such rows are masked out of the softmax).  Each of the NW waves
// issues exactly 2*ROWS/(512/D)/NW instructions.
template <int D, int ROWS, int NW, typename RowFn>
__device__ __forceinline__ void issue_tile(char* slot, const bf16* __restrict__ kbase, const bf16* __restrict__ vbase,
                                           int wid, int lane, RowFn row_off) {
  using T = Tile<D>;
  constexpr int per_tensor = ROWS / T::kRowsPerDma;
  constexpr int total = 2 * per_tensor;
  static_assert(ROWS % T::kRowsPerDma == 0 && total % NW == 0, "uniform DMA split");
  const int rsub = lane / T::kSegs;  // row within the instruction
  const int pseg = lane % T::kSegs;  // LDS segment position this lane fills
#pragma unroll
  for (int k = 0; k < total / NW; ++k) {
    const int i = wid + k * NW;
    const bool is_v = i >= per_tensor;
    const int rg = is_v ? i - per_tensor : i;
    const int row = rg * T::kRowsPerDma + rsub;
    const int gseg = pseg ^ T::swz(row);
    const bf16* src = (is_v ? vbase : kbase) + row_off(row, is_v) + gseg * 8;
    char* dst = slot + (is_v ? ROWS * T::kRowBytes : 0) + rg * T::kRowsPerDma * T::kRowBytes;
    __builtin_amdgcn_global_load_lds((const void*)src, (lds_void*)dst, 16, 0, 0);
  }
}

// Per-wave state for 32 A rows.
template <int D>
struct RowBlock {
  bf16x8 a[D / 16];     // A^T fragments (B operand of S^T = K·A^T)
  floatx16 o[D / 32];   // O^T accumulators, d-block db holds d = 32*db + acc_row(r, half)
  float m;              // running max (log2 domain), identical in both halves
  float z;              // running sum of this lane's 16 keys per chunk (halves added at the end)

  __device__ __forceinline__ void reset() {
#pragma unroll
    for (int i = 0; i < D / 32; ++i) o[i] = floatx16{};
    m = -INFINITY;
    z = 0.f;
  }

  // a_row = bf16(q ⊙ k1_row) for the lane's row; q_neg flips the sign of q
  // (used to keep the softmax scale non-negative).  k1 == nullptr -> zero row.
  __device__ __forceinline__ void form_a(const bf16* __restrict__ q, const bf16* __restrict__ k1, int half,
                                         bool q_neg) {
#pragma unroll
    for (int t = 0; t < D / 16; ++t) {
      if (k1 == nullptr) {
        a[t] = bf16x8{};
        continue;
      }
      const int d0 = 16 * t + 8 * half;
      bf16x8 qv = *(const bf16x8*)(q + d0);
      bf16x8 kv = *(const bf16x8*)(k1 + d0);
      bf16x8 r;
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        float x = (float)qv[u] * (float)kv[u];
        r[u] = (bf16)(q_neg ? -x : x);
      }
      a[t] = r;
    }
  }

  // One 32-key chunk: tile rows row0 .. row0+31 of the K tile at `ktile` and
  // the V tile at `vtile`.  sl2 = |scale|*log2(e) >= 0.  key_lo/key_hi: range
  // of valid chunk keys (0..31) for this wave's query; masking is applied only
  // when the chunk is not fully valid.
  __device__ __forceinline__ void chunk(const char* ktile, const char* vtile, int row0, int lane, float sl2,
                                        int key_lo, int key_hi) {
    using T = Tile<D>;
    const int n = lane & 31, half = lane >> 5;
    floatx16 s = floatx16{};
    {
      const int row = row0 + n;
#pragma unroll
      for (int t = 0; t < D / 16; ++t) {
        bf16x8 kf = *(const bf16x8*)(ktile + T::seg_off(row, 2 * t + half));
        s = mfma32x32x16(kf, a[t], s);
      }
    }
    const bool masked = key_lo > 0 || key_hi < kChunk - 1;
    // register r holds chunk key 8*(r/4) + r%4 + 4*half: compare the
    // compile-time part against bounds shifted by 4*half
    const int lo_h = key_lo - 4 * half, hi_h = key_hi - 4 * half;
    float rmax = -INFINITY;
    if (masked) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int kr = 8 * (r >> 2) + (r & 3);
        if (kr < lo_h || kr > hi_h) s[r] = -INFINITY;
        rmax = fmaxf(rmax, s[r]);
      }
    } else {
#pragma unroll
      for (int r = 0; r < 16; ++r) rmax = fmaxf(rmax, s[r]);
    }
    rmax = pair_max(rmax);
    const float cand = rmax * sl2;
    // Lazy rescale: keep the reference max unless some row grew by > 2^8.
    const bool grow = cand > m + 8.0f;
    if (__builtin_amdgcn_ballot_w64(grow) != 0ull) {
      const float mn = fmaxf(m, cand);
      const float alpha = fast_exp2(m - mn);
#pragma unroll
      for (int i = 0; i < D / 32; ++i) o[i] *= alpha;
      z *= alpha;
      m = mn;
    }
    float zs = 0.f;
    bf16x8 pb[2];
    if (masked) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int kr = 8 * (r >> 2) + (r & 3);
        const bool ok = kr >= lo_h && kr <= hi_h;
        const float p = ok ? fast_exp2(fmaf(s[r], sl2, -m)) : 0.f;
        zs += p;
        pb[r >> 3][r & 7] = (bf16)p;
      }
    } else {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = fast_exp2(fmaf(s[r], sl2, -m));
        zs += p;
        pb[r >> 3][r & 7] = (bf16)p;
      }
    }
    z += zs;
    // V^T operand through the transposing read: within each 16-lane group,
    // source lane (4e + q) fetches 4 consecutive d of row (key e); output lane
    // i then holds d = d0 + i for the 4 keys.  Lane l ends with d = 32*db + l%32
    // and keys 16t + 4*half + {0..3} (+8 for the second read).
    const int g16 = (lane >> 4) & 1, i16 = lane & 15;
    const int e_src = i16 >> 2, q_src = i16 & 3;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int r1 = row0 + 16 * t + 4 * half + e_src;
      const int r2 = r1 + 8;
#pragma unroll
      for (int db = 0; db < D / 32; ++db) {
        const int seg = 4 * db + 2 * g16 + (q_src >> 1);
        const int sub = (q_src & 1) * 8;
        shortx4 v1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_shortx4*)(vtile + T::seg_off(r1, seg) + sub));
        shortx4 v2 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_shortx4*)(vtile + T::seg_off(r2, seg) + sub));
        shortx8 vv = {v1[0], v1[1], v1[2], v1[3], v2[0], v2[1], v2[2], v2[3]};
        o[db] = mfma32x32x16(__builtin_bit_cast(bf16x8, vv), pb[t], o[db]);
      }
    }
  }
};

}  // namespace sa
