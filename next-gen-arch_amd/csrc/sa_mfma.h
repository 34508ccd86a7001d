// Wave-level MFMA core shared by the bf16 prefill and paged kernels.
//
// A wave owns 32 "A rows" (one query token x one head x up to 32 short-axis
// keys j).  Lane l holds row n = l % 32 and half h = l / 32.  Per 32-key chunk
// of the long axis staged in LDS:
//
//   S^T = K_chunk · A^T     8 (D=128) v_mfma_f32_32x32x16_bf16, K from LDS
//   P^T = exp2(S^T*c - m)   per-row online softmax, lazy rescale
//   O^T += V^T · P^T        D/32 x 2 MFMAs, V^T read from a transposed LDS tile
//
// LDS chunk layouts (bf16, no padding, XOR swizzles keep reads conflict-free):
//   K  [32 keys][D]   16-byte segment s of key k stored at segment s ^ (k & 15)
//   Vt [D][32 keys]   8-byte unit u (4 keys) of row d stored at unit u ^ ((d >> 2) & 7)
#pragma once

#include "sa_common.h"

namespace sa {

template <int D>
struct ChunkLayout {
  static constexpr int kSegs = D / 8;                       // 16-byte segments per K row
  static constexpr int kSwz = (kSegs < 16 ? kSegs : 16) - 1;
  static constexpr int kKBytes = kChunk * D * 2;            // K tile bytes
  static constexpr int kVBytes = D * kChunk * 2;            // V^T tile bytes
  static constexpr int kBytes = kKBytes + kVBytes;
  __device__ static __forceinline__ int k_off(int key, int seg) { return key * (D * 2) + ((seg ^ (key & kSwz)) << 4); }
  // byte offset of the dword holding keys (2p, 2p+1) of V^T row d
  __device__ static __forceinline__ int vt_pair_off(int d, int p) {
    return kKBytes + d * 64 + ((((p >> 1) ^ ((d >> 2) & 7))) << 3) + ((p & 1) << 2);
  }
  // byte offset of 8-byte unit u (keys 4u..4u+3) of V^T row d
  __device__ static __forceinline__ int vt_unit_off(int d, int u) {
    return kKBytes + d * 64 + ((u ^ ((d >> 2) & 7)) << 3);
  }
};

// Cooperative global -> register -> LDS staging of one 32-key chunk.
// Each thread owns K segments and V^T key pairs; `nthreads` threads in total.
template <int D, int NTHREADS>
struct ChunkStager {
  static constexpr int kKTasks = kChunk * (D / 8);          // 16-byte K segments per chunk
  static constexpr int kVTasks = (kChunk / 2) * (D / 8);    // (key pair, segment) tasks per chunk
  static constexpr int kKPer = (kKTasks + NTHREADS - 1) / NTHREADS;
  static constexpr int kVPer = (kVTasks + NTHREADS - 1) / NTHREADS;
  u32x4 kreg[kKPer];
  u32x4 vreg[kVPer][2];

  // key_row(kk) returns the element offset of key kk's row for K (second arg false)
  // or V (true), or -1 when that key lies outside the tensor (zero-filled).
  template <typename RowFn>
  __device__ __forceinline__ void load(const bf16* __restrict__ kbase, const bf16* __restrict__ vbase, int tid,
                                       RowFn key_row) {
#pragma unroll
    for (int i = 0; i < kKPer; ++i) {
      int task = tid + i * NTHREADS;
      kreg[i] = u32x4{0, 0, 0, 0};
      if (task < kKTasks) {
        int key = task / (D / 8), seg = task % (D / 8);
        int64_t off = key_row(key, false);
        if (off >= 0) kreg[i] = *(const u32x4*)(kbase + off + seg * 8);
      }
    }
#pragma unroll
    for (int i = 0; i < kVPer; ++i) {
      int task = tid + i * NTHREADS;
      vreg[i][0] = u32x4{0, 0, 0, 0};
      vreg[i][1] = u32x4{0, 0, 0, 0};
      if (task < kVTasks) {
        int p = task % (kChunk / 2), seg = task / (kChunk / 2);
        int64_t o0 = key_row(2 * p, true), o1 = key_row(2 * p + 1, true);
        if (o0 >= 0) vreg[i][0] = *(const u32x4*)(vbase + o0 + seg * 8);
        if (o1 >= 0) vreg[i][1] = *(const u32x4*)(vbase + o1 + seg * 8);
      }
    }
  }

  __device__ __forceinline__ void store(char* slot, int tid) const {
    using L = ChunkLayout<D>;
#pragma unroll
    for (int i = 0; i < kKPer; ++i) {
      int task = tid + i * NTHREADS;
      if (task < kKTasks) {
        int key = task / (D / 8), seg = task % (D / 8);
        *(u32x4*)(slot + L::k_off(key, seg)) = kreg[i];
      }
    }
#pragma unroll
    for (int i = 0; i < kVPer; ++i) {
      int task = tid + i * NTHREADS;
      if (task < kVTasks) {
        int p = task % (kChunk / 2), seg = task / (kChunk / 2);
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          uint32_t a = vreg[i][0][w], b = vreg[i][1][w];
          // element 2w (low half) and 2w+1 (high half) of each key
          uint32_t lo = (a & 0xffffu) | (b << 16);
          uint32_t hi = (a >> 16) | (b & 0xffff0000u);
          *(uint32_t*)(slot + L::vt_pair_off(seg * 8 + 2 * w, p)) = lo;
          *(uint32_t*)(slot + L::vt_pair_off(seg * 8 + 2 * w + 1, p)) = hi;
        }
      }
    }
  }
};

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

  // One 32-key chunk.  `slot` is the LDS chunk, sl2 = |scale|*log2(e) >= 0.
  // key_lo/key_hi: chunk-relative range [key_lo, key_hi] of valid keys for
  // this wave's query (masking only when the chunk is not fully valid).
  __device__ __forceinline__ void chunk(const char* slot, int lane, float sl2, int key_lo, int key_hi) {
    using L = ChunkLayout<D>;
    const int n = lane & 31, half = lane >> 5;
    floatx16 s = floatx16{};
#pragma unroll
    for (int t = 0; t < D / 16; ++t) {
      bf16x8 kf = *(const bf16x8*)(slot + L::k_off(n, 2 * t + half));
      s = mfma32x32x16(kf, a[t], s);
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
    rmax = fmaxf(rmax, swap_halves(rmax));
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
    float p[16];
    float zs = 0.f;
    if (masked) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int kr = 8 * (r >> 2) + (r & 3);
        const bool ok = kr >= lo_h && kr <= hi_h;
        p[r] = ok ? fast_exp2(fmaf(s[r], sl2, -m)) : 0.f;
        zs += p[r];
      }
    } else {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        p[r] = fast_exp2(fmaf(s[r], sl2, -m));
        zs += p[r];
      }
    }
    z += zs;
    bf16x8 pb[2];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int u = 0; u < 8; ++u) pb[t][u] = (bf16)p[8 * t + u];
#pragma unroll
    for (int db = 0; db < D / 32; ++db) {
      const int d = 32 * db + n;
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        u32x2 lo = *(const u32x2*)(slot + L::vt_unit_off(d, 4 * t + half));
        u32x2 hi = *(const u32x2*)(slot + L::vt_unit_off(d, 4 * t + 2 + half));
        u32x4 vv = u32x4{lo[0], lo[1], hi[0], hi[1]};
        o[db] = mfma32x32x16(__builtin_bit_cast(bf16x8, vv), pb[t], o[db]);
      }
    }
  }
};

}  // namespace sa
