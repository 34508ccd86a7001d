// Backward of the 2-simplicial prefill (dense or packed varlen): gradients of
// q, k1, k2, v1, v2 from dout, the forward output and its LSE.  Replaces the
// reference's SimplicialFunction.backward / Triton _backward
// (archlab/architectures/simplicial_kernels.py:55-106, :133-143) and, being
// free of atomics, also its deterministic variant
// (simplicial_deterministic.py:17-104).
//
// Per query i, head h (a_j = q ⊙ k1_j, score s_jk = scale a_j·k2_k):
//   P_jk   = exp(s_jk - lse_i)                 delta_i = dout_i · out_i
//   dP_jk  = (dout_i ⊙ v1_j) · v2_k             dS_jk  = P_jk (dP_jk - delta_i) scale
//   dq_i   = Σ_j (Σ_k dS_jk k2_k) ⊙ k1_j        dk1_j += (Σ_k dS_jk k2_k) ⊙ q_i
//   dk2_k += Σ_j dS_jk a_j                      dv1_j += (Σ_k P_jk v2_k) ⊙ dout_i
//   dv2_k += Σ_j P_jk (dout_i ⊙ v1_j)
// (a gradient of the LSE output, when given, enters as delta_i - dlse_i; for
// a single-pair query only that term remains: dS = P dlse scale)
// with the reference's rounding points: a, dout ⊙ v1 and dS rounded to the
// input dtype, P rounded to it on the value paths, fp32 accumulation; dS is
// zero for a query with a single valid pair (first token of a sequence, or
// both windows of one key).
//
// Three passes, each writing its outputs exactly once (no atomics, fixed
// summation order, so the result is bitwise reproducible):
//   bwd_dq_kernel    one workgroup per (query, head)      -> dq
//   bwd_dkv1_kernel  one workgroup per (short key, KV head) -> dk1, dv1
//   bwd_dkv2_kernel  one workgroup per (tile of long keys, KV head) -> dk2, dv2
// Each recomputes P from the saved LSE.  These are portable fp32-arithmetic
// kernels (any D in {16..512}, DV in {16..256}); they are not MFMA-tiled.
#include "sa_generic.h"
#include "sa_launch.h"
#include "sa_backward.h"

namespace sa {

constexpr int kBwdThreads = 256;
constexpr int kBwdJB = 16;  // rows per group
__host__ __device__ constexpr int bwd_kb(int d) { return d >= 512 ? 16 : (d >= 256 ? 32 : 64); }
// Long keys per dkv2 workgroup: per-thread accumulators KB*D/256 <= 32 and KB*DV/256 <= 16.
__host__ __device__ constexpr int bwd_kb2(int d, int dv) {
  const int a = 8192 / d, b = 4096 / dv;
  return (a < b ? a : b) < 64 ? (a < b ? a : b) : 64;
}

// [start, end) of the sequence that holds token t.
__device__ __forceinline__ void seq_bounds(const BwdParams& p, int t, int& start, int& end) {
  if (p.cu == nullptr) {
    start = (t / p.seqlen) * p.seqlen;
    end = start + p.seqlen;
    return;
  }
  int lo = 0, hi = p.num_seqs - 1;  // largest s with cu[s] <= t
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (p.cu[mid] <= t) lo = mid;
    else hi = mid - 1;
  }
  start = min(max(p.cu[lo], 0), t);
  end = max(min(p.cu[lo + 1], p.tokens), t + 1);
}

// dS is identically zero when query t has exactly one valid (j, k) pair.
__device__ __forceinline__ bool single_pair(const BwdParams& p, int t, int start) {
  return t == start || (p.ws == 1 && p.wl == 1);
}

// delta = dout · out - dlse per (token, head): 16 lanes per row, each lane
// 16 bytes of dout and out per step, reduced over the 16 lanes.
template <typename T>
__global__ __launch_bounds__(kBwdThreads) void bwd_delta_kernel(BwdParams p) {
  constexpr int E = 16 / sizeof(T);  // elements per 16-byte load
  const int64_t th = (int64_t)bid_x() * (kBwdThreads / 16) + tid_x() / 16;
  const int l = tid_x() & 15;
  const bool ok = th < (int64_t)p.tokens * p.hq;
  const int64_t tc = ok ? th : 0;
  const int t = (int)(tc / p.hq), h = (int)(tc % p.hq);
  const T* o = (const T*)p.out + (int64_t)t * p.o_st + (int64_t)h * p.o_sh;
  const T* g = (const T*)p.dout + (int64_t)t * p.do_st + (int64_t)h * p.do_sh;
  float s = 0.f;
  if (ok) {
    if (p.dv % E == 0 && ((uintptr_t)o % 16) == 0 && ((uintptr_t)g % 16) == 0) {
      for (int e = l * E; e < p.dv; e += 16 * E) {
        const uint4 ov = *(const uint4*)(o + e), gv = *(const uint4*)(g + e);
        const T* ot = (const T*)&ov;
        const T* gt = (const T*)&gv;
#pragma unroll
        for (int u = 0; u < E; ++u) s = fmaf(ld(gt + u), ld(ot + u), s);
      }
    } else {
      for (int e = l; e < p.dv; e += 16) s = fmaf(ld(g + e), ld(o + e), s);
    }
  }
  // sum over the 16 lanes of the row (xor shuffles stay inside the 16-lane group)
#pragma unroll
  for (int m = 8; m > 0; m >>= 1) s += __shfl_xor(s, m, 16);
  if (ok && l == 0) {
    // an LSE gradient adds dlse * P to dL/ds: folded in as delta - dlse
    const float gl = p.dlse ? p.dlse[(int64_t)t * p.dlse_st + h] : 0.f;
    p.delta[th] = s - gl;
    p.dl[th] = gl;
  }
}

// ---------------------------------------------------------------------------
// dq: one workgroup per (query t, head h).
template <typename T>
__global__ __launch_bounds__(kBwdThreads) void bwd_dq_kernel(BwdParams p) {
  extern __shared__ float smem[];
  const int t = bid_x(), h = bid_y();
  const int D = p.d, DV = p.dv, KB = bwd_kb(D), JB = kBwdJB;
  const int g = h / p.group;
  const int tid = tid_x();
  float* Qs = smem;                 // [D]
  float* Gs = Qs + D;               // [DV] dout
  float* As = Gs + DV;              // [JB][D+1]  a rows
  float* K1s = As + JB * (D + 1);   // [JB][D]    k1 rows
  float* Ws = K1s + JB * D;         // [JB][DV+1] dout ⊙ v1 rows
  float* Ks = Ws + JB * (DV + 1);   // [KB][D+1]  k2 rows
  float* V2s = Ks + KB * (D + 1);   // [KB][DV+1] v2 rows
  float* Ss = V2s + KB * (DV + 1);  // [JB][KB+1] dS

  int s0, s1;
  seq_bounds(p, t, s0, s1);
  const T* q = (const T*)p.q + (int64_t)t * p.q_st + (int64_t)h * p.q_sh;
  const T* gr = (const T*)p.dout + (int64_t)t * p.do_st + (int64_t)h * p.do_sh;
  for (int d = tid; d < D; d += kBwdThreads) Qs[d] = ld(q + d);
  for (int e = tid; e < DV; e += kBwdThreads) Gs[e] = ld(gr + e);
  const float lse = p.lse[(int64_t)t * p.lse_st + h];
  const float delta = p.delta[(int64_t)t * p.hq + h];
  const float dl = p.dl[(int64_t)t * p.hq + h];
  const bool zero_ds = single_pair(p, t, s0);
  const int lo1 = max(s0, t - p.ws + 1), lo2 = max(s0, t - p.wl + 1);
  const int64_t kg = (int64_t)g * p.k_sh, vg = (int64_t)g * p.v_sh;
  const T* k1 = (const T*)p.k1;
  const T* k2 = (const T*)p.k2;
  const T* v1 = (const T*)p.v1;
  const T* v2 = (const T*)p.v2;
  float dq[2] = {0.f, 0.f};  // d = tid, tid + 256
  __syncthreads();

  for (int j0 = lo1; j0 <= t; j0 += JB) {
    const int nj = min(JB, t - j0 + 1);
    for (int e = tid; e < nj * D; e += kBwdThreads) {
      const int jj = e / D, d = e % D;
      const float kv = ld(k1 + (int64_t)(j0 + jj) * p.k_st + kg + d);
      K1s[jj * D + d] = kv;
      As[jj * (D + 1) + d] = round_to<T>(Qs[d] * kv);
    }
    for (int e = tid; e < nj * DV; e += kBwdThreads) {
      const int jj = e / DV, d = e % DV;
      Ws[jj * (DV + 1) + d] = round_to<T>(Gs[d] * ld(v1 + (int64_t)(j0 + jj) * p.v_st + vg + d));
    }
    for (int k0 = lo2; k0 <= t; k0 += KB) {
      const int nk = min(KB, t - k0 + 1);
      __syncthreads();  // previous tile consumed; A / W rows written
      for (int e = tid; e < nk * D; e += kBwdThreads) {
        const int kk = e / D, d = e % D;
        Ks[kk * (D + 1) + d] = ld(k2 + (int64_t)(k0 + kk) * p.k_st + kg + d);
      }
      for (int e = tid; e < nk * DV; e += kBwdThreads) {
        const int kk = e / DV, d = e % DV;
        V2s[kk * (DV + 1) + d] = ld(v2 + (int64_t)(k0 + kk) * p.v_st + vg + d);
      }
      __syncthreads();
      for (int e = tid; e < nj * nk; e += kBwdThreads) {
        const int jj = e / nk, kk = e % nk;
        const float* a = As + jj * (D + 1);
        const float* b = Ks + kk * (D + 1);
        float s = 0.f;
        for (int d = 0; d < D; ++d) s = fmaf(a[d], b[d], s);
        const float* w = Ws + jj * (DV + 1);
        const float* v = V2s + kk * (DV + 1);
        float dp = 0.f;
        for (int d = 0; d < DV; ++d) dp = fmaf(w[d], v[d], dp);
        const float pr = __expf(s * p.scale - lse);
        Ss[jj * (KB + 1) + kk] = round_to<T>(pr * (zero_ds ? dl : dp - delta) * p.scale);
      }
      __syncthreads();
      for (int u = 0; u < 2; ++u) {
        const int d = tid + u * kBwdThreads;
        if (d < D) {
          float acc = 0.f;
          for (int jj = 0; jj < nj; ++jj) {
            float da = 0.f;
            const float* srow = Ss + jj * (KB + 1);
            for (int kk = 0; kk < nk; ++kk) da = fmaf(srow[kk], Ks[kk * (D + 1) + d], da);
            acc = fmaf(da, K1s[jj * D + d], acc);
          }
          dq[u] += acc;
        }
      }
    }
    __syncthreads();
  }
  T* out = (T*)p.dq + (int64_t)t * p.dq_st + (int64_t)h * p.dq_sh;
  for (int u = 0; u < 2; ++u) {
    const int d = tid + u * kBwdThreads;
    if (d < D) out[d] = (T)dq[u];
  }
}

// ---------------------------------------------------------------------------
// dk1, dv1: one workgroup per (short key j, KV head g).  Rows are the (query
// i, head h) pairs whose short window holds j: i in [j, j + ws - 1] of the same
// sequence, h in the group; each row walks its own long window.
template <typename T>
__global__ __launch_bounds__(kBwdThreads) void bwd_dkv1_kernel(BwdParams p) {
  extern __shared__ float smem[];
  const int j = bid_x(), g = bid_y();
  const int D = p.d, DV = p.dv, KB = bwd_kb(D), JB = kBwdJB;
  const int tid = tid_x();
  float* K1r = smem;                // [D]   k1_j
  float* V1r = K1r + D;             // [DV]  v1_j
  float* As = V1r + DV;             // [JB][D+1]  a rows
  float* Qr = As + JB * (D + 1);    // [JB][D]    q rows
  float* Ws = Qr + JB * D;          // [JB][DV+1] dout ⊙ v1 rows
  float* Gr = Ws + JB * (DV + 1);   // [JB][DV]   dout rows
  float* Ks = Gr + JB * DV;         // [KB][D+1]
  float* V2s = Ks + KB * (D + 1);   // [KB][DV+1]
  float* Ss = V2s + KB * (DV + 1);  // [JB][KB+1] dS
  float* Ps = Ss + JB * (KB + 1);   // [JB][KB+1] P rounded
  float* RowF = Ps + JB * (KB + 1); // [JB][5]: lse, delta, dlse, (int) first long key, (int) single pair

  int s0, s1;
  seq_bounds(p, j, s0, s1);
  const int64_t kg = (int64_t)g * p.k_sh, vg = (int64_t)g * p.v_sh;
  const T* k2 = (const T*)p.k2;
  const T* v2 = (const T*)p.v2;
  for (int d = tid; d < D; d += kBwdThreads) K1r[d] = ld((const T*)p.k1 + (int64_t)j * p.k_st + kg + d);
  for (int e = tid; e < DV; e += kBwdThreads) V1r[e] = ld((const T*)p.v1 + (int64_t)j * p.v_st + vg + e);
  const int i_end = min(s1, j + p.ws);  // queries j .. i_end-1
  const int nrows = (i_end - j) * p.group;
  // per-thread accumulators over (row, d) / (row, e) of the current group,
  // folded into dk1 / dv1 after each group
  float dk1[2] = {0.f, 0.f}, dv1 = 0.f;
  __syncthreads();

  for (int r0 = 0; r0 < nrows; r0 += JB) {
    const int nr = min(JB, nrows - r0);
    // load the group's rows
    for (int e = tid; e < nr * D; e += kBwdThreads) {
      const int rr = e / D, d = e % D;
      const int i = j + (r0 + rr) / p.group, h = g * p.group + (r0 + rr) % p.group;
      const float qv = ld((const T*)p.q + (int64_t)i * p.q_st + (int64_t)h * p.q_sh + d);
      Qr[rr * D + d] = qv;
      As[rr * (D + 1) + d] = round_to<T>(qv * K1r[d]);
    }
    for (int e = tid; e < nr * DV; e += kBwdThreads) {
      const int rr = e / DV, d = e % DV;
      const int i = j + (r0 + rr) / p.group, h = g * p.group + (r0 + rr) % p.group;
      const float gv = ld((const T*)p.dout + (int64_t)i * p.do_st + (int64_t)h * p.do_sh + d);
      Gr[rr * DV + d] = gv;
      Ws[rr * (DV + 1) + d] = round_to<T>(gv * V1r[d]);
    }
    if (tid < nr) {
      const int i = j + (r0 + tid) / p.group, h = g * p.group + (r0 + tid) % p.group;
      RowF[tid * 5 + 0] = p.lse[(int64_t)i * p.lse_st + h];
      RowF[tid * 5 + 1] = p.delta[(int64_t)i * p.hq + h];
      RowF[tid * 5 + 2] = p.dl[(int64_t)i * p.hq + h];
      ((int*)RowF)[tid * 5 + 3] = max(s0, i - p.wl + 1);
      ((int*)RowF)[tid * 5 + 4] = single_pair(p, i, s0);
    }
    // long keys of the union of the group's windows
    const int i_lo = j + r0 / p.group, i_hi = j + (r0 + nr - 1) / p.group;
    const int klo = max(s0, i_lo - p.wl + 1);
    // per-thread partial sums da[row][d], pv[row][e] for this group
    float da[kBwdJB * 512 / kBwdThreads];
    float pv[kBwdJB * 256 / kBwdThreads];
    const int nda = (nr * D + kBwdThreads - 1) / kBwdThreads, npv = (nr * DV + kBwdThreads - 1) / kBwdThreads;
#pragma unroll
    for (int u = 0; u < kBwdJB * 512 / kBwdThreads; ++u) da[u] = 0.f;
#pragma unroll
    for (int u = 0; u < kBwdJB * 256 / kBwdThreads; ++u) pv[u] = 0.f;
    for (int k0 = klo; k0 <= i_hi; k0 += KB) {
      const int nk = min(KB, i_hi - k0 + 1);
      __syncthreads();
      for (int e = tid; e < nk * D; e += kBwdThreads) {
        const int kk = e / D, d = e % D;
        Ks[kk * (D + 1) + d] = ld(k2 + (int64_t)(k0 + kk) * p.k_st + kg + d);
      }
      for (int e = tid; e < nk * DV; e += kBwdThreads) {
        const int kk = e / DV, d = e % DV;
        V2s[kk * (DV + 1) + d] = ld(v2 + (int64_t)(k0 + kk) * p.v_st + vg + d);
      }
      __syncthreads();
      for (int e = tid; e < nr * nk; e += kBwdThreads) {
        const int rr = e / nk, kk = e % nk;
        const int i = j + (r0 + rr) / p.group;
        const int key = k0 + kk;
        float ds = 0.f, pr = 0.f;
        if (key <= i && key >= ((const int*)RowF)[rr * 5 + 3]) {
          const float* a = As + rr * (D + 1);
          const float* b = Ks + kk * (D + 1);
          float s = 0.f;
          for (int d = 0; d < D; ++d) s = fmaf(a[d], b[d], s);
          const float* w = Ws + rr * (DV + 1);
          const float* v = V2s + kk * (DV + 1);
          float dp = 0.f;
          for (int d = 0; d < DV; ++d) dp = fmaf(w[d], v[d], dp);
          const float pe = __expf(s * p.scale - RowF[rr * 5 + 0]);
          const float dd = ((const int*)RowF)[rr * 5 + 4] ? RowF[rr * 5 + 2] : dp - RowF[rr * 5 + 1];
          ds = round_to<T>(pe * dd * p.scale);
          pr = round_to<T>(pe);
        }
        Ss[rr * (KB + 1) + kk] = ds;
        Ps[rr * (KB + 1) + kk] = pr;
      }
      __syncthreads();
#pragma unroll
      for (int u = 0; u < kBwdJB * 512 / kBwdThreads; ++u) {
        const int e = tid + u * kBwdThreads;
        if (u < nda && e < nr * D) {
          const int rr = e / D, d = e % D;
          const float* srow = Ss + rr * (KB + 1);
          float acc = da[u];
          for (int kk = 0; kk < nk; ++kk) acc = fmaf(srow[kk], Ks[kk * (D + 1) + d], acc);
          da[u] = acc;
        }
      }
#pragma unroll
      for (int u = 0; u < kBwdJB * 256 / kBwdThreads; ++u) {
        const int e = tid + u * kBwdThreads;
        if (u < npv && e < nr * DV) {
          const int rr = e / DV, d = e % DV;
          const float* prow = Ps + rr * (KB + 1);
          float acc = pv[u];
          for (int kk = 0; kk < nk; ++kk) acc = fmaf(prow[kk], V2s[kk * (DV + 1) + d], acc);
          pv[u] = acc;
        }
      }
    }
    __syncthreads();
    // fold: dk1[d] += Σ_rows da[row][d] q_row[d]; dv1[e] += Σ_rows pv[row][e] dout_row[e]
    // (per-thread partials go through LDS so each output has one owner and a fixed order)
    float* red = Ks;  // reuse of the K2 and V2 tiles (>= JB * max(D, DV) floats): [JB][D] then [JB][DV]
#pragma unroll
    for (int u = 0; u < kBwdJB * 512 / kBwdThreads; ++u) {
      const int e = tid + u * kBwdThreads;
      if (u < nda && e < nr * D) red[e] = da[u] * Qr[e];
    }
    __syncthreads();
    for (int u = 0; u < 2; ++u) {
      const int d = tid + u * kBwdThreads;
      if (d < D) {
        float acc = dk1[u];
        for (int rr = 0; rr < nr; ++rr) acc += red[rr * D + d];
        dk1[u] = acc;
      }
    }
    __syncthreads();
#pragma unroll
    for (int u = 0; u < kBwdJB * 256 / kBwdThreads; ++u) {
      const int e = tid + u * kBwdThreads;
      if (u < npv && e < nr * DV) red[e] = pv[u] * Gr[e];
    }
    __syncthreads();
    if (tid < DV) {
      float acc = dv1;
      for (int rr = 0; rr < nr; ++rr) acc += red[rr * DV + tid];
      dv1 = acc;
    }
    __syncthreads();
  }
  T* o1 = (T*)p.dk1 + (int64_t)j * p.dk_st + (int64_t)g * p.dk_sh;
  for (int u = 0; u < 2; ++u) {
    const int d = tid + u * kBwdThreads;
    if (d < D) o1[d] = (T)dk1[u];
  }
  if (tid < DV) ((T*)p.dv1 + (int64_t)j * p.dv_st + (int64_t)g * p.dv_sh)[tid] = (T)dv1;
}

// ---------------------------------------------------------------------------
// dk2, dv2: one workgroup per (tile of KB long keys, KV head g).  Rows are the
// (query i, head h, short key j) triples whose windows reach a key of the
// tile: for each sequence the tile touches, i runs over that sequence's
// queries from the tile's first key to the last key + wl - 1, h over the
// group, j over i's short window.  Keys outside a query's window (including
// keys of another sequence) are masked.
template <typename T>
__global__ __launch_bounds__(kBwdThreads) void bwd_dkv2_kernel(BwdParams p) {
  extern __shared__ float smem[];
  const int D = p.d, DV = p.dv, KB = bwd_kb2(D, DV), JB = kBwdJB;
  const int k0 = bid_x() * KB, g = bid_y();
  const int tid = tid_x();
  float* Ks = smem;                 // [KB][D+1]
  float* V2s = Ks + KB * (D + 1);   // [KB][DV+1]
  float* As = V2s + KB * (DV + 1);  // [JB][D+1]  a rows
  float* Ws = As + JB * (D + 1);    // [JB][DV+1] dout ⊙ v1 rows
  float* Ss = Ws + JB * (DV + 1);   // [JB][KB+1] dS
  float* Ps = Ss + JB * (KB + 1);   // [JB][KB+1] P rounded
  float* RowF = Ps + JB * (KB + 1); // [JB][4]: lse, delta, dlse, (int) single pair

  if (k0 >= p.tokens) return;
  const int kend = min(k0 + KB, p.tokens);
  const int64_t kg = (int64_t)g * p.k_sh, vg = (int64_t)g * p.v_sh;
  for (int e = tid; e < KB * D; e += kBwdThreads) {
    const int kk = e / D, d = e % D;
    Ks[kk * (D + 1) + d] = k0 + kk < kend ? ld((const T*)p.k2 + (int64_t)(k0 + kk) * p.k_st + kg + d) : 0.f;
  }
  for (int e = tid; e < KB * DV; e += kBwdThreads) {
    const int kk = e / DV, d = e % DV;
    V2s[kk * (DV + 1) + d] = k0 + kk < kend ? ld((const T*)p.v2 + (int64_t)(k0 + kk) * p.v_st + vg + d) : 0.f;
  }
  // accumulators over (key, d) and (key, e): KB*D <= 8192 and KB*DV <= 4096 values
  constexpr int kMaxKD = 8192 / kBwdThreads, kMaxKV = 4096 / kBwdThreads;
  float dk2[kMaxKD], dv2[kMaxKV];
#pragma unroll
  for (int u = 0; u < kMaxKD; ++u) dk2[u] = 0.f;
#pragma unroll
  for (int u = 0; u < kMaxKV; ++u) dv2[u] = 0.f;
  const int nkd = (KB * D) / kBwdThreads, nkv = (KB * DV + kBwdThreads - 1) / kBwdThreads;

  for (int cur = k0; cur < kend;) {
    int s0, s1;
    seq_bounds(p, cur, s0, s1);
    const int seg_end = min(kend, s1);               // keys [cur, seg_end) of this sequence
    const int i_end = min(s1, seg_end - 1 + p.wl);   // queries cur .. i_end-1
    for (int i = cur; i < i_end; ++i) {
      const int lo1 = max(s0, i - p.ws + 1);
      const int lo2 = max(s0, i - p.wl + 1);
      const int nj_all = i - lo1 + 1;
      const int rows = nj_all * p.group;  // (h, j) pairs of query i
      for (int r0 = 0; r0 < rows; r0 += JB) {
        const int nr = min(JB, rows - r0);
        __syncthreads();  // K/V tile loaded; previous group consumed
        for (int e = tid; e < nr * D; e += kBwdThreads) {
          const int rr = e / D, d = e % D;
          const int h = g * p.group + (r0 + rr) / nj_all, jj = lo1 + (r0 + rr) % nj_all;
          const float qv = ld((const T*)p.q + (int64_t)i * p.q_st + (int64_t)h * p.q_sh + d);
          As[rr * (D + 1) + d] = round_to<T>(qv * ld((const T*)p.k1 + (int64_t)jj * p.k_st + kg + d));
        }
        for (int e = tid; e < nr * DV; e += kBwdThreads) {
          const int rr = e / DV, d = e % DV;
          const int h = g * p.group + (r0 + rr) / nj_all, jj = lo1 + (r0 + rr) % nj_all;
          const float gv = ld((const T*)p.dout + (int64_t)i * p.do_st + (int64_t)h * p.do_sh + d);
          Ws[rr * (DV + 1) + d] = round_to<T>(gv * ld((const T*)p.v1 + (int64_t)jj * p.v_st + vg + d));
        }
        if (tid < nr) {
          const int h = g * p.group + (r0 + tid) / nj_all;
          RowF[tid * 4 + 0] = p.lse[(int64_t)i * p.lse_st + h];
          RowF[tid * 4 + 1] = p.delta[(int64_t)i * p.hq + h];
          RowF[tid * 4 + 2] = p.dl[(int64_t)i * p.hq + h];
          ((int*)RowF)[tid * 4 + 3] = single_pair(p, i, s0);
        }
        __syncthreads();
        for (int e = tid; e < nr * KB; e += kBwdThreads) {
          const int rr = e / KB, kk = e % KB;
          const int key = k0 + kk;
          float ds = 0.f, pr = 0.f;
          if (key >= cur && key < seg_end && key <= i && key >= lo2) {
            const float* a = As + rr * (D + 1);
            const float* b = Ks + kk * (D + 1);
            float s = 0.f;
            for (int d = 0; d < D; ++d) s = fmaf(a[d], b[d], s);
            const float* w = Ws + rr * (DV + 1);
            const float* v = V2s + kk * (DV + 1);
            float dp = 0.f;
            for (int d = 0; d < DV; ++d) dp = fmaf(w[d], v[d], dp);
            const float pe = __expf(s * p.scale - RowF[rr * 4 + 0]);
            const float dd = ((const int*)RowF)[rr * 4 + 3] ? RowF[rr * 4 + 2] : dp - RowF[rr * 4 + 1];
            ds = round_to<T>(pe * dd * p.scale);
            pr = round_to<T>(pe);
          }
          Ss[rr * (KB + 1) + kk] = ds;
          Ps[rr * (KB + 1) + kk] = pr;
        }
        __syncthreads();
#pragma unroll
        for (int u = 0; u < kMaxKD; ++u) {
          if (u < nkd) {
            const int e = tid + u * kBwdThreads;
            const int kk = e / D, d = e % D;
            float acc = dk2[u];
            for (int rr = 0; rr < nr; ++rr) acc = fmaf(Ss[rr * (KB + 1) + kk], As[rr * (D + 1) + d], acc);
            dk2[u] = acc;
          }
        }
#pragma unroll
        for (int u = 0; u < kMaxKV; ++u) {
          const int e = tid + u * kBwdThreads;
          if (u < nkv && e < KB * DV) {
            const int kk = e / DV, d = e % DV;
            float acc = dv2[u];
            for (int rr = 0; rr < nr; ++rr) acc = fmaf(Ps[rr * (KB + 1) + kk], Ws[rr * (DV + 1) + d], acc);
            dv2[u] = acc;
          }
        }
      }
    }
    cur = seg_end;
  }
#pragma unroll
  for (int u = 0; u < kMaxKD; ++u) {
    if (u < nkd) {
      const int e = tid + u * kBwdThreads;
      const int kk = e / D, d = e % D;
      if (k0 + kk < kend) ((T*)p.dk2 + (int64_t)(k0 + kk) * p.dk_st + (int64_t)g * p.dk_sh)[d] = (T)dk2[u];
    }
  }
#pragma unroll
  for (int u = 0; u < kMaxKV; ++u) {
    const int e = tid + u * kBwdThreads;
    if (u < nkv && e < KB * DV) {
      const int kk = e / DV, d = e % DV;
      if (k0 + kk < kend) ((T*)p.dv2 + (int64_t)(k0 + kk) * p.dv_st + (int64_t)g * p.dv_sh)[d] = (T)dv2[u];
    }
  }
}

// ---------------------------------------------------------------------------
// Host side

static size_t dq_lds(int d, int dv) {
  const int kb = bwd_kb(d), jb = kBwdJB;
  return sizeof(float) * ((size_t)d + dv + jb * (d + 1) + jb * d + jb * (dv + 1) + kb * (d + 1) + kb * (dv + 1) +
                          jb * (kb + 1));
}
static size_t dkv1_lds(int d, int dv) {
  const int kb = bwd_kb(d), jb = kBwdJB;
  size_t f = (size_t)d + dv + jb * (d + 1) + jb * d + jb * (dv + 1) + jb * dv + kb * (d + 1) + kb * (dv + 1) +
             2 * jb * (kb + 1) + jb * 5;
  return sizeof(float) * f;
}
static size_t dkv2_lds(int d, int dv) {
  const int kb = bwd_kb2(d, dv), jb = kBwdJB;
  return sizeof(float) *
         ((size_t)kb * (d + 1) + kb * (dv + 1) + jb * (d + 1) + jb * (dv + 1) + 2 * jb * (kb + 1) + jb * 4);
}

static size_t bwd_row_bytes(const sa_prefill_bwd_args* a) {
  return ((size_t)a->fwd.total_tokens * a->fwd.heads_q * sizeof(float) + 255) & ~(size_t)255;
}
// fp32 inputs on the matrix cores: equal widths of 64 or 128 and one 32-row
// group of short keys (the dq pass; the other passes fall back to the
// portable kernels where their fp32 forms do not apply), 16-byte rows.
static bool f32_mfma_shape(const sa_prefill_args& f) {
  if (f.dtype != SA_DTYPE_F32 || (f.flags & SA_FLAG_FORCE_GENERIC)) return false;
  if (f.head_dim != f.value_dim || (f.head_dim != 64 && f.head_dim != 128) || f.short_window > 32) return false;
  const int64_t st[] = {f.q_stride_t, f.q_stride_h, f.k_stride_t, f.k_stride_h, f.v_stride_t, f.v_stride_h};
  for (int64_t x : st)
    if (x % 4) return false;
  return true;
}
// hi/lo rows of k2 and v2 for fp32 inputs on the matrix cores: [tokens][hk][2 D] bf16 each
static size_t f32_split_bytes(const sa_prefill_bwd_args* a) {
  const sa_prefill_args& f = a->fwd;
  if (!f32_mfma_shape(f)) return 0;
  return ((size_t)f.total_tokens * f.heads_kv * f.head_dim * 4 + 255) / 256 * 256;
}
// Shapes whose dk1 may come from the dq pass (bwd_dk1_fused_ok adds the
// stride and alignment conditions): the partials' workspace is reserved for
// every such call.
static bool dk1_fused_shape(const sa_prefill_bwd_args* a) {
  const sa_prefill_args& f = a->fwd;
  const bool narrow = (f.head_dim == 64 || f.head_dim == 128) && (f.value_dim == 64 || f.value_dim == 128);
  const bool wide = f.head_dim == 256 && (f.value_dim == 128 || f.value_dim == 256);
  if (f.flags & SA_FLAG_SEPARATE_DK1) return false;
  if (f.dtype == SA_DTYPE_F32) return f32_mfma_shape(f) && f.heads_kv > 0;
  return f.dtype == SA_DTYPE_BF16 && !(f.flags & SA_FLAG_FORCE_GENERIC) && (narrow || wide) &&
         f.short_window <= 64 && f.heads_kv > 0;
}
// The partials take 16-17.5x the bytes of q per row group; past kDk1PartialCap (or with
// SA_FLAG_SEPARATE_DK1, for callers short of memory) the separate dk1 pass
// runs instead (no workspace beyond the delta / dlse rows).
constexpr size_t kDk1PartialCap = (size_t)8 << 30;
static size_t dk1_partial_bytes(const sa_prefill_bwd_args* a) {
  if (!dk1_fused_shape(a)) return 0;
  const sa_prefill_args& f = a->fwd;
  const int nq = dq_queries_per_block(f.heads_q / f.heads_kv);
  const size_t qblocks = ((size_t)f.total_tokens + nq - 1) / nq;
  const size_t heads = (size_t)f.heads_q / (4 / nq);  // hk * head sub-groups
  const size_t nr = ((size_t)f.short_window + 31) / 32;  // row groups of short keys
  const size_t bytes = (qblocks * heads * nr * (31 + nq) * f.head_dim * sizeof(float) + 255) & ~(size_t)255;
  return bytes <= kDk1PartialCap ? bytes : 0;
}
// fp32 inputs with dk1 from the dq pass: dv1 from it as well, the same rows
// at the value width; both together within kDk1PartialCap (else the dk1 / dv1
// pass computes dv1)
static size_t dv1_partial_bytes(const sa_prefill_bwd_args* a) {
  const sa_prefill_args& f = a->fwd;
  const size_t k = dk1_partial_bytes(a);
  if (f.dtype != SA_DTYPE_F32 || !k) return 0;
  const int nq = dq_queries_per_block(f.heads_q / f.heads_kv);
  const size_t qblocks = ((size_t)f.total_tokens + nq - 1) / nq;
  const size_t heads = (size_t)f.heads_q / (4 / nq);
  const size_t nr = ((size_t)f.short_window + 31) / 32;
  const size_t v = (qblocks * heads * nr * (31 + nq) * f.value_dim * sizeof(float) + 255) & ~(size_t)255;
  return k + v <= kDk1PartialCap ? v : 0;
}
// Short windows past what one MFMA dk2 / dv2 launch holds (64 keys at widths
// <= 128, 32 at score width 256) and up to twice that: the first launch's fp32
// dk2 and dv2 sums.
static size_t dkv2_partial_bytes(const sa_prefill_bwd_args* a) {
  const sa_prefill_args& f = a->fwd;
  const bool narrow = (f.head_dim == 64 || f.head_dim == 128) && (f.value_dim == 64 || f.value_dim == 128);
  const bool wide = f.head_dim == 256 && (f.value_dim == 128 || f.value_dim == 256);
  const int one = wide ? 32 : 64;
  if (f.dtype != SA_DTYPE_BF16 || (f.flags & SA_FLAG_FORCE_GENERIC) || !(narrow || wide) ||
      f.short_window <= one || f.short_window > 2 * one)
    return 0;
  return ((size_t)f.total_tokens * f.heads_kv * (f.head_dim + f.value_dim) * sizeof(float) + 255) & ~(size_t)255;
}
// bf16 dk2 / dv2 on the matrix cores in one launch (widths 64 / 128, short
// window <= 64) whose plan cuts the walks into pieces: the pieces' fp32 sums,
// [splits][tokens][hk][max(D, DV)] (dk2's, then, reused, dv2's)
static size_t dkv2_split_bytes(const sa_prefill_bwd_args* a) {
  const sa_prefill_args& f = a->fwd;
  const bool narrow = (f.head_dim == 64 || f.head_dim == 128) && (f.value_dim == 64 || f.value_dim == 128);
  if (f.dtype != SA_DTYPE_BF16 || (f.flags & SA_FLAG_FORCE_GENERIC) || !narrow || f.short_window > 64 ||
      f.heads_kv <= 0)
    return 0;
  const Dkv2Plan pl = bwd_dkv2_plan(f.total_tokens, f.heads_kv, f.head_dim, f.value_dim, f.short_window,
                                    f.long_window, false, device_cu_count());
  if (pl.splits <= 1) return 0;
  const size_t w = (size_t)(f.head_dim > f.value_dim ? f.head_dim : f.value_dim);
  return ((size_t)pl.splits * f.total_tokens * f.heads_kv * w * sizeof(float) + 255) & ~(size_t)255;
}
size_t prefill_bwd_workspace_bytes(const sa_prefill_bwd_args* a) {
  return 2 * bwd_row_bytes(a) + dk1_partial_bytes(a) + dkv2_partial_bytes(a) + 2 * f32_split_bytes(a) +
         dkv2_split_bytes(a) + dv1_partial_bytes(a);
}

template <typename T>
static hipError_t launch_bwd_t(const BwdParams& p, hipStream_t stream) {
  const int64_t nth = (int64_t)p.tokens * p.hq;
  constexpr int kRowsPerBlock = kBwdThreads / 16;
  hipLaunchKernelGGL(bwd_delta_kernel<T>, dim3((unsigned)((nth + kRowsPerBlock - 1) / kRowsPerBlock)),
                     dim3(kBwdThreads), 0, stream, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  struct K {
    const void* f;
    size_t lds;
    dim3 grid;
  } ks[3] = {
      {(const void*)bwd_dq_kernel<T>, dq_lds(p.d, p.dv), dim3(p.tokens, p.hq)},
      {(const void*)bwd_dkv1_kernel<T>, dkv1_lds(p.d, p.dv), dim3(p.tokens, p.hk)},
      {(const void*)bwd_dkv2_kernel<T>, dkv2_lds(p.d, p.dv),
       dim3((p.tokens + bwd_kb2(p.d, p.dv) - 1) / bwd_kb2(p.d, p.dv), p.hk)},
  };
  for (const K& k : ks) {
    e = set_lds_limit(k.f, k.lds);
    if (e != hipSuccess) return e;
  }
  // each pass runs on MFMA tiles where its kernel covers the call, else on the portable kernel
  e = launch_bwd_dq_mfma(p, stream);
  if (e == hipErrorNotSupported) {
    hipLaunchKernelGGL(bwd_dq_kernel<T>, ks[0].grid, dim3(kBwdThreads), ks[0].lds, stream, p);
    e = hipGetLastError();
  }
  if (e != hipSuccess) return e;
  if (p.dk1p) {  // dk1 from the dq pass's partials; the dkv1 launch below computes dv1 only
    e = launch_bwd_dk1_sum(p, stream);
    if (e != hipSuccess) return e;
  }
  if (p.dv1p) {  // dv1 from the dq pass's partials as well: no dk1 / dv1 pass
    e = launch_bwd_dv1_sum(p, stream);
  } else {
    e = launch_bwd_dkv1_mfma(p, stream);
    if (e == hipErrorNotSupported) {
      hipLaunchKernelGGL(bwd_dkv1_kernel<T>, ks[1].grid, dim3(kBwdThreads), ks[1].lds, stream, p);
      e = hipGetLastError();
    }
  }
  if (e != hipSuccess) return e;
  e = launch_bwd_dkv2_mfma(p, stream);
  if (e == hipErrorNotSupported) {
    hipLaunchKernelGGL(bwd_dkv2_kernel<T>, ks[2].grid, dim3(kBwdThreads), ks[2].lds, stream, p);
    e = hipGetLastError();
  }
  return e;
}

hipError_t launch_prefill_bwd(const sa_prefill_bwd_args* a, void* ws, hipStream_t stream) {
  const sa_prefill_args& f = a->fwd;
  if (f.total_tokens == 0) return hipSuccess;
  BwdParams p{};
  p.q = f.q;
  p.k1 = f.k1;
  p.k2 = f.k2;
  p.v1 = f.v1;
  p.v2 = f.v2;
  p.out = f.out;
  p.lse = f.lse;
  p.dout = a->dout;
  p.dq = a->dq;
  p.dk1 = a->dk1;
  p.dk2 = a->dk2;
  p.dv1 = a->dv1;
  p.dv2 = a->dv2;
  p.delta = (float*)ws;
  p.dl = (float*)((char*)ws + bwd_row_bytes(a));
  p.dlse = a->dlse;
  p.dlse_st = a->dlse_stride_t;
  p.cu = f.cu_seqlens;
  p.q_st = f.q_stride_t;
  p.q_sh = f.q_stride_h;
  p.k_st = f.k_stride_t;
  p.k_sh = f.k_stride_h;
  p.v_st = f.v_stride_t;
  p.v_sh = f.v_stride_h;
  p.o_st = f.o_stride_t;
  p.o_sh = f.o_stride_h;
  p.lse_st = f.lse_stride_t;
  p.do_st = a->do_stride_t;
  p.do_sh = a->do_stride_h;
  p.dq_st = a->dq_stride_t;
  p.dq_sh = a->dq_stride_h;
  p.dk_st = a->dk_stride_t;
  p.dk_sh = a->dk_stride_h;
  p.dv_st = a->dv_stride_t;
  p.dv_sh = a->dv_stride_h;
  p.tokens = f.total_tokens;
  p.seqlen = f.seqlen;
  p.num_seqs = f.num_seqs;
  p.hq = f.heads_q;
  p.hk = f.heads_kv;
  p.group = f.heads_q / f.heads_kv;
  p.ws = f.short_window;
  p.wl = f.long_window;
  p.d = f.head_dim;
  p.dv = f.value_dim;
  p.scale = f.scale;
  p.f32 = f.dtype == SA_DTYPE_F32;
  p.mfma = (f.dtype == SA_DTYPE_BF16 && !(f.flags & SA_FLAG_FORCE_GENERIC)) || f32_mfma_shape(f);
  if (size_t sb = f32_split_bytes(a)) {
    // k2 and v2 as hi/lo bf16 rows for the fp32 matrix-core passes
    char* base = (char*)ws + 2 * bwd_row_bytes(a) + dk1_partial_bytes(a) + dkv2_partial_bytes(a);
    bf16* k2s = (bf16*)base;
    bf16* v2s = (bf16*)(base + sb);
    hipError_t e = launch_split_hilo((const float*)f.k2, f.k_stride_t, f.k_stride_h, f.total_tokens, f.heads_kv,
                                     f.head_dim, k2s, stream);
    if (e == hipSuccess)
      e = launch_split_hilo((const float*)f.v2, f.v_stride_t, f.v_stride_h, f.total_tokens, f.heads_kv,
                            f.value_dim, v2s, stream);
    if (e != hipSuccess) return e;
    p.k2s = k2s;
    p.v2s = v2s;
  }
  if (dk1_partial_bytes(a) && bwd_dk1_fused_ok(p)) p.dk1p = (float*)((char*)ws + 2 * bwd_row_bytes(a));
  if (dv1_partial_bytes(a) && p.dk1p)
    p.dv1p = (float*)((char*)ws + 2 * bwd_row_bytes(a) + dk1_partial_bytes(a) + dkv2_partial_bytes(a) +
                      2 * f32_split_bytes(a) + dkv2_split_bytes(a));
  if (dkv2_partial_bytes(a)) p.dkv2p = (float*)((char*)ws + 2 * bwd_row_bytes(a) + dk1_partial_bytes(a));
  if (dkv2_split_bytes(a))
    p.dkv2s = (float*)((char*)ws + 2 * bwd_row_bytes(a) + dk1_partial_bytes(a) + dkv2_partial_bytes(a) +
                       2 * f32_split_bytes(a));
  if (f.dtype == SA_DTYPE_F32) return launch_bwd_t<float>(p, stream);
  return launch_bwd_t<bf16>(p, stream);
}

}  // namespace sa
