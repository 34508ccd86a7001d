// Prefill forward (dense [B,S,H,D] or packed variable-length) for the
// 2-simplicial attention library.  Replaces the reference's Triton _forward
// (archlab/architectures/simplicial_kernels.py:16-52) behind
// simplicial_attention (simplicial_attention.py:77-97).
//
// bf16 MFMA kernel (D in {64, 128, 256}, DV == D)
// ------------------------------------------------
// A workgroup of 4 waves owns NQ query tokens spaced 32 apart
// (t_w = base + 32*w), NH query heads of one KV group and NRG short-axis row
// groups, NQ*NH*NRG == 4.  Each wave handles one (token, head, row group):
// 32 A rows a_j = bf16(q_t ⊙ k1_j).  All queries of the block walk the long
// window in 32-key chunks that start at t - long_window + 1, so a query's
// window is covered by exactly ceil(long_window / 32) chunks and tokens spaced
// 32 apart share the same chunk grid: wave w uses block chunk (c + qw) in
// iteration c.  Chunks stream through an LDS ring of NQ + 1 slots, one chunk
// prefetched per iteration, one barrier per iteration.
//
// The joint softmax is kept per A row (running max / sum); the epilogue merges
// the rows with their log-sum-exp weights and applies v1:
//     out = sum_j w_j (v1_j ⊙ O_j) / sum_j w_j z_j,   w_j = exp(m_j - max m).
#include "sa_generic.h"
#include "sa_mfma.h"
#include "sa_launch.h"

namespace sa {

struct PrefillParams {
  const bf16* q;
  const bf16* k1;
  const bf16* k2;
  const bf16* v1;
  const bf16* v2;
  bf16* out;
  float* lse;
  const int32_t* cu;
  int64_t q_st, q_sh, k_st, k_sh, v_st, v_sh, o_st, o_sh, lse_st;
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
};

// Start of token t's sequence, clamped to [0, t] so that a malformed
// cu_seqlens cannot move any row access outside the tensors.
__device__ __forceinline__ int seq_start(const int32_t* cu, int num_seqs, int seqlen, int t) {
  if (cu == nullptr) return (t / seqlen) * seqlen;
  int lo = 0, hi = num_seqs - 1;  // largest s with cu[s] <= t
  while (lo < hi) {
    int mid = (lo + hi + 1) >> 1;
    if (cu[mid] <= t) lo = mid;
    else hi = mid - 1;
  }
  return min(max(cu[lo], 0), t);
}

__device__ __forceinline__ int seq_start_of(const PrefillParams& p, int t) { return seq_start(p.cu, p.num_seqs, p.seqlen, t); }

// Workgroups are dispatched round-robin over the 8 XCDs; remap so that each
// XCD (own L2) walks a contiguous range of logical blocks (neighbouring
// queries of the same heads share their key windows).
__device__ __forceinline__ int xcd_remap(int b, int n) {
  const int q = n / 8, r = n % 8;
  const int x = b % 8, i = b / 8;
  return x * q + min(x, r) + i;
}

template <int D, int NQ, int NH, int NRG>
__global__ __launch_bounds__(256, 1) void prefill_mfma_kernel(PrefillParams p) {
  static_assert(NQ * NH * NRG == 4, "4 waves per block");
  using L = ChunkLayout<D>;
  constexpr int R = NQ + 1;  // ring slots
  extern __shared__ __attribute__((aligned(16))) char lds[];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wid = tid >> 6;
  const int rg = wid % NRG;
  const int hw = (wid / NRG) % NH;
  const int qw = wid / (NRG * NH);

  const int lb = xcd_remap(blockIdx.x, p.nblocks);
  const int qb = lb % p.qblocks;
  const int hg = lb / p.qblocks;  // = g * hsub + hs
  const int g = hg / p.hsub, hs = hg % p.hsub;
  const int base = (qb / 32) * (32 * NQ) + (qb % 32);
  if (base >= p.total) return;

  const int t = base + 32 * qw;
  const bool qvalid = t < p.total;
  const int h = g * p.group + hs * NH + hw;
  const int s0 = qvalid ? seq_start_of(p, t) : 0;
  const int lo2 = max(s0, t - p.wl + 1);
  const int lo1 = max(s0, t - p.ws + 1);
  // first chunk with a valid key, for this wave and for the block
  const int cfirst = qvalid ? (lo2 - (t - p.wl + 1)) / kChunk : p.nc;
  int c0 = p.nc;
#pragma unroll
  for (int w = 0; w < NQ; ++w) {
    const int tw = base + 32 * w;
    if (tw < p.total) {
      const int sw = seq_start_of(p, tw);
      const int l2 = max(sw, tw - p.wl + 1);
      c0 = min(c0, (l2 - (tw - p.wl + 1)) / kChunk);
    }
  }

  const int kbase0 = base - p.wl + 1;  // first key of block chunk 0
  const int total = p.total;
  const int64_t k_st = p.k_st, k_sh = p.k_sh, v_st = p.v_st, v_sh = p.v_sh;
  auto stage = [&](ChunkStager<D, 256>& st, int e) {
    const int k0 = kbase0 + kChunk * e;
    st.load(p.k2, p.v2, tid, [&](int kk, bool is_v) -> int64_t {
      const int key = k0 + kk;
      if (key < 0 || key >= total) return -1;
      return is_v ? (int64_t)key * v_st + (int64_t)g * v_sh : (int64_t)key * k_st + (int64_t)g * k_sh;
    });
  };

  const int half = lane >> 5, n = lane & 31;
  RowBlock<D> rb;
  // Running merge over this wave's row-group passes: out slice values for
  // d = 64*i + lane, plus (M, Z) in the log2 domain.
  float orun[D / 64];
#pragma unroll
  for (int i = 0; i < D / 64; ++i) orun[i] = 0.f;
  float Mrun = -INFINITY, Zrun = 0.f;

  const int npass = (p.nr + NRG - 1) / NRG;
  for (int ps = 0; ps < npass; ++ps) {
    const int r = ps * NRG + rg;
    const int j = t - 32 * r - n;  // this lane's short-axis key
    const bool row_ok = qvalid && r < p.nr && j >= lo1;
    rb.reset();
    rb.form_a(p.q + (int64_t)t * p.q_st + (int64_t)h * p.q_sh,
              row_ok ? p.k1 + (int64_t)j * k_st + (int64_t)g * k_sh : nullptr, half, p.q_neg != 0);

    // ---- ring prologue: chunks c0 .. c0+NQ-1
    {
      ChunkStager<D, 256> st;
#pragma unroll 1
      for (int e = 0; e < NQ; ++e) {
        stage(st, c0 + e);
        st.store(lds + ((c0 + e) % R) * L::kBytes, tid);
      }
    }
    __syncthreads();
    for (int c = c0; c < p.nc; ++c) {
      ChunkStager<D, 256> st;
      const int enext = c + NQ;
      const bool pre = enext <= p.nc - 1 + NQ - 1;
      if (pre) stage(st, enext);
      if (qvalid && c >= cfirst) {
        const int kfirst = t - p.wl + 1 + kChunk * c;  // key of chunk row 0
        const int klo = max(lo2 - kfirst, 0);
        const int khi = min(t - kfirst, kChunk - 1);
        rb.chunk(lds + ((c + qw) % R) * L::kBytes, lane, p.sl2, klo, khi);
      }
      if (pre) st.store(lds + (enext % R) * L::kBytes, tid);
      __syncthreads();
    }

    // ---- epilogue of this pass: merge the 32 rows of the wave
    const float zrow = rb.z + swap_halves(rb.z);
    const float mrow = row_ok ? rb.m : -INFINITY;
    const float Mw = wave_max(mrow);
    const float wgt = (row_ok && Mw > -INFINITY) ? fast_exp2(mrow - Mw) : 0.f;
    const float Zw = half_sum(wgt * zrow);
    float* red = (float*)lds + wid * (64 * 36);  // [64 d][36] per wave
    const bf16* v1row = p.v1 + (int64_t)(row_ok ? j : 0) * v_st + (int64_t)g * v_sh;
#pragma unroll
    for (int sl = 0; sl < D / 64; ++sl) {
#pragma unroll
      for (int dbl = 0; dbl < 2; ++dbl) {
        const int db = 2 * sl + dbl;
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
          const int dd = 32 * dbl + 8 * q4 + 4 * half;  // first of 4 consecutive d
          bf16x4 vv = row_ok ? *(const bf16x4*)(v1row + 64 * sl + dd) : bf16x4{};
#pragma unroll
          for (int e = 0; e < 4; ++e) red[(dd + e) * 36 + n] = wgt * (float)vv[e] * rb.o[db][4 * q4 + e];
        }
      }
      __syncthreads();
      float acc = 0.f;
      const floatx4* row4 = (const floatx4*)(red + lane * 36);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        floatx4 x = row4[i];
        acc += (x[0] + x[1]) + (x[2] + x[3]);
      }
      __syncthreads();
      // merge into the running result of this wave
      const float Mn = fmaxf(Mrun, Mw);
      const float a0 = Mrun > -INFINITY ? fast_exp2(Mrun - Mn) : 0.f;
      const float a1 = Mw > -INFINITY ? fast_exp2(Mw - Mn) : 0.f;
      orun[sl] = orun[sl] * a0 + acc * a1;
    }
    {
      const float Mn = fmaxf(Mrun, Mw);
      const float a0 = Mrun > -INFINITY ? fast_exp2(Mrun - Mn) : 0.f;
      const float a1 = Mw > -INFINITY ? fast_exp2(Mw - Mn) : 0.f;
      Zrun = Zrun * a0 + Zw * a1;
      Mrun = Mn;
    }
  }

  // ---- merge the NRG waves of the same (token, head) and write out / lse
  if constexpr (NRG > 1) {
    float* part = (float*)lds + wid * (D + 2);
#pragma unroll
    for (int i = 0; i < D / 64; ++i) part[64 * i + lane] = orun[i];
    if (lane == 0) {
      part[D] = Mrun;
      part[D + 1] = Zrun;
    }
    __syncthreads();
    if (rg == 0) {
      float M = -INFINITY;
#pragma unroll
      for (int k = 0; k < NRG; ++k) M = fmaxf(M, ((float*)lds + (wid + k) * (D + 2))[D]);
      float Z = 0.f;
      for (int i = 0; i < D / 64; ++i) orun[i] = 0.f;
#pragma unroll
      for (int k = 0; k < NRG; ++k) {
        const float* pk = (float*)lds + (wid + k) * (D + 2);
        const float wk = pk[D] > -INFINITY ? fast_exp2(pk[D] - M) : 0.f;
        Z += wk * pk[D + 1];
#pragma unroll
        for (int i = 0; i < D / 64; ++i) orun[i] += wk * pk[64 * i + lane];
      }
      Mrun = M;
      Zrun = Z;
    }
  }
  if (rg == 0 && qvalid) {
    const float inv = 1.f / Zrun;
    bf16* orow = p.out + (int64_t)t * p.o_st + (int64_t)h * p.o_sh;
#pragma unroll
    for (int i = 0; i < D / 64; ++i) orow[64 * i + lane] = (bf16)(orun[i] * inv);
    if (p.lse && lane == 0) p.lse[(int64_t)t * p.lse_st + h] = (Mrun + __log2f(Zrun)) * kLn2;
  }
}

// ---------------------------------------------------------------------------
// Generic (portable) prefill kernel: one workgroup per (token, query head).
template <typename T>
__global__ __launch_bounds__(kGenThreads) void prefill_generic_kernel(GenericPrefillParams gp) {
  const int t = blockIdx.x;
  const int h = blockIdx.y;
  const int s0 = seq_start(gp.cu, gp.num_seqs, gp.seqlen, t);
  const int g = h / gp.group;
  DenseRows rows{gp.k1, gp.k2, gp.v1, gp.v2, gp.k_st, gp.k_sh, gp.v_st, gp.v_sh, (int64_t)s0};
  const T* q = (const T*)gp.q + (int64_t)t * gp.q_st + (int64_t)h * gp.q_sh;
  T* out = (T*)gp.out + (int64_t)t * gp.o_st + (int64_t)h * gp.o_sh;
  float* lse = gp.lse ? gp.lse + (int64_t)t * gp.lse_st + h : nullptr;
  generic_query<T, T, T>(q, rows, g, t - s0, gp.ws, gp.wl, gp.d, gp.dv, gp.scale, out, lse);
}

// ---------------------------------------------------------------------------
// Host launchers

template <int D, int NQ, int NH, int NRG>
static hipError_t launch_prefill_mfma(const PrefillParams& base_p, hipStream_t stream) {
  PrefillParams p = base_p;
  const int span = 32 * NQ;
  p.qblocks = ((p.total + span - 1) / span) * 32;
  p.hsub = p.group / NH;
  p.nblocks = p.qblocks * p.hk * p.hsub;
  constexpr int R = NQ + 1;
  size_t lds = (size_t)R * ChunkLayout<D>::kBytes;
  const size_t red = (size_t)4 * 64 * 36 * sizeof(float);
  if (lds < red) lds = red;
  auto kern = prefill_mfma_kernel<D, NQ, NH, NRG>;
  hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(kern, dim3(p.nblocks), dim3(256), lds, stream, p);
  return hipGetLastError();
}

template <int D>
static hipError_t dispatch_prefill_mfma_d(const PrefillParams& p, hipStream_t stream) {
  const int G = p.group;
  const bool multi_rg = p.nr >= 2;
  if (G % 4 == 0) {
    return launch_prefill_mfma<D, 1, 4, 1>(p, stream);
  }
  if (G % 2 == 0) {
    if (multi_rg) return launch_prefill_mfma<D, 1, 2, 2>(p, stream);
    return launch_prefill_mfma<D, 2, 2, 1>(p, stream);
  }
  if (multi_rg) return launch_prefill_mfma<D, 2, 1, 2>(p, stream);
  if (D >= 256) return launch_prefill_mfma<D, 2, 1, 2>(p, stream);
  return launch_prefill_mfma<D, 4, 1, 1>(p, stream);
}

hipError_t launch_prefill_bf16_mfma(const sa_prefill_args* a, hipStream_t stream) {
  PrefillParams p{};
  p.q = (const bf16*)a->q;
  p.k1 = (const bf16*)a->k1;
  p.k2 = (const bf16*)a->k2;
  p.v1 = (const bf16*)a->v1;
  p.v2 = (const bf16*)a->v2;
  p.out = (bf16*)a->out;
  p.lse = a->lse;
  p.cu = a->cu_seqlens;
  p.q_st = a->q_stride_t;
  p.q_sh = a->q_stride_h;
  p.k_st = a->k_stride_t;
  p.k_sh = a->k_stride_h;
  p.v_st = a->v_stride_t;
  p.v_sh = a->v_stride_h;
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
  p.sl2 = fabsf(a->scale) * kLog2e;
  p.q_neg = a->scale < 0.f;
  switch (a->head_dim) {
    case 64: return dispatch_prefill_mfma_d<64>(p, stream);
    case 128: return dispatch_prefill_mfma_d<128>(p, stream);
    case 256: return dispatch_prefill_mfma_d<256>(p, stream);
    default: return hipErrorInvalidValue;
  }
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
    hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(kern, grid, dim3(kGenThreads), lds, stream, gp);
  } else {
    auto kern = prefill_generic_kernel<bf16>;
    hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(kern, grid, dim3(kGenThreads), lds, stream, gp);
  }
  return hipGetLastError();
}

}  // namespace sa
