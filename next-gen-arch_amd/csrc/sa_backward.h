// Parameters shared by the backward kernels (portable: sa_backward.hip, MFMA:
// sa_backward_mfma.hip).
#pragma once

#include "sa_common.h"

namespace sa {

struct BwdParams {
  const void* q;
  const void* k1;
  const void* k2;
  const void* v1;
  const void* v2;
  const void* out;
  const float* lse;
  const void* dout;
  void* dq;
  void* dk1;
  void* dk2;
  void* dv1;
  void* dv2;
  float* delta;  // [tokens, hq] workspace: dout·out - dlse
  float* dl;     // [tokens, hq] workspace: dlse (0 without an LSE gradient)
  const float* dlse;  // optional gradient of the LSE output
  int64_t dlse_st;
  const int32_t* cu;
  int64_t q_st, q_sh, k_st, k_sh, v_st, v_sh, o_st, o_sh, lse_st;
  int64_t do_st, do_sh, dq_st, dq_sh, dk_st, dk_sh, dv_st, dv_sh;
  int tokens, seqlen, num_seqs, hq, hk, group, ws, wl, d, dv;
  float scale;
  int mfma;  // bf16 inputs and the MFMA passes allowed (not forced onto the portable kernels)
  // dk1 from the dq pass (bwd_dk1_fused_ok): per dq workgroup (NQ queries x
  // NH heads of one KV group) and row group r of short keys, the 31 + NQ
  // short-key rows of Σ dA_{t,j} ⊙ q_{t,h}, fp32 [hk * hsub][qblocks][nr]
  // [31 + NQ][D], summed by bwd_dk1_sum_kernel; null: the separate dk1 pass
  float* dk1p;
  // fp32 inputs with dk1p: dv1 from the dq pass as well, the same rows of
  // Σ O''_{t,j} ⊙ dout_{t,h} (O''_{t,j} = Σ_k P_{t,j,k} v2_k), [hk * hsub]
  // [qblocks][nr][31 + NQ][DV]; null: the dk1 / dv1 pass computes dv1
  float* dv1p;
  // Short windows of 65-128 keys (33-64 at score width 256): the dk2 / dv2
  // passes run as two launches and carry the first one's fp32 sums here,
  // [tokens][hk][D] then [tokens][hk][DV]; null: the portable dk2 / dv2 pass
  float* dkv2p;
  // fp32 inputs on the matrix cores: k2 and v2 as rows of [hi: D | lo: D]
  // bf16 terms ([tokens][hk][2 D], split_hilo in the workspace); q, k1, v1,
  // dout stay fp32 and their products are split in the kernels
  const bf16* k2s;
  const bf16* v2s;
  int f32;
  // dk2 / dv2 walk splits (bwd_dkv2_plan): each split's fp32 sums over its
  // part of the queries reaching a key, [splits][tokens][hk][max(D, DV)],
  // added in split order by a second kernel; null with one split
  float* dkv2s;
};

// Queries per dq workgroup (4 waves: NQ queries x NH = 4 / NQ heads of one KV
// group), by GQA group size; the dk1 partial of a workgroup has 31 + NQ rows.
inline int dq_queries_per_block(int group) { return group % 4 == 0 ? 1 : group % 2 == 0 ? 2 : 4; }

// MFMA passes (sa_backward_mfma.hip).  Each returns hipErrorNotSupported when
// the call's shapes, dtype or strides are outside what its kernel covers; the
// portable pass runs instead.
hipError_t launch_bwd_dq_mfma(const BwdParams& p, hipStream_t stream);
hipError_t launch_bwd_dkv1_mfma(const BwdParams& p, hipStream_t stream);
hipError_t launch_bwd_dkv2_mfma(const BwdParams& p, hipStream_t stream);
// The dq pass can produce dk1 (p.dk1p set): the MFMA passes apply and the
// short window fits two 32-row groups (one for fp32 inputs).  The MFMA dkv1
// launch then computes dv1 only.
bool bwd_dk1_fused_ok(const BwdParams& p);
// dk1 = the fixed-order sum of the dq pass's partials (p.dk1p)
hipError_t launch_bwd_dk1_sum(const BwdParams& p, hipStream_t stream);
// dv1 = the same sum of the dq pass's dv1 partials (p.dv1p, fp32 inputs)
hipError_t launch_bwd_dv1_sum(const BwdParams& p, hipStream_t stream);

// MFMA dk2 / dv2 pass: waves per workgroup (32 long keys each) and walk
// splits (pieces of each workgroup's walk over the queries, for shapes whose
// (key block, KV head) workgroups leave CUs idle).  A function of the shape
// and the device's CU count only, so that the workspace query and the launch
// agree.
struct Dkv2Plan {
  int nwk, splits;
};
Dkv2Plan bwd_dkv2_plan(int tokens, int hk, int d, int dv, int ws, int wl, bool f32, int cus);

}  // namespace sa
