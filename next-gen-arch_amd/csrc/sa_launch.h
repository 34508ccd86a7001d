// Host-side launch interface between the C ABI (sa_capi.hip) and the kernel
// translation units.
#pragma once

#include <hip/hip_runtime.h>

#include "../../include/simplicial_mi355x.h"

namespace sa {

struct GenericPrefillParams {
  const void* q;
  const void* k1;
  const void* k2;
  const void* v1;
  const void* v2;
  void* out;
  float* lse;
  const int32_t* cu;
  int64_t q_st, q_sh, k_st, k_sh, v_st, v_sh, o_st, o_sh, lse_st;
  int seqlen, num_seqs, group, ws, wl, d, dv;
  float scale;
};

// MFMA prefill: bf16 inputs, or fp32 inputs with a->workspace of
// prefill_f32_workspace_bytes(a) bytes (the hi/lo split of k2, v2, v1).
hipError_t launch_prefill_mfma(const sa_prefill_args* a, hipStream_t stream);
size_t prefill_f32_workspace_bytes(const sa_prefill_args* a);
hipError_t launch_prefill_generic(const sa_prefill_args* a, hipStream_t stream);
// fp32 rows [tokens][heads][d] (element strides st_t, st_h) -> bf16 rows
// [tokens][heads][hi: d | lo: d], hi + lo = x to 2^-17 relative
hipError_t launch_split_hilo(const float* src, int64_t st_t, int64_t st_h, int64_t tokens, int heads, int d,
                             __bf16* dst, hipStream_t stream);

// Paged: number of split partials per (token, head) and the launch itself.
int paged_mfma_supported(const sa_paged_args* a);
int paged_choose_splits(const sa_paged_args* a);
size_t paged_workspace_bytes(const sa_paged_args* a, int splits);
hipError_t launch_paged(const sa_paged_args* a, int splits, void* ws, size_t ws_bytes, hipStream_t stream);

// Backward (sa_backward.hip).
size_t prefill_bwd_workspace_bytes(const sa_prefill_bwd_args* a);
hipError_t launch_prefill_bwd(const sa_prefill_bwd_args* a, void* ws, hipStream_t stream);

int device_cu_count();

// Raise a kernel's dynamic-LDS limit (hipFuncSetAttribute) once per kernel,
// device and size; repeated launches do not call the runtime again.
hipError_t set_lds_limit(const void* kern, size_t bytes);

}  // namespace sa
