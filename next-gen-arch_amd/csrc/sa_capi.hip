// extern "C" entry points of libsimplicial_mi355x.so (declared in
// include/simplicial_mi355x.h).  Argument checks mirror the reference's
// ValueError contracts (simplicial_attention.py:17-38, :87-92;
// simplicial_paged.py:78-103); the Python shim raises the same messages before
// calling in, these checks guard C callers.
#include <map>
#include <mutex>
#include <string>
#include <utility>

#include "sa_launch.h"

namespace sa {

static thread_local std::string g_last_error;
constexpr int64_t kChunkClip = 32;  // keys per chunk of the MFMA kernels' long-axis grid

static int fail(int code, const char* msg) {
  g_last_error = msg;
  return code;
}

int device_cu_count() {
  static std::mutex mu;
  static int counts[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  std::lock_guard<std::mutex> lock(mu);
  if (counts[dev] == 0) {
    int c = 0;
    if (hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || c <= 0) c = 256;
    counts[dev] = c;
  }
  return counts[dev];
}

hipError_t set_lds_limit(const void* kern, size_t bytes) {
  // hipFuncSetAttribute once per (kernel, device) and size: later launches of
  // the same instantiation skip the runtime call.
  static std::mutex mu;
  static std::map<std::pair<const void*, int>, size_t> done;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) dev = -1;
  std::lock_guard<std::mutex> lock(mu);
  size_t& have = done[{kern, dev}];
  if (have >= bytes) return hipSuccess;
  hipError_t e = hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
  if (e == hipSuccess) have = bytes;
  return e;
}

// Windows longer than any sequence can reach are clipped before the launch:
// a key is valid when s0 <= j <= t and j > t - w, and t - s0 is below the
// bound (the dense sequence length, the packed token count, or a block
// table's capacity), so every window w >= bound selects the same keys.  The
// clip removes whole 32-key chunks only (w mod 32 is kept): the chunk grid
// starts at t - w + 1, so the clipped call runs the same chunks in the same
// order and its results are bit-identical to the unclipped ones, while chunk
// counts, row-group passes and int32 arithmetic on the window stay bounded
// (callers pass 1 << 30 and more for global layers).
static int32_t clip_window(int32_t w, int64_t bound) {
  if (bound < 1) bound = 1;
  if (w <= bound) return w;
  return (int32_t)(w - (w - bound) / kChunkClip * kChunkClip);
}

static sa_prefill_args clip_prefill(const sa_prefill_args* a) {
  sa_prefill_args c = *a;
  const int64_t bound = a->cu_seqlens ? a->total_tokens : a->seqlen;
  c.short_window = clip_window(c.short_window, bound);
  c.long_window = clip_window(c.long_window, bound);
  return c;
}

// Paged: a well-formed token's own slot is in both tables, so its position is
// below width * block_size of each table.
static sa_paged_args clip_paged(const sa_paged_args* a) {
  sa_paged_args c = *a;
  c.short_window = clip_window(c.short_window, (int64_t)a->short_table_width * a->block_size);
  c.long_window = clip_window(c.long_window, (int64_t)a->long_table_width * a->block_size);
  return c;
}

static bool pow2_dim(int d, int lo, int hi) { return d >= lo && d <= hi && (d & (d - 1)) == 0; }

static int check_prefill(const sa_prefill_args* a) {
  if (!a) return fail(SA_ERR_INVALID, "null arguments");
  if (!a->q || !a->k1 || !a->k2 || !a->v1 || !a->v2 || !a->out) return fail(SA_ERR_INVALID, "null tensor pointer");
  if (a->short_window < 1 || a->long_window < a->short_window)
    return fail(SA_ERR_INVALID, "require 1 <= short_window <= long_window");
  if (a->heads_q < 1 || a->heads_kv < 1 || a->head_dim < 1 || a->value_dim < 1 || a->num_seqs < 1)
    return fail(SA_ERR_INVALID, "empty attention dimensions are unsupported");
  if (a->heads_q % a->heads_kv) return fail(SA_ERR_INVALID, "incompatible grouped-query geometry");
  if (a->heads_q / a->heads_kv > 128) return fail(SA_ERR_INVALID, "at most 128 query heads per KV group");
  if (!pow2_dim(a->head_dim, 16, 512)) return fail(SA_ERR_INVALID, "unsupported score head dimension");
  if (!pow2_dim(a->value_dim, 16, 256)) return fail(SA_ERR_INVALID, "unsupported value head dimension");
  if (a->dtype != SA_DTYPE_F32 && a->dtype != SA_DTYPE_BF16)
    return fail(SA_ERR_INVALID, "kernel supports float32/bfloat16");
  if (a->cu_seqlens == nullptr) {
    if (a->seqlen < 1 || (int64_t)a->seqlen * a->num_seqs != a->total_tokens)
      return fail(SA_ERR_INVALID, "dense layout needs total_tokens == num_seqs * seqlen");
  }
  if (a->total_tokens < 0) return fail(SA_ERR_INVALID, "negative token count");
  return SA_OK;
}

// fp32 inputs on the matrix cores: D == DV in {64, 128}, 16-byte aligned
// rows (strides in multiples of 4 elements), and the hi/lo workspace
static bool f32_mfma_shape(const sa_prefill_args* a) {
  if (a->dtype != SA_DTYPE_F32 || (a->flags & SA_FLAG_FORCE_GENERIC)) return false;
  if (a->head_dim != a->value_dim || (a->head_dim != 64 && a->head_dim != 128)) return false;
  const int64_t st[] = {a->q_stride_t, a->q_stride_h, a->k_stride_t, a->k_stride_h,
                        a->v_stride_t, a->v_stride_h, a->o_stride_t, a->o_stride_h};
  for (int64_t s : st)
    if (s % 4) return false;
  const uintptr_t ptrs = (uintptr_t)a->q | (uintptr_t)a->k1 | (uintptr_t)a->k2 | (uintptr_t)a->v1 |
                         (uintptr_t)a->v2 | (uintptr_t)a->out;
  return (ptrs & 15) == 0;
}

static bool mfma_prefill_ok(const sa_prefill_args* a) {
  if (a->flags & SA_FLAG_FORCE_GENERIC) return false;
  if (a->dtype == SA_DTYPE_F32)
    return f32_mfma_shape(a) && a->workspace && !((uintptr_t)a->workspace & 255) &&
           a->workspace_bytes >= prefill_f32_workspace_bytes(a);
  if (a->dtype != SA_DTYPE_BF16) return false;
  // score width DK, value width DV: DK == DV in {64, 128, 256}, or DK == 2 DV
  // in {128, 256, 512} (the determinant-score expansion of DV = 64 / 128 / 256)
  const int dk = a->head_dim, dv = a->value_dim;
  const bool same = dk == dv && (dk == 64 || dk == 128 || dk == 256);
  const bool expanded = (dk == 128 && dv == 64) || (dk == 256 && dv == 128) || (dk == 512 && dv == 256);
  if (!same && !expanded) return false;
  const int64_t st[] = {a->q_stride_t, a->q_stride_h, a->k_stride_t, a->k_stride_h,
                        a->v_stride_t, a->v_stride_h, a->o_stride_t, a->o_stride_h};
  for (int64_t s : st)
    if (s % 8) return false;
  // per-lane tile offsets are 32-bit buffer offsets below 2^31 bytes
  if (a->k_stride_t >= (int64_t(1) << 24) || a->v_stride_t >= (int64_t(1) << 24)) return false;
  const uintptr_t ptrs = (uintptr_t)a->q | (uintptr_t)a->k1 | (uintptr_t)a->k2 | (uintptr_t)a->v1 |
                         (uintptr_t)a->v2 | (uintptr_t)a->out;
  return (ptrs & 15) == 0;
}

static int check_paged(const sa_paged_args* a) {
  if (!a) return fail(SA_ERR_INVALID, "null arguments");
  if (a->tokens < 0) return fail(SA_ERR_INVALID, "negative token count");
  if (a->short_window < 1 || a->long_window < a->short_window)
    return fail(SA_ERR_INVALID, "require 1 <= short_window <= long_window");
  if (a->heads_q < 1 || a->heads_kv < 1 || a->heads_q % a->heads_kv || a->block_size < 1 ||
      !pow2_dim(a->head_dim, 16, 256))
    return fail(SA_ERR_INVALID, "incompatible paged simplicial geometry");
  if (a->heads_q / a->heads_kv > 128) return fail(SA_ERR_INVALID, "at most 128 query heads per KV group");
  // queries fp32 / bf16 (simplicial_paged.py:88); caches also fp16 (the
  // reference's loads take any float cache and cast, :42-52)
  auto fp = [](int32_t d) { return d == SA_DTYPE_F32 || d == SA_DTYPE_BF16; };
  auto cf = [](int32_t d) { return d == SA_DTYPE_F32 || d == SA_DTYPE_BF16 || d == SA_DTYPE_F16; };
  auto ix = [](int32_t d) { return d == SA_INDEX_I32 || d == SA_INDEX_I64; };
  if (!fp(a->q_dtype) || !cf(a->cache_dtype) || !cf(a->long_cache_dtype) || !ix(a->table_index_dtype) ||
      !ix(a->long_table_index_dtype) || !ix(a->token_index_dtype) || !ix(a->token_pos_index_dtype))
    return fail(SA_ERR_INVALID, "invalid paged simplicial inputs");
  if (a->tokens > 0 && (a->num_seqs < 1 || a->short_table_width < 1 || a->long_table_width < 1 ||
                        a->short_blocks < 1 || a->long_blocks < 1))
    return fail(SA_ERR_INVALID, "invalid paged simplicial inputs");
  if (a->tokens > 0 && (!a->q || !a->short_cache || !a->long_cache || !a->short_table || !a->long_table ||
                        !a->token_seq || !a->token_pos || !a->out))
    return fail(SA_ERR_INVALID, "null tensor pointer");
  return SA_OK;
}

// ---------------------------------------------------------------------------
// Static scratch for sa_paged_fwd_noalloc: the split partials of the paged
// launch live in this device array instead of a caller workspace.  Each GPU
// the library runs on holds its own copy (kScratchBytes) until the process
// ends.  Host code must not pass `scratch` itself to a kernel (in host code
// the name is a stand-in, not a device address): the device address is
// looked up once per device with hipGetSymbolAddress and kept in
// g_scratch_ptr, and only that pointer is used.  The paged kernels write every
// partial of a launch before the combine reads it, so nothing needs clearing
// between calls.  Calls that overlap on one GPU share the array and race.
constexpr size_t kScratchBytes = size_t(16) << 20;
static __device__ __align__(256) char scratch[kScratchBytes];
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[64];

static int scratch_address(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(SA_ERR_HIP, hipGetErrorString(e));
  if (dev < 0 || dev >= 64) return fail(SA_ERR_UNSUPPORTED, "device index beyond the scratch table (64)");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) return fail(SA_ERR_HIP, e != hipSuccess ? hipGetErrorString(e) : "null scratch address");
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return SA_OK;
}

}  // namespace sa

extern "C" {

const char* sa_last_error(void) { return sa::g_last_error.c_str(); }

const char* sa_version(void) { return "simplicial_mi355x 0.3 (gfx950)"; }

int sa_abi_version(void) { return SIMPLICIAL_MI355X_ABI_VERSION; }

int sa_prefill_fwd(const sa_prefill_args* a, sa_stream_t stream) {
  int rc = sa::check_prefill(a);
  if (rc != SA_OK) return rc;
  if (a->total_tokens == 0) return SA_OK;
  const sa_prefill_args c = sa::clip_prefill(a);
  hipError_t e = sa::mfma_prefill_ok(&c) ? sa::launch_prefill_mfma(&c, (hipStream_t)stream)
                                         : sa::launch_prefill_generic(&c, (hipStream_t)stream);
  if (e != hipSuccess) return sa::fail(SA_ERR_HIP, hipGetErrorString(e));
  sa::g_last_error.clear();
  return SA_OK;
}

size_t sa_prefill_workspace_bytes(const sa_prefill_args* a) {
  if (sa::check_prefill(a) != SA_OK || !sa::f32_mfma_shape(a)) return 0;
  return sa::prefill_f32_workspace_bytes(a);
}

size_t sa_prefill_bwd_workspace_bytes(const sa_prefill_bwd_args* a) {
  if (!a || sa::check_prefill(&a->fwd) != SA_OK) return 0;
  sa_prefill_bwd_args c = *a;
  c.fwd = sa::clip_prefill(&a->fwd);
  return sa::prefill_bwd_workspace_bytes(&c);
}

int sa_prefill_bwd(const sa_prefill_bwd_args* a, void* workspace, size_t workspace_bytes, sa_stream_t stream) {
  if (!a) return sa::fail(SA_ERR_INVALID, "null arguments");
  int rc = sa::check_prefill(&a->fwd);
  if (rc != SA_OK) return rc;
  if (a->fwd.total_tokens == 0) return SA_OK;
  if (!a->fwd.lse || !a->dout || !a->dq || !a->dk1 || !a->dk2 || !a->dv1 || !a->dv2)
    return sa::fail(SA_ERR_INVALID, "null tensor pointer");
  sa_prefill_bwd_args c = *a;
  c.fwd = sa::clip_prefill(&a->fwd);
  const size_t need = sa::prefill_bwd_workspace_bytes(&c);
  if (workspace_bytes < need || !workspace) return sa::fail(SA_ERR_INVALID, "workspace too small");
  if ((uintptr_t)workspace & 255) return sa::fail(SA_ERR_INVALID, "workspace must be 256-byte aligned");
  hipError_t e = sa::launch_prefill_bwd(&c, workspace, (hipStream_t)stream);
  if (e != hipSuccess) return sa::fail(SA_ERR_HIP, hipGetErrorString(e));
  sa::g_last_error.clear();
  return SA_OK;
}

const char* sa_prefill_kernel(const sa_prefill_args* a) {
  if (sa::check_prefill(a) != SA_OK) return nullptr;
  return sa::mfma_prefill_ok(a) ? "mfma" : "generic";
}

const char* sa_paged_kernel(const sa_paged_args* a) {
  if (sa::check_paged(a) != SA_OK) return nullptr;
  return sa::paged_mfma_supported(a) ? "mfma" : "generic";
}

int sa_paged_splits(const sa_paged_args* a) {
  if (sa::check_paged(a) != SA_OK) return -1;
  const sa_paged_args c = sa::clip_paged(a);
  return sa::paged_choose_splits(&c);
}

size_t sa_paged_workspace_bytes(const sa_paged_args* a) {
  if (sa::check_paged(a) != SA_OK) return 0;
  const sa_paged_args c = sa::clip_paged(a);
  return sa::paged_workspace_bytes(&c, sa::paged_choose_splits(&c));
}

int sa_paged_fwd(const sa_paged_args* a, void* workspace, size_t workspace_bytes, sa_stream_t stream) {
  int rc = sa::check_paged(a);
  if (rc != SA_OK) return rc;
  if (a->tokens == 0) return SA_OK;
  const sa_paged_args c = sa::clip_paged(a);
  const int splits = sa::paged_choose_splits(&c);
  const size_t need = sa::paged_workspace_bytes(&c, splits);
  if (workspace_bytes < need) return sa::fail(SA_ERR_INVALID, "workspace too small");
  if (need && !workspace) return sa::fail(SA_ERR_INVALID, "null workspace");
  if (need && ((uintptr_t)workspace & 255)) return sa::fail(SA_ERR_INVALID, "workspace must be 256-byte aligned");
  hipError_t e = sa::launch_paged(&c, splits, workspace, workspace_bytes, (hipStream_t)stream);
  if (e != hipSuccess) return sa::fail(SA_ERR_HIP, hipGetErrorString(e));
  sa::g_last_error.clear();
  return SA_OK;
}

int sa_paged_fwd_noalloc(const sa_paged_args* a, sa_stream_t stream) {
  int rc = sa::check_paged(a);
  if (rc != SA_OK) return rc;
  if (a->tokens == 0) return SA_OK;
  const sa_paged_args c = sa::clip_paged(a);
  const int splits = sa::paged_choose_splits(&c);
  const size_t need = sa::paged_workspace_bytes(&c, splits);
  if (need > sa::kScratchBytes)
    return sa::fail(SA_ERR_INVALID,
                    "split partials exceed the static scratch (16 MiB); fix fewer splits or call sa_paged_fwd "
                    "with a workspace");
  void* ws = nullptr;
  if (need) {
    rc = sa::scratch_address(&ws);
    if (rc != SA_OK) return rc;
  }
  hipError_t e = sa::launch_paged(&c, splits, ws, need ? sa::kScratchBytes : 0, (hipStream_t)stream);
  if (e != hipSuccess) return sa::fail(SA_ERR_HIP, hipGetErrorString(e));
  sa::g_last_error.clear();
  return SA_OK;
}

}  // extern "C"
