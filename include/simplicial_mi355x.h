/*
 * C ABI of the MI355X (gfx950) 2-simplicial attention library
 * (libsimplicial_mi355x.so).
 *
 * The reference exposes this path only as Python functions over torch
 * tensors whose kernels are Triton JIT code; there is no native FFI to mirror.
 * Each entry point below replaces the kernel launch that sits behind one of
 * those functions, so a host shim keeping the reference's Python signatures
 * can call it with plain device pointers:
 *
 *   sa_prefill_fwd            replaces SimplicialFunction.forward / _forward
 *                             (archlab/architectures/simplicial_kernels.py:109-131, :16-52)
 *                             behind simplicial_attention (simplicial_attention.py:77-97);
 *                             with cu_seqlens != NULL it is the packed
 *                             variable-length form ("same-document" visibility,
 *                             recipes/deepseek_v41/proposals.yaml:76).
 *   sa_paged_fwd              replaces the _paged launch plus the torch split
 *                             merge (simplicial_paged.py:105-128) behind
 *                             simplicial_paged_attention (simplicial_paged.py:68-128).
 *   sa_paged_workspace_bytes  size of the split partials that the reference
 *                             allocates with torch.empty/full/zeros
 *                             (simplicial_paged.py:112-114).
 *   sa_prefill_bwd            replaces SimplicialFunction.backward / _backward
 *                             (simplicial_kernels.py:133-143, :55-106) and the
 *                             deterministic backward
 *                             (simplicial_deterministic.py:86-104): gradients
 *                             of q, k1, k2, v1, v2 without atomics.
 *   sa_prefill_bwd_workspace_bytes  size of its workspace: the per-(token,
 *                             head) delta and dlse rows and, for bf16 calls
 *                             whose short window is one 32-row group, the
 *                             dk1 partials written by the dq pass (fp32:
 *                             dk1 and dv1 partials; at most 8 GiB; beyond
 *                             that, or with SA_FLAG_SEPARATE_DK1, a separate
 *                             dk1 / dv1 pass runs).
 *
 * Conventions
 *   - All pointers are device pointers; strides are in ELEMENTS; the last
 *     dimension of every tensor is contiguous (stride 1).
 *   - Score operands (q, k1, k2) have head_dim D, values (v1, v2, out) have
 *     value_dim DV.  Query head h reads KV head h / (heads_q / heads_kv).
 *   - (k1, v1, short_window) is the short key axis, (k2, v2, long_window) the
 *     long one (reference argument order and names).
 *   - The library never allocates or frees device memory and never reads
 *     device memory back to the host: every launch is asynchronous on the
 *     given stream and can be captured into a hipGraph.
 *   - Return value 0 = success; otherwise an SA_ERR_* code, with a message
 *     available from sa_last_error() (thread-local).
 */
#ifndef SIMPLICIAL_MI355X_H
#define SIMPLICIAL_MI355X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Version of the argument structs and enums below.  It changes whenever a
 * struct gains, loses or moves a field or an enum value changes meaning, so a
 * caller built against another header can detect the mismatch at load time
 * (compare sa_abi_version() with this value before the first call; the
 * structs carry no size field, and a shorter caller struct would otherwise
 * be read past its end).  3: fp16 paged caches, SA_FLAG_SEPARATE_DK1. */
#define SIMPLICIAL_MI355X_ABI_VERSION 3

/* The library is built with hidden symbol visibility; the declarations below
 * are its only exports. */
#pragma GCC visibility push(default)

typedef struct ihipStream_t* sa_stream_t; /* a hipStream_t; NULL = default stream */

enum {
  SA_OK = 0,
  SA_ERR_INVALID = 1,     /* argument / geometry check failed (ValueError) */
  SA_ERR_UNSUPPORTED = 2, /* valid but not implemented shape/dtype (ValueError) */
  SA_ERR_HIP = 3          /* HIP runtime error at launch (RuntimeError) */
};

/* Element types.  SA_DTYPE_F16 is accepted for the paged caches only (the
 * reference's paged Triton loads read any float cache, simplicial_paged.py:42-52);
 * queries and the prefill tensors are float32 or bfloat16 as in the reference
 * (simplicial_attention.py:87-88, simplicial_paged.py:88). */
enum { SA_DTYPE_F32 = 0, SA_DTYPE_BF16 = 1, SA_DTYPE_F16 = 2 };
enum { SA_INDEX_I32 = 0, SA_INDEX_I64 = 1 };

enum {
  SA_FLAG_FORCE_GENERIC = 1, /* use the portable (non-MFMA) kernel; for cross-checks */
  /* sa_prefill_bwd only: compute dk1 in a pass of its own instead of from
   * partials written by the dq pass.  The workspace then holds no dk1
   * partials (those take 16-17.5x the bytes of q per 32 keys of short
   * window); the backward runs one more recomputation pass (about 20 % more
   * time at the benchmark shape). */
  SA_FLAG_SEPARATE_DK1 = 2
};

typedef struct sa_prefill_args {
  const void* q;  /* [tokens, heads_q, D]   dtype */
  const void* k1; /* [tokens, heads_kv, D]  dtype */
  const void* k2; /* [tokens, heads_kv, D]  dtype */
  const void* v1; /* [tokens, heads_kv, DV] dtype */
  const void* v2; /* [tokens, heads_kv, DV] dtype */
  void* out;      /* [tokens, heads_q, DV]  dtype */
  float* lse;     /* [tokens, heads_q] fp32 natural-log LSE, or NULL */
  const int32_t* cu_seqlens; /* [num_seqs + 1] token offsets (varlen), or NULL (dense) */
  int64_t q_stride_t, q_stride_h;
  int64_t k_stride_t, k_stride_h; /* shared by k1 and k2 */
  int64_t v_stride_t, v_stride_h; /* shared by v1 and v2 */
  int64_t o_stride_t, o_stride_h;
  int64_t lse_stride_t;           /* lse[t * lse_stride_t + h] */
  int32_t num_seqs;     /* dense: batch; varlen: number of sequences */
  int32_t seqlen;       /* dense: tokens per sequence; varlen: ignored */
  int32_t total_tokens; /* dense: batch * seqlen; varlen: cu_seqlens[num_seqs] */
  int32_t heads_q, heads_kv, head_dim, value_dim;
  int32_t short_window, long_window;
  float scale;
  int32_t dtype; /* SA_DTYPE_* of every tensor except lse */
  int32_t flags; /* SA_FLAG_* */
  /* Device workspace for fp32 inputs (sa_prefill_workspace_bytes bytes,
   * 256-byte aligned): with it, fp32 calls run on the matrix cores (k2, v2
   * and v1 split into hi/lo bf16 terms there); without it (NULL), on the
   * portable kernel.  Unused for bf16. */
  void* workspace;
  size_t workspace_bytes;
} sa_prefill_args;

typedef struct sa_paged_args {
  const void* q; /* [tokens, heads_q, D], q_dtype */
  int64_t q_stride_t, q_stride_h;
  const void* short_cache; /* [2 (K,V), blocks, block_size, heads_kv, D], cache_dtype (f32, bf16 or f16) */
  int64_t sc_stride[4];    /* element strides of dims 0..3 */
  const void* long_cache; /* same geometry, long_cache_dtype */
  int64_t lc_stride[4];
  const void* short_table; /* [num_seqs, short_table_width] of table_index_dtype */
  int64_t st_stride;
  const void* long_table;  /* [num_seqs, long_table_width] of long_table_index_dtype; may equal short_table */
  int64_t lt_stride;
  const void* token_seq; /* [tokens] token_index_dtype */
  const void* token_pos; /* [tokens] token_pos_index_dtype */
  float* out;            /* [tokens, heads_q, D] fp32 */
  int64_t o_stride_t, o_stride_h;
  float* lse;            /* [tokens, heads_q] fp32 natural log, or NULL */
  int32_t tokens, heads_q, heads_kv, head_dim, block_size;
  int32_t num_seqs;                 /* rows of both tables */
  int32_t short_table_width, long_table_width;
  int32_t short_blocks, long_blocks; /* dim 1 of each cache; table entries are clamped to it */
  int32_t short_window, long_window;
  int32_t splits;        /* long-window splits; <= 0 selects automatically */
  float scale;
  int32_t q_dtype;           /* SA_DTYPE_* of q */
  int32_t cache_dtype;       /* SA_DTYPE_* of short_cache (F32, BF16 or F16) */
  int32_t table_index_dtype; /* SA_INDEX_* of short_table */
  int32_t token_index_dtype; /* SA_INDEX_* of token_seq */
  int32_t flags;
  int32_t long_cache_dtype;       /* SA_DTYPE_* of long_cache (F32, BF16 or F16) */
  int32_t long_table_index_dtype; /* SA_INDEX_* of long_table */
  int32_t token_pos_index_dtype;  /* SA_INDEX_* of token_pos */
  /* Optional per-token window limits, int32 [tokens][2] on the device, or
   * NULL: token t uses min(short_window, caps[t][0]) and
   * min(long_window, caps[t][1]) keys (limits below 1 act as 1).  Lets
   * callers bound windows by device-resident lengths without a host read. */
  const int32_t* token_window_caps;
} sa_paged_args;

/* Dense or packed-varlen prefill forward: out and (optionally) lse. */
int sa_prefill_fwd(const sa_prefill_args* args, sa_stream_t stream);

/* Bytes of workspace that lets sa_prefill_fwd run fp32 inputs on the matrix
 * cores (0 when the call's shape or dtype has no use for one).  No
 * counterpart in the reference: its fp32 path keeps tf32x3 dots on the same
 * Triton kernel (simplicial_kernels.py:42, :48). */
size_t sa_prefill_workspace_bytes(const sa_prefill_args* args);

typedef struct sa_prefill_bwd_args {
  sa_prefill_args fwd;   /* the forward call: out = its output, lse (required) its LSE */
  const void* dout;      /* [tokens, heads_q, DV] dtype: gradient of out */
  int64_t do_stride_t, do_stride_h;
  void* dq;              /* [tokens, heads_q, D]   dtype */
  int64_t dq_stride_t, dq_stride_h;
  void* dk1;             /* [tokens, heads_kv, D]  dtype */
  void* dk2;             /* [tokens, heads_kv, D]  dtype, strides shared with dk1 */
  int64_t dk_stride_t, dk_stride_h;
  void* dv1;             /* [tokens, heads_kv, DV] dtype */
  void* dv2;             /* [tokens, heads_kv, DV] dtype, strides shared with dv1 */
  int64_t dv_stride_t, dv_stride_h;
  const float* dlse;     /* [tokens, heads_q] fp32 gradient of lse (dlse[t * dlse_stride_t + h]), or NULL */
  int64_t dlse_stride_t;
} sa_prefill_bwd_args;

/* Bytes of device workspace sa_prefill_bwd needs (256-byte aligned): two fp32
 * [tokens, heads_q] rows, plus
 * - the dq pass's dk1 partials where it produces dk1 (bf16 with head_dim and
 *   value_dim each 64 or 128, or head_dim 256 over value_dim 128 / 256, short
 *   window <= 64; fp32 with head_dim == value_dim in {64, 128}, short window
 *   <= 32): 16-17.5x the bytes of q per 32 keys of short window, up to 8 GiB;
 *   none with SA_FLAG_SEPARATE_DK1 in args->fwd.flags; fp32 calls also hold
 *   the dq pass's dv1 partials, the same size at value_dim (dk1 and dv1
 *   partials together up to 8 GiB, else the dv1 pass runs);
 * - for short windows of 65-128 (33-64 at head_dim 256), the fp32 dk2 and dv2
 *   sums of the first of two dk2 / dv2 launches ([tokens][heads_kv][head_dim +
 *   value_dim]);
 * - for fp32 inputs on the matrix cores, k2 and v2 as hi/lo bf16 rows
 *   ([tokens][heads_kv][2 head_dim] each);
 * - for bf16 at widths 64 / 128 and short windows <= 64 whose (key block, KV
 *   head) work leaves CUs idle (few KV heads over few tokens), the fp32 sums of
 *   the dk2 / dv2 pass's walk pieces ([pieces <= 8][tokens][heads_kv]
 *   [max(head_dim, value_dim)]). */
size_t sa_prefill_bwd_workspace_bytes(const sa_prefill_bwd_args* args);

/* Backward of sa_prefill_fwd: writes dq, dk1, dk2, dv1, dv2 (each exactly
 * once, fixed reduction order: bitwise reproducible). */
int sa_prefill_bwd(const sa_prefill_bwd_args* args, void* workspace, size_t workspace_bytes,
                   sa_stream_t stream);

/* Bytes of device workspace sa_paged_fwd needs for these arguments. */
size_t sa_paged_workspace_bytes(const sa_paged_args* args);

/* Paged forward for any mix of prefill and decode tokens; workspace must hold
 * sa_paged_workspace_bytes(args) bytes (256-byte aligned). */
int sa_paged_fwd(const sa_paged_args* args, void* workspace, size_t workspace_bytes,
                 sa_stream_t stream);

/* sa_paged_fwd without a caller workspace, for callers that cannot allocate
 * device memory (code under hipGraph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  No counterpart in the reference (its paged call
 * allocates its split partials with torch, simplicial_paged.py:112-114).
 * The split partials live in a static device array of 16 MiB per GPU, held
 * until the process ends; arguments whose partials need more (see
 * sa_paged_workspace_bytes) fail with SA_ERR_INVALID.  The call allocates
 * nothing.  Calls that overlap on one GPU share that array and race: order
 * them on one stream (or otherwise serialise them). */
int sa_paged_fwd_noalloc(const sa_paged_args* args, sa_stream_t stream);

/* Splits the paged launch would use for these arguments (after auto-selection). */
int sa_paged_splits(const sa_paged_args* args);

/* Name of the kernel family a call with these arguments runs: "mfma" (bf16
 * matrix-core path) or "generic" (portable path, fp32 and other shapes);
 * NULL if the arguments are invalid. */
const char* sa_prefill_kernel(const sa_prefill_args* args);
const char* sa_paged_kernel(const sa_paged_args* args);

/* Message describing the last failed call on this thread ("" if none). */
const char* sa_last_error(void);

/* Library version string. */
const char* sa_version(void);

/* SIMPLICIAL_MI355X_ABI_VERSION of the header the library was built from. */
int sa_abi_version(void);

#pragma GCC visibility pop

#ifdef __cplusplus
}
#endif

#endif /* SIMPLICIAL_MI355X_H */
