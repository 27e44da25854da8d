/*
 * rpa.h -- C ABI of librpa_hip.so, the MI355X (gfx950) Ragged Paged Attention
 * library.
 *
 * Every pointer is a device pointer; the library never synchronises the host
 * and never allocates device memory on the rpa_forward path (the caller
 * passes a workspace of rpa_workspace_size() bytes; its contents need no
 * initialisation, and calls sharing one workspace must be ordered on one
 * stream).  q, k, v, kv_cache and out must be 16-byte aligned.  Calls are
 * ordered on the given HIP stream (a hipStream_t passed as void*; NULL =
 * default stream).
 *
 * Reference interfaces replaced (paths relative to the vllm-torchtpu tree):
 *   rpa_forward          <- ragged_paged_attention(...)
 *                           src/vllm_torchtpu/kernels/ragged_paged_attention/v3/kernel.py:1633-1984
 *                           (the three pallas_call launches at :1950-1974 and the
 *                           fused cache write at :652-715)
 *   rpa_kv_cache_update  <- the cache-write half of the same call
 *                           (kernel.py:652-715; reference semantics kernel.py:154-166)
 *   rpa_get_kv_cache_shape <- get_kv_cache_shape, kernel.py:278-292
 *   rpa_workspace_size   <- get_vmem_estimate_bytes / scratch_shapes,
 *                           kernel.py:231-275, :1804-1841 (scratch sizing)
 *   rpa_status_str       <- the ValueError messages of static_validate_inputs,
 *                           kernel.py:1366-1538 (status codes instead of exceptions)
 */
#ifndef RPA_H_
#define RPA_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define RPA_ABI_VERSION 1

/* Element types (kernel.py accepts any float KV dtype; these are the ones
 * this library implements). */
typedef enum rpa_dtype {
  RPA_DTYPE_F32 = 0,
  RPA_DTYPE_BF16 = 1,
  RPA_DTYPE_F16 = 2,
  RPA_DTYPE_FP8_E4M3FN = 3,
  RPA_DTYPE_FP8_E5M2 = 4,
} rpa_dtype;

/* Status codes.  Negative = error.  The Python layer maps INVALID_ARG and
 * UNSUPPORTED to ValueError/NotImplementedError and the rest to RuntimeError. */
typedef enum rpa_status {
  RPA_OK = 0,
  RPA_ERR_INVALID_ARG = -1,  /* descriptor violates a kernel.py:1366-1538 rule */
  RPA_ERR_UNSUPPORTED = -2,  /* valid for the reference, not implemented here  */
  RPA_ERR_WORKSPACE = -3,    /* workspace NULL or smaller than required        */
  RPA_ERR_LAUNCH = -4,       /* a HIP launch failed                            */
  RPA_ERR_NULL_PTR = -5,     /* a required pointer is NULL                     */
  RPA_ERR_ABI = -6,          /* descriptor abi_version mismatch                */
  RPA_ERR_SCRATCH = -7,      /* rpa_forward_noalloc: needs more than its scratch */
} rpa_status;

/* Kernel-path selection (rpa_desc.path). */
typedef enum rpa_path {
  RPA_PATH_AUTO = 0,    /* pick the fastest implementation for the shape       */
  RPA_PATH_GENERIC = 1, /* force the shape-generic wave-per-row implementation */
  /* Measurement only: launch the decode kernel alone (the kernel the
   * benchmark's roofline times).  Outputs of decode rows whose key range is
   * split over several units, and every non-decode row, are left unfinished;
   * RPA_ERR_UNSUPPORTED when the decode kernel does not take the descriptor's
   * dtypes or extents (which rows are decode rows is decided on the device). */
  RPA_PATH_DECODE_ONLY = 2,
} rpa_path;

/* Plain-old-data descriptor of one call.  Shapes follow kernel.py:1609-1631:
 *   queries  [max_num_tokens, num_q_heads, head_dim]           (q_dtype)
 *   keys     [max_num_tokens, num_kv_heads, head_dim]          (kv_dtype)
 *   values   [max_num_tokens, num_kv_heads, head_dim]          (kv_dtype)
 *   kv_cache [total_num_pages, page_size, kv_heads_x2 / kv_packing,
 *             kv_packing, head_dim_padded]                      (kv_dtype)
 *   kv_lens  i32[max_num_seqs], page_indices i32[max_num_seqs * pages_per_seq],
 *   cu_q_lens i32[max_num_seqs + 1], distribution i32[3]
 *   out      [max_num_tokens, num_q_heads, head_dim]           (out_dtype)
 * All tensors are dense row-major.  The kernels may load every one of the
 * max_num_seqs entries of kv_lens and cu_q_lens (so all must be allocated);
 * entries of sequences at or past distribution[2] change nothing, whatever
 * they hold. */
typedef struct rpa_desc {
  int32_t abi_version; /* = RPA_ABI_VERSION */
  int32_t q_dtype;     /* rpa_dtype of queries                */
  int32_t kv_dtype;    /* rpa_dtype of keys, values, kv_cache */
  int32_t out_dtype;   /* rpa_dtype of out                    */
  int32_t max_num_tokens;
  int32_t num_q_heads;
  int32_t num_kv_heads;
  int32_t head_dim;        /* actual head_dim of q/k/v            */
  int32_t head_dim_padded; /* align(head_dim, 128): cache last axis (64: hd64 packed) */
  int32_t total_num_pages;
  int32_t page_size;
  int32_t kv_packing;      /* 32 / bits(kv_dtype)                  */
  int32_t kv_heads_x2;     /* align(2 * num_kv_heads, kv_packing); hd64 packed:
                              2 * align(num_kv_heads, kv_packing) */
  int32_t max_num_seqs;
  int32_t pages_per_seq;
  int32_t use_causal_mask; /* bool */
  int32_t skip_kv_update;  /* bool */
  int32_t sliding_window;  /* <= 0 means None */
  int32_t has_soft_cap;    /* bool */
  float soft_cap;
  float sm_scale;
  float q_scale; /* multiplies the logits; 1.0 when None */
  float k_scale; /* multiplies the logits; 1.0 when None */
  float v_scale; /* multiplies the output; 1.0 when None */
  int32_t path;  /* rpa_path */
  /* Largest q_len of a decode row group (spec-verify windows of K + 1 query
   * tokens), as batched_rpa/wrapper.py:549 `decode_query_size`; 0 or 1 = one
   * token.  Sequences with 1 <= q_len <= min(decode_query_size,
   * 16 / (num_q_heads / num_kv_heads)) run on the decode kernel; the result
   * does not depend on it. */
  int32_t decode_query_size;
  /* bool: sliding_window also masks rows without the causal mask (keys
   * j <= p - sliding_window excluded, p the row's position), as the head_dim-64
   * reference does (kernel_hd64.py:155-158, :443-446).  0 = the window masks
   * causal rows only (kernel.py:196-204).  With use_causal_mask = 0 and a
   * window, such calls run on the shape-generic kernels. */
  int32_t window_all_rows;
  int32_t reserved[5];
} rpa_desc;

/* ABI version compiled into the library. */
int rpa_abi_version(void);

/* Human-readable text for a status code (static storage). */
const char* rpa_status_str(int status);

/* Check a descriptor against the static rules of kernel.py:1366-1538 that
 * apply at this level.  Returns RPA_OK or a negative status. */
int rpa_validate_desc(const rpa_desc* d);

/* Cache shape contract, kernel.py:278-292: writes 5 extents to shape_out. */
int rpa_get_kv_cache_shape(int32_t total_num_pages, int32_t page_size,
                           int32_t num_kv_heads, int32_t head_dim,
                           int32_t kv_dtype, int64_t shape_out[5]);

/* Workspace bytes rpa_forward needs for this descriptor (depends only on
 * the static extents, never on metadata values). */
size_t rpa_workspace_size(const rpa_desc* d);

/* Write the new tokens' K/V into their pages: for every sequence
 * s < distribution[2] and new token t, position
 * j = kv_lens[s] - q_len + (t - cu_q_lens[s]) of page
 * page_indices[s * pages_per_seq + j / page_size], slot j % page_size, gets the
 * merged record (K_h at combined head 2h, V_h at 2h+1, zero padding).
 * No other cache byte changes.  Metadata that points outside the cache is
 * skipped, never written through. */
int rpa_kv_cache_update(const rpa_desc* d, const void* keys, const void* values,
                        void* kv_cache, const int32_t* kv_lens,
                        const int32_t* page_indices, const int32_t* cu_q_lens,
                        const int32_t* distribution, void* stream);

/* Full RPA call: cache update (unless skip_kv_update) and attention for
 * sequences [0, distribution[2]); attention reads this call's new tokens from
 * k/v (as the Pallas kernel does, kernel.py:634-641), or from the cache when
 * skip_kv_update.  Output rows >= cu_q_lens[num_seqs] are left untouched. */
int rpa_forward(const rpa_desc* d, const void* queries, const void* keys,
                const void* values, void* kv_cache, const int32_t* kv_lens,
                const int32_t* page_indices, const int32_t* cu_q_lens,
                const int32_t* distribution, void* out, void* workspace,
                size_t workspace_bytes, void* stream);

/* rpa_forward that also writes lse (f32 [max_num_tokens, num_q_heads],
 * device memory): the natural-log log-sum-exp m + log(l) of every computed
 * output row over the keys it attends (logits after sm_scale, k_scale,
 * q_scale and the soft cap; -inf for a row that attends no key).  Rows of lse
 * >= cu_q_lens[num_seqs] are left untouched.  Replaces the return_lse output
 * of the batched RPA wrapper,
 *   src/vllm_torchtpu/kernels/experimental/batched_rpa/wrapper.py:553, :610-623
 *   (LSE = m + log(max(l, 1e-9)), batched_rpa/kernel.py:116-124),
 * the partial results that context-parallel attention merges. */
int rpa_forward_lse(const rpa_desc* d, const void* queries, const void* keys,
                    const void* values, void* kv_cache, const int32_t* kv_lens,
                    const int32_t* page_indices, const int32_t* cu_q_lens,
                    const int32_t* distribution, void* out, float* lse, void* workspace,
                    size_t workspace_bytes, void* stream);

/* rpa_forward with the optional outputs and inputs of the reference's kernel
 * variants.  attention_sink (f32 [num_q_heads], device memory, or NULL): a
 * per-q-head logit that joins every row's softmax with value 0, as
 * ragged_paged_attention_hd64's attention_sink does
 *   src/vllm_torchtpu/kernels/ragged_paged_attention/v3/kernel_hd64.py:1377-1388,
 *   reference semantics :161-172.
 * lse as in rpa_forward_lse; lse and attention_sink together are
 * RPA_ERR_UNSUPPORTED.  The head_dim 64 packed cache of kernel_hd64.py
 * (:246-261, K|V of a head in one 128-wide row) is described by head_dim = 64,
 * head_dim_padded = 64 and kv_heads_x2 = 2 * align(num_kv_heads, kv_packing):
 * the same bytes. */
int rpa_forward_ex(const rpa_desc* d, const void* queries, const void* keys,
                   const void* values, void* kv_cache, const int32_t* kv_lens,
                   const int32_t* page_indices, const int32_t* cu_q_lens,
                   const int32_t* distribution, void* out, const float* attention_sink,
                   float* lse, void* workspace, size_t workspace_bytes, void* stream);

/* LSE-weighted merge of num_parts partial attentions of the same rows:
 * outs [num_parts, rows, head_dim] and lses [num_parts, rows] (f32, natural
 * log) -> out [rows, head_dim] and, when lse_out is not NULL, lse_out [rows].
 * dtype (RPA_DTYPE_BF16 or RPA_DTYPE_F32) is that of outs, out_dtype that of
 * out (the reference returns f32: its f32 weights promote bf16 partials);
 * head_dim <= 512.  Replaces merge_attn_results,
 *   src/vllm_torchtpu/layers/adapter/cp_attention.py:45-72
 * (exactly, for num_parts = 2: NaN and +-inf partial outputs count as 0, a NaN
 * lse propagates through the max as torch.maximum does) and the local
 * combine of cp_lse_ag_out_rs, distributed/dcp_comm.py:23-68. */
int rpa_merge_attn_states(int32_t num_parts, int64_t rows, int32_t head_dim, int32_t dtype,
                          int32_t out_dtype, const void* outs, const float* lses, void* out,
                          float* lse_out, void* stream);

/* Size of rpa_forward_noalloc's fixed device scratch (per GPU). */
#define RPA_NOALLOC_SCRATCH_BYTES ((size_t)32 << 20)

/* rpa_forward without a workspace argument: the same kernels, with the decode
 * partials and work plan in a fixed RPA_NOALLOC_SCRATCH_BYTES device buffer
 * that the library holds per GPU (a static device array; each GPU it runs on
 * keeps its own copy until the process ends).  It allocates nothing: no
 * hipMalloc, hipFree or allocating library call, ever.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Returns RPA_ERR_SCRATCH when rpa_workspace_size(d) exceeds
 * RPA_NOALLOC_SCRATCH_BYTES (call rpa_forward with a workspace then).  Every
 * call on one GPU shares that GPU's buffer, so calls that overlap on one GPU
 * (different streams, or different host threads without ordering) race;
 * calls ordered on one stream are safe.  Nothing in the buffer needs
 * clearing between calls. */
int rpa_forward_noalloc(const rpa_desc* d, const void* queries, const void* keys,
                        const void* values, void* kv_cache, const int32_t* kv_lens,
                        const int32_t* page_indices, const int32_t* cu_q_lens,
                        const int32_t* distribution, void* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* RPA_H_ */
