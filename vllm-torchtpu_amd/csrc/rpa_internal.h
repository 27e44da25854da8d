// Host-side launcher declarations shared between the kernel translation
// units and the C ABI (rpa_api.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "rpa_common.h"

namespace rpa {

hipError_t launch_kv_update(const Params& p, int elem_bytes, const void* k, const void* v,
                            void* cache, const int32_t* kv_lens, const int32_t* page_indices,
                            const int32_t* cu, const int32_t* dist, hipStream_t stream);

// Largest max_num_seqs the in-LDS work plan of the decode and finish kernels
// accepts.
constexpr int kMaxDecodeSeqs = 2048;

// Slices of the caller's workspace used by the decode path (no
// initialisation needed).
struct DecodeWorkspace {
  float* part_o;   // [slots][rows][Dp] un-normalised partial outputs
  float* part_ml;  // [slots][rows][2] (row max in log2 units, row sum)
  int32_t* plan;   // the decode kernel's plan for the finish kernel (layout below)
  int64_t slots;   // decode wavefronts + max_num_seqs * Hkv (the stream-K slot bound)
};


// Plan written by the decode kernel (rpa_plan.h): [0] num_seqs n, [1] tiles
// per wavefront, [2] total tiles G, [3] sequences with non-decode rows;
// base[S + 1] (exclusive prefix of tiles per sequence, base[n] = total),
// dkv[S] (kv_len of a decode sequence, else 0), tq[S] (q row of the
// sequence), rowseq[T] (sequence of a token row the finish kernel owns, -1 for
// decode rows and padding rows).
struct PlanView {
  const int32_t* hdr;
  const int32_t* base;
  const int32_t* dkv;
  const int32_t* tq;
  const int32_t* rowseq;
};
__host__ __device__ inline PlanView plan_view(const int32_t* plan, int32_t S) {
  PlanView v;
  v.hdr = plan;
  v.base = plan + 4;
  v.dkv = v.base + (S + 1);
  v.tq = v.dkv + S;
  v.rowseq = v.tq + S;
  return v;
}
__host__ __device__ inline int64_t plan_ints(int32_t S, int32_t T) {
  return 4 + (S + 1) + 2 * static_cast<int64_t>(S) + S + T;
}

bool decode_supported(const Params& p, int q_dtype, int kv_dtype, int out_dtype);
int decode_waves(const Params& p, int num_cus);
size_t decode_workspace_bytes(const Params& p);
DecodeWorkspace carve_decode_workspace(const Params& p, void* base);

// Decode rows: stream-K split MFMA decode; writes the outputs of pairs one
// wavefront finishes and partials of the others, and the decode rows' new
// tokens into the cache.
hipError_t launch_decode(const Params& p, int kv_dtype, int out_dtype, const DecodeWorkspace& ws,
                         const void* q, const void* k, const void* v, void* cache,
                         const int32_t* kv_lens, const int32_t* page_indices, const int32_t* cu,
                         const int32_t* dist, void* out, hipStream_t stream);

// Prefill kernel: MFMA attention of every row the decode kernel does not
// take (new tokens read from k/v), plus, in finish workgroups appended to its
// grid, the finish kernel's merge and write items (the finish kernel is then
// not launched) -- at padded head_dim <= 128, and in the LDS-DMA kernel (bf16
// KV, head_dim 128 or 256, unpadded).  Otherwise the finish kernel runs after
// it with the merge and write items.
template <int DP>
constexpr bool kPrefillFinishRoles = DP <= 128;
inline bool prefill_dma_path(const Params& p) {
  return p.kv_bytes == 2 && p.D == p.Dp && (p.Dp == 128 || p.Dp == 256);
}
inline bool prefill_has_finish_roles(const Params& p) {
  return p.Dp <= 128 || prefill_dma_path(p);
}
bool prefill_supported(const Params& p, int q_dtype, int kv_dtype, int out_dtype);
int prefill_merge_blocks(const Params& p, int num_cus);
int prefill_write_blocks(const Params& p, int num_cus);
// With the decode kernel on (p.decode_waves > 0) `ws` holds its partials and
// published plan, and a batch without non-decode rows ends the attention
// blocks at once.
hipError_t launch_prefill(const Params& p, int kv_dtype, int out_dtype, const void* q,
                          const void* k, const void* v, void* cache, const int32_t* kv_lens,
                          const int32_t* page_indices, const int32_t* cu, const int32_t* dist,
                          void* out, const DecodeWorkspace& ws, int num_cus,
                          hipStream_t stream);

// Finish kernel: merges the decode partials, writes the new tokens of every
// non-decode row into the cache and, unless p.prefill_on, attends those rows
// too.  With p.decode_waves == 0 every row is a non-decode row.
bool finish_supported(const Params& p, int q_dtype, int kv_dtype, int out_dtype);
int finish_blocks(const Params& p, int num_cus);
hipError_t launch_finish(const Params& p, int kv_dtype, int out_dtype, const DecodeWorkspace& ws,
                         const void* q, const void* k, const void* v, void* cache,
                         const int32_t* kv_lens, const int32_t* page_indices, const int32_t* cu,
                         const int32_t* dist, void* out, int num_cus, hipStream_t stream);

// Shape-generic attention: one wavefront per (token row, q head); reads every
// key from the cache (run after launch_kv_update).
hipError_t launch_attn_generic(const Params& p, int q_dtype, int kv_dtype, int out_dtype,
                               const void* q, const void* kv_cache, const int32_t* kv_lens,
                               const int32_t* page_indices, const int32_t* cu,
                               const int32_t* dist, void* out, hipStream_t stream);

}  // namespace rpa
