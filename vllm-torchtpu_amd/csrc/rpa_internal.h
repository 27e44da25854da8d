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

// Largest max_num_seqs the decode kernel's in-LDS work plan accepts, and the
// largest kv head count its fixed counter region holds.
constexpr int kMaxDecodeSeqs = 2048;
constexpr int kMaxDecodeHeads = 128;

// Slices of the caller's workspace used by the decode path.  `counters` (a
// fixed-size region at the start of the workspace) must be zero when a call
// starts; the decode kernel leaves it zero again.
struct DecodeWorkspace {
  int32_t* counters;  // [max_num_seqs * Hkv] partial arrival counters
  float* part_o;      // [max_units * Hkv][rows][Dp] un-normalised partial outputs
  float* part_ml;     // [max_units * Hkv][rows][2] (row max in log2 units, row sum)
  int32_t max_units;  // capacity in (sequence, unit) pairs
};

bool decode_supported(const Params& p, int q_dtype, int kv_dtype, int out_dtype);
int decode_grid(const Params& p, int num_cus);
size_t decode_workspace_bytes(const Params& p, int kv_bytes);
DecodeWorkspace carve_decode_workspace(const Params& p, void* base, int kv_bytes);

// Single-token rows: balanced split-K MFMA decode with in-kernel merge.
hipError_t launch_decode(const Params& p, int q_dtype, int kv_dtype, int out_dtype,
                         const DecodeWorkspace& ws, const void* q, const void* cache,
                         const int32_t* kv_lens, const int32_t* page_indices, const int32_t* cu,
                         const int32_t* dist, void* out, int num_cus, hipStream_t stream);

// Shape-generic attention: one wavefront per (token row, q head).
hipError_t launch_attn_generic(const Params& p, int q_dtype, int kv_dtype, int out_dtype,
                               const void* q, const void* kv_cache, const int32_t* kv_lens,
                               const int32_t* page_indices, const int32_t* cu,
                               const int32_t* dist, void* out, hipStream_t stream);

}  // namespace rpa
