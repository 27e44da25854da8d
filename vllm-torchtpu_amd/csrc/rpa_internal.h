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

// Shape-generic attention: one wavefront per (token row, q head).
hipError_t launch_attn_generic(const Params& p, int q_dtype, int kv_dtype, int out_dtype,
                               const void* q, const void* kv_cache, const int32_t* kv_lens,
                               const int32_t* page_indices, const int32_t* cu,
                               const int32_t* dist, void* out, hipStream_t stream);

}  // namespace rpa
