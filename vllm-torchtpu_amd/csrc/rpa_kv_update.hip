// KV-page write: scatter the new tokens' K/V records into their cache pages.
//
// Reference semantics: kernel.py:154-166 (ref) and the fused write of the
// Pallas kernel, kernel.py:652-715.  One workgroup per token row t of the
// k/v inputs; the owning sequence is found by binary search over cu_q_lens,
// so the launch needs no host-side knowledge of the metadata values.
//
// The record for token t is merge_kv(k, v)[t] (kernel.py:1140-1168): combined
// head c = 2h holds K_h, c = 2h + 1 holds V_h, heads >= 2*Hkv and dims >= D
// are zero.  When D == Dp the copy is done in 16-byte chunks; the payload is
// moved as raw bits, so NaN payloads and signed zeros are preserved.
#include "rpa_common.h"
#include "rpa_internal.h"

namespace rpa {

namespace {

// Returns the destination record offset (in elements) for token t, or -1 if
// the token is padding or its metadata points outside the cache.
__device__ __forceinline__ int64_t record_offset(const Params& p, const int32_t* kv_lens,
                                                 const int32_t* page_indices,
                                                 const int32_t* cu, int32_t num_seqs,
                                                 int32_t t) {
  const int32_t s = find_seq(cu, num_seqs + 1, t);
  if (s < 0 || s >= num_seqs) return -1;
  const int32_t q_start = cu[s];
  const int32_t q_len = cu[s + 1] - q_start;
  if (t >= q_start + q_len) return -1;
  const int32_t kv_len = kv_lens[s];
  const int32_t j = kv_len - q_len + (t - q_start);
  if (j < 0 || j >= p.pps * p.ps) return -1;
  const int32_t page = page_indices[static_cast<int64_t>(s) * p.pps + j / p.ps];
  if (page < 0 || page >= p.P) return -1;
  return (static_cast<int64_t>(page) * p.ps + (j % p.ps)) * p.rec;
}

// Generic element copy: Elem is the raw storage type (uint8/uint16/uint32).
template <typename Elem>
__global__ void __launch_bounds__(256)
kv_update_kernel(Params p, const Elem* __restrict__ keys, const Elem* __restrict__ values,
                 Elem* __restrict__ cache, const int32_t* __restrict__ kv_lens,
                 const int32_t* __restrict__ page_indices, const int32_t* __restrict__ cu,
                 const int32_t* __restrict__ distribution) {
  const int32_t num_seqs = num_seqs_of(distribution, p.S);
  const int32_t t = blockIdx.x;
  const int64_t dst = record_offset(p, kv_lens, page_indices, cu, num_seqs, t);
  if (dst < 0) return;
  const int64_t src_row = static_cast<int64_t>(t) * p.Hkv * p.D;
  for (int64_t idx = threadIdx.x; idx < p.rec; idx += blockDim.x) {
    const int32_t c = static_cast<int32_t>(idx / p.Dp);
    const int32_t d = static_cast<int32_t>(idx - static_cast<int64_t>(c) * p.Dp);
    Elem val = 0;
    if (c < 2 * p.Hkv && d < p.D) {
      const Elem* src = (c & 1) ? values : keys;
      val = src[src_row + static_cast<int64_t>(c >> 1) * p.D + d];
    }
    cache[dst + idx] = val;
  }
}

// Vector copy when D == Dp (no dim padding): 16-byte chunks.  Dp*sizeof(Elem)
// is a multiple of 128 bytes, so a chunk never straddles two heads.
template <typename Elem>
__global__ void __launch_bounds__(256)
kv_update_vec_kernel(Params p, const Elem* __restrict__ keys, const Elem* __restrict__ values,
                     Elem* __restrict__ cache, const int32_t* __restrict__ kv_lens,
                     const int32_t* __restrict__ page_indices, const int32_t* __restrict__ cu,
                     const int32_t* __restrict__ distribution) {
  constexpr int kPer = 16 / sizeof(Elem);
  const int32_t num_seqs = num_seqs_of(distribution, p.S);
  const int32_t t = blockIdx.x;
  const int64_t dst = record_offset(p, kv_lens, page_indices, cu, num_seqs, t);
  if (dst < 0) return;
  const int64_t src_row = static_cast<int64_t>(t) * p.Hkv * p.D;
  const int32_t chunks_per_head = p.Dp / kPer;
  const int32_t nchunks = p.Kx2 * chunks_per_head;
  uint4* out = reinterpret_cast<uint4*>(cache + dst);
  for (int32_t i = threadIdx.x; i < nchunks; i += blockDim.x) {
    const int32_t c = i / chunks_per_head;
    const int32_t d = (i - c * chunks_per_head) * kPer;
    uint4 val = make_uint4(0u, 0u, 0u, 0u);
    if (c < 2 * p.Hkv) {
      const Elem* src = ((c & 1) ? values : keys) + src_row + static_cast<int64_t>(c >> 1) * p.D + d;
      val = *reinterpret_cast<const uint4*>(src);
    }
    out[i] = val;
  }
}

template <typename Elem>
hipError_t launch_typed(const Params& p, const void* k, const void* v, void* cache,
                        const int32_t* kv_lens, const int32_t* page_indices,
                        const int32_t* cu, const int32_t* dist, hipStream_t stream,
                        bool vec_ok) {
  if (p.T <= 0) return hipSuccess;
  dim3 grid(p.T), block(256);
  if (vec_ok) {
    hipLaunchKernelGGL(kv_update_vec_kernel<Elem>, grid, block, 0, stream, p,
                       static_cast<const Elem*>(k), static_cast<const Elem*>(v),
                       static_cast<Elem*>(cache), kv_lens, page_indices, cu, dist);
  } else {
    hipLaunchKernelGGL(kv_update_kernel<Elem>, grid, block, 0, stream, p,
                       static_cast<const Elem*>(k), static_cast<const Elem*>(v),
                       static_cast<Elem*>(cache), kv_lens, page_indices, cu, dist);
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_kv_update(const Params& p, int elem_bytes, const void* k, const void* v,
                            void* cache, const int32_t* kv_lens, const int32_t* page_indices,
                            const int32_t* cu, const int32_t* dist, hipStream_t stream) {
  // 16-byte chunks need D == Dp and 16-byte aligned rows in every tensor.
  const bool aligned = ((reinterpret_cast<uintptr_t>(k) | reinterpret_cast<uintptr_t>(v) |
                         reinterpret_cast<uintptr_t>(cache)) & 15u) == 0;
  const bool vec_ok = aligned && p.D == p.Dp && (static_cast<int64_t>(p.D) * elem_bytes) % 16 == 0;
  switch (elem_bytes) {
    case 1: return launch_typed<uint8_t>(p, k, v, cache, kv_lens, page_indices, cu, dist, stream, vec_ok);
    case 2: return launch_typed<uint16_t>(p, k, v, cache, kv_lens, page_indices, cu, dist, stream, vec_ok);
    case 4: return launch_typed<uint32_t>(p, k, v, cache, kv_lens, page_indices, cu, dist, stream, vec_ok);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace rpa
