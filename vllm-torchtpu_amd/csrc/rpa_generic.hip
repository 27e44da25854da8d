// Shape-generic RPA attention: one wavefront per (token row, q head).
//
// This path covers every shape and dtype combination the library accepts
// (any q-heads-per-kv-head ratio, any head_dim up to 512, f32/bf16/f16/fp8
// KV, f32/bf16/f16 output).  It runs after the KV-page write kernel, so every key is
// read from the cache.  The per-row computation (generic_row) is shared with
// the finish kernel.
#include "rpa_common.h"
#include "rpa_generic_row.h"
#include "rpa_internal.h"

namespace rpa {

namespace {

constexpr int kMaxDp = kGenericMaxDp;

template <typename QT, typename KVT, typename OutS>
__global__ void __launch_bounds__(256)
attn_generic_kernel(Params p, const typename QT::storage* __restrict__ q,
                    const typename KVT::storage* __restrict__ cache,
                    const int32_t* __restrict__ kv_lens, const int32_t* __restrict__ page_indices,
                    const int32_t* __restrict__ cu, const int32_t* __restrict__ distribution,
                    OutS* __restrict__ out) {
  __shared__ float qs[4][kMaxDp];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t w = static_cast<int64_t>(blockIdx.x) * 4 + wave;
  const int32_t num_seqs = num_seqs_of(distribution, p.S);

  // Identify the row; invalid waves still take part in the barrier below.
  int32_t t = static_cast<int32_t>(w / p.Hq);
  const int32_t g = static_cast<int32_t>(w - static_cast<int64_t>(t) * p.Hq);
  bool valid = t < p.T && num_seqs > 0 && t < cu[num_seqs];
  int32_t s = -1;
  if (valid) {
    s = find_seq(cu, num_seqs + 1, t);
    valid = s >= 0 && s < num_seqs;
  }
  if (valid) {
    const typename QT::storage* qrow = q + (static_cast<int64_t>(t) * p.Hq + g) * p.D;
    for (int d = lane; d < p.Dp; d += 64) qs[wave][d] = d < p.D ? QT::load(qrow, d) : 0.0f;
  }
  __syncthreads();
  if (!valid) return;

  const int32_t q_start = cu[s];
  const int32_t q_len = cu[s + 1] - q_start;
  const int32_t kv_len = min(kv_lens[s], p.pps * p.ps);
  generic_row<KVT, OutS>(p, qs[wave], cache, nullptr, nullptr, false, page_indices, s, t, g,
                         q_start, q_len, kv_len, out);
}

template <typename QT, typename KVT, typename OutS>
hipError_t launch3(const Params& p, const void* q, const void* cache, const int32_t* kv_lens,
                   const int32_t* page_indices, const int32_t* cu, const int32_t* dist,
                   void* out, hipStream_t stream) {
  const int64_t waves = static_cast<int64_t>(p.T) * p.Hq;
  if (waves <= 0) return hipSuccess;
  const int64_t blocks = (waves + 3) / 4;
  if (blocks > 0x7fffffffLL) return hipErrorInvalidValue;
  hipLaunchKernelGGL((attn_generic_kernel<QT, KVT, OutS>), dim3(static_cast<uint32_t>(blocks)),
                     dim3(256), 0, stream, p, static_cast<const typename QT::storage*>(q),
                     static_cast<const typename KVT::storage*>(cache), kv_lens, page_indices, cu,
                     dist, static_cast<OutS*>(out));
  return hipGetLastError();
}

template <typename QT, typename OutS>
hipError_t dispatch_kv(const Params& p, int kv_dtype, const void* q, const void* cache,
                       const int32_t* kv_lens, const int32_t* page_indices, const int32_t* cu,
                       const int32_t* dist, void* out, hipStream_t stream) {
  switch (kv_dtype) {
    case RPA_DTYPE_F32:
      return launch3<QT, TF32, OutS>(p, q, cache, kv_lens, page_indices, cu, dist, out, stream);
    case RPA_DTYPE_BF16:
      return launch3<QT, TBF16, OutS>(p, q, cache, kv_lens, page_indices, cu, dist, out, stream);
    case RPA_DTYPE_F16:
      return launch3<QT, TF16, OutS>(p, q, cache, kv_lens, page_indices, cu, dist, out, stream);
    case RPA_DTYPE_FP8_E4M3FN:
      return launch3<QT, TE4M3, OutS>(p, q, cache, kv_lens, page_indices, cu, dist, out, stream);
    case RPA_DTYPE_FP8_E5M2:
      return launch3<QT, TE5M2, OutS>(p, q, cache, kv_lens, page_indices, cu, dist, out, stream);
    default:
      return hipErrorInvalidValue;
  }
}

template <typename OutS>
hipError_t dispatch_q(const Params& p, int q_dtype, int kv_dtype, const void* q,
                      const void* cache, const int32_t* kv_lens, const int32_t* page_indices,
                      const int32_t* cu, const int32_t* dist, void* out, hipStream_t stream) {
  switch (q_dtype) {
    case RPA_DTYPE_F32:
      return dispatch_kv<TF32, OutS>(p, kv_dtype, q, cache, kv_lens, page_indices, cu, dist, out, stream);
    case RPA_DTYPE_BF16:
      return dispatch_kv<TBF16, OutS>(p, kv_dtype, q, cache, kv_lens, page_indices, cu, dist, out, stream);
    case RPA_DTYPE_F16:
      return dispatch_kv<TF16, OutS>(p, kv_dtype, q, cache, kv_lens, page_indices, cu, dist, out, stream);
    case RPA_DTYPE_FP8_E4M3FN:
      return launch3<TE4M3, TE4M3, OutS>(p, q, cache, kv_lens, page_indices, cu, dist, out, stream);
    case RPA_DTYPE_FP8_E5M2:
      return launch3<TE5M2, TE5M2, OutS>(p, q, cache, kv_lens, page_indices, cu, dist, out, stream);
    default:
      return hipErrorInvalidValue;
  }
}

}  // namespace

hipError_t launch_attn_generic(const Params& p, int q_dtype, int kv_dtype, int out_dtype,
                               const void* q, const void* kv_cache, const int32_t* kv_lens,
                               const int32_t* page_indices, const int32_t* cu,
                               const int32_t* dist, void* out, hipStream_t stream) {
  if (p.Dp > kMaxDp) return hipErrorInvalidValue;
  if (out_dtype == RPA_DTYPE_F32)
    return dispatch_q<float>(p, q_dtype, kv_dtype, q, kv_cache, kv_lens, page_indices, cu, dist, out, stream);
  if (out_dtype == RPA_DTYPE_BF16)
    return dispatch_q<uint16_t>(p, q_dtype, kv_dtype, q, kv_cache, kv_lens, page_indices, cu, dist, out, stream);
  if (out_dtype == RPA_DTYPE_F16)
    return dispatch_q<_Float16>(p, q_dtype, kv_dtype, q, kv_cache, kv_lens, page_indices, cu, dist, out, stream);
  return hipErrorInvalidValue;
}

}  // namespace rpa
