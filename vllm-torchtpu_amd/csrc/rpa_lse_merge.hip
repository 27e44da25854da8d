// LSE-weighted merge of R partial attentions of the same rows (the combine
// step of context-parallel decoding).
//
// Restates merge_attn_results (layers/adapter/cp_attention.py:45-72) for R
// partials instead of two: for each row (token, head)
//   m      = max_r lse_r (NaN if any lse_r is NaN, as torch.maximum);
//            m_safe = m if finite else 0
//   e_r    = exp(lse_r - m_safe);  norm = sum_r e_r
//   out    = sum_r e_r * clean(out_r) / (norm if norm > 0 else 1)
//   lse    = m + log(norm if norm > 0 else 1) if m is finite, else m
// where clean() maps NaN and +-inf to 0 (torch.nan_to_num(..., 0, 0, 0)).
// For R = 2 this is the reference function exactly.  The partials are
// stacked: outs [R, rows, D] (bf16 or f32), lses [R, rows] f32.  The
// reference's out is f32 (the f32 weights promote bf16 partials); a bf16 out
// is offered for callers that want the partials' dtype back.
//
// One wavefront per row: lane r < R holds lse_r for the reductions, and each
// lane owns head dims {lane, lane + 64, ...} of the weighted sum.
#include "rpa.h"
#include "rpa_common.h"
#include "rpa_internal.h"

namespace rpa {

namespace {

constexpr int kMergeThreads = 256;
constexpr int kMergeMaxDim = 512;

template <typename T>
__device__ __forceinline__ float load_val(const T* p, int64_t i);
template <>
__device__ __forceinline__ float load_val<float>(const float* p, int64_t i) { return p[i]; }
template <>
__device__ __forceinline__ float load_val<uint16_t>(const uint16_t* p, int64_t i) {
  return bf16_bits_to_f32(p[i]);
}

// max that propagates NaN (torch.maximum), unlike fmaxf.
__device__ __forceinline__ float nan_max(float a, float b) {
  return (a != a || b != b) ? __builtin_nanf("") : fmaxf(a, b);
}

template <typename T, typename TO>
__global__ void __launch_bounds__(kMergeThreads)
lse_merge_kernel(int32_t parts, int64_t rows, int32_t dim, const T* __restrict__ outs,
                 const float* __restrict__ lses, TO* __restrict__ out, float* __restrict__ lse_out) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * (kMergeThreads / 64) + (threadIdx.x >> 6);
  if (row >= rows) return;
  // Row max of the LSEs (lanes past R hold -inf).
  float m = -INFINITY;
  for (int32_t r = lane; r < parts; r += 64) m = nan_max(m, lses[static_cast<int64_t>(r) * rows + row]);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) m = nan_max(m, __shfl_xor(m, o, 64));
  const bool finite = isfinite(m);
  const float m_safe = finite ? m : 0.0f;
  float norm = 0.0f;
  for (int32_t r = lane; r < parts; r += 64)
    norm += expf(lses[static_cast<int64_t>(r) * rows + row] - m_safe);
  norm = warp_sum(norm);
  const float norm_safe = norm > 0.0f ? norm : 1.0f;
  float acc[kMergeMaxDim / 64];
#pragma unroll
  for (int c = 0; c < kMergeMaxDim / 64; ++c) acc[c] = 0.0f;
  for (int32_t r = 0; r < parts; ++r) {
    const float e = expf(lses[static_cast<int64_t>(r) * rows + row] - m_safe);
    const T* src = outs + (static_cast<int64_t>(r) * rows + row) * dim;
#pragma unroll
    for (int c = 0; c < kMergeMaxDim / 64; ++c) {
      const int d = lane + 64 * c;
      if (d < dim) {
        float v = load_val<T>(src, d);
        if (!isfinite(v)) v = 0.0f;
        acc[c] += e * v;
      }
    }
  }
  TO* dst = out + row * dim;
#pragma unroll
  for (int c = 0; c < kMergeMaxDim / 64; ++c) {
    const int d = lane + 64 * c;
    if (d < dim) store_out(dst, d, acc[c] / norm_safe);
  }
  if (lse_out != nullptr && lane == 0) lse_out[row] = finite ? m + logf(norm_safe) : m;
}

}  // namespace

}  // namespace rpa

extern "C" int rpa_merge_attn_states(int32_t num_parts, int64_t rows, int32_t head_dim,
                                     int32_t dtype, int32_t out_dtype, const void* outs,
                                     const float* lses, void* out, float* lse_out,
                                     void* stream) {
  if (num_parts <= 0 || rows < 0 || head_dim <= 0) return RPA_ERR_INVALID_ARG;
  if (head_dim > rpa::kMergeMaxDim) return RPA_ERR_UNSUPPORTED;
  if (dtype != RPA_DTYPE_BF16 && dtype != RPA_DTYPE_F32) return RPA_ERR_UNSUPPORTED;
  if (out_dtype != RPA_DTYPE_BF16 && out_dtype != RPA_DTYPE_F32) return RPA_ERR_UNSUPPORTED;
  if (rows == 0) return RPA_OK;
  if (outs == nullptr || lses == nullptr || out == nullptr) return RPA_ERR_NULL_PTR;
  const int64_t blocks = (rows + rpa::kMergeThreads / 64 - 1) / (rpa::kMergeThreads / 64);
  if (blocks > 0x7fffffff) return RPA_ERR_INVALID_ARG;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<uint32_t>(blocks)), block(rpa::kMergeThreads);
#define RPA_MERGE_LAUNCH(TI, TOUT)                                                             \
  hipLaunchKernelGGL((rpa::lse_merge_kernel<TI, TOUT>), grid, block, 0, s, num_parts, rows,     \
                     head_dim, static_cast<const TI*>(outs), lses, static_cast<TOUT*>(out),     \
                     lse_out)
  if (dtype == RPA_DTYPE_F32 && out_dtype == RPA_DTYPE_F32) RPA_MERGE_LAUNCH(float, float);
  else if (dtype == RPA_DTYPE_F32) RPA_MERGE_LAUNCH(float, uint16_t);
  else if (out_dtype == RPA_DTYPE_F32) RPA_MERGE_LAUNCH(uint16_t, float);
  else RPA_MERGE_LAUNCH(uint16_t, uint16_t);
#undef RPA_MERGE_LAUNCH
  return hipGetLastError() == hipSuccess ? RPA_OK : RPA_ERR_LAUNCH;
}
