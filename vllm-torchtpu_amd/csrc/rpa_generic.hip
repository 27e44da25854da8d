// Shape-generic RPA attention: one wavefront per (token row, q head).
//
// This path covers every shape and dtype combination the library accepts
// (any q-heads-per-kv-head ratio, any head_dim up to 512, f32/bf16/fp8 KV,
// f32/bf16 output).  The specialised decode and prefill kernels take the
// common shapes; this one is the general case.
//
// Semantics follow ref_ragged_paged_attention (kernel.py:74-214): for q row i
// of sequence s at logical position p = kv_len - q_len + i and q head g,
//   s_j = (q_g . k_{g/qpk, j}) * sm_scale * k_scale * q_scale,
//   s_j = cap * tanh(s_j / cap)                 (soft cap, kernel.py:193-194)
//   keys with j > p, or j <= p - W under a window, are excluded
//   (causal mask kernel.py:196-204)
//   out = softmax(s) . v * v_scale               (kernel.py:205-209)
// Masked keys get weight exactly 0 (mask_value = finfo.min underflows).
//
// Work split inside a wavefront: lane j scores key (k0 + j) of a 64-key tile
// against the q row held in LDS, the wavefront reduces max/sum with
// shuffles, and for P.V each lane owns head dims {lane, lane + 64, ...}.
#include "rpa_common.h"
#include "rpa_internal.h"

namespace rpa {

namespace {

constexpr int kMaxDp = 512;
constexpr int kMaxChunks = kMaxDp / 64;

template <typename KVT>
__device__ __forceinline__ float kv_elem(const typename KVT::storage* base, int d) {
  return KVT::load(base, d);
}

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
  // Rows the decode path owns (same predicate as its work plan).
  if (p.skip_decode_rows && q_len == 1 && kv_len >= 1 && q_start >= 0 && q_start < p.T) return;
  const int32_t pos = kv_len - q_len + (t - q_start);
  int32_t hi = kv_len, lo = 0;
  if (p.causal) {
    hi = min(kv_len, pos + 1);
    if (p.window > 0) lo = max(0, pos - p.window + 1);
  }
  const int32_t h = g / p.qpk;
  const int64_t k_off = static_cast<int64_t>(2 * h) * p.Dp;
  const int64_t v_off = k_off + p.Dp;
  const int32_t* ptab = page_indices + static_cast<int64_t>(s) * p.pps;

  float m_run = -INFINITY, l_run = 0.0f;
  float acc[kMaxChunks];
#pragma unroll
  for (int c = 0; c < kMaxChunks; ++c) acc[c] = 0.0f;

  for (int32_t k0 = lo; k0 < hi; k0 += 64) {
    const int32_t j = k0 + lane;
    const bool kvalid = j < hi;
    int64_t rec_base = 0;
    float sc = -INFINITY;
    if (kvalid) {
      int32_t page = ptab[j / p.ps];
      page = min(max(page, 0), p.P - 1);
      rec_base = (static_cast<int64_t>(page) * p.ps + (j % p.ps)) * p.rec;
      const typename KVT::storage* krow = cache + rec_base + k_off;
      float dot = 0.0f;
      for (int d = 0; d < p.D; ++d) dot += qs[wave][d] * kv_elem<KVT>(krow, d);
      sc = dot * p.score_scale;
      if (p.has_cap) sc = soft_cap_fn(sc, p.cap, p.inv_cap);
    }
    const float m_tile = warp_max(sc);
    const float m_new = fmaxf(m_run, m_tile);
    if (m_new == -INFINITY) continue;  // wave-uniform: no valid key yet
    const float alpha = __expf(m_run - m_new);
    const float pj = kvalid ? __expf(sc - m_new) : 0.0f;
    l_run = l_run * alpha + warp_sum(pj);
    m_run = m_new;
#pragma unroll
    for (int c = 0; c < kMaxChunks; ++c) acc[c] *= alpha;
    const int nkeys = min(64, hi - k0);
    for (int jj = 0; jj < nkeys; ++jj) {
      const float pw = __shfl(pj, jj, 64);
      const int64_t vb = __shfl(rec_base, jj, 64);
      const typename KVT::storage* vrow = cache + vb + v_off;
#pragma unroll
      for (int c = 0; c < kMaxChunks; ++c) {
        const int d = lane + 64 * c;
        if (d < p.D) acc[c] += pw * kv_elem<KVT>(vrow, d);
      }
    }
  }

  const float inv_l = (l_run == 0.0f) ? 0.0f : p.v_scale / l_run;
  OutS* orow = out + (static_cast<int64_t>(t) * p.Hq + g) * p.D;
#pragma unroll
  for (int c = 0; c < kMaxChunks; ++c) {
    const int d = lane + 64 * c;
    if (d < p.D) store_out(orow, d, acc[c] * inv_l);
  }
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
  return hipErrorInvalidValue;
}

}  // namespace rpa
