// Finish kernel: everything of a call that the decode kernel does not do.
//
// Launched right after the decode kernel on the same stream (or alone, when
// the decode kernel does not apply).  A persistent grid walks three kinds of
// items in grid-stride order:
//   merge   (decode sequence s, kv head h) cut between several decode
//           wavefronts (rpa_plan.h): combine their partials (m, l, O) --
//           the split-K form of the online softmax, out = sum_k 2^(m_k - M)
//           O_k / sum_k 2^(m_k - M) l_k * v_scale.  The kernel boundary makes
//           the partials visible; nothing waits on another wavefront.
//   write   token row t of a non-decode sequence: its new K/V record into
//           its cache page (kernel.py:154-166), unless skip_kv_update.
//   attend  (token row t, q head g) of a non-decode sequence: generic_row
//           attention, reading this call's new tokens from the k/v inputs
//           (the write items of the same launch may not have run yet); only
//           when the prefill kernel (rpa_prefill.hip) did not run.
// Every workgroup first derives the decode kernel's plan (rpa_plan.h) from
// the device-resident metadata.
#include "rpa_common.h"
#include "rpa_finish_items.h"
#include "rpa_generic_row.h"
#include "rpa_internal.h"
#include "rpa_plan.h"

namespace rpa {

namespace {

constexpr int kWaves = kPlanWaves;
constexpr int kThreads = kPlanThreads;

template <typename KVT, int DP, typename OutS>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2)))
finish_kernel(Params p, const uint16_t* __restrict__ q, const typename KVT::storage* __restrict__ keys,
              const typename KVT::storage* __restrict__ values,
              typename KVT::storage* __restrict__ cache, const int32_t* __restrict__ kv_lens,
              const int32_t* __restrict__ page_indices, const int32_t* __restrict__ cu,
              const int32_t* __restrict__ dist, OutS* __restrict__ out,
              const float* __restrict__ part_o, const float* __restrict__ part_ml,
              const int32_t* __restrict__ plan) {
  using E = typename KVT::storage;
  __shared__ PlanCore L;
  __shared__ PlanRows R;
  __shared__ float qs[kWaves][DP];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  // With the decode kernel, its published plan drives this launch (no
  // workgroup-wide plan here); without it, every workgroup builds one.
  const bool decode_on = p.decode_waves > 0;
  const PlanView pv = plan_view(plan, p.S);
  int32_t n;
  if (decode_on) {
    n = min(max(pv.hdr[0], 0), p.S);
  } else {
    n = build_plan(p, kv_lens, cu, dist, decode_tile_tokens(DP, sizeof(E)), false, L, &R).num_seqs;
  }
  const int32_t nmerge = decode_on ? n * p.Hkv : 0;
  const int32_t nwrite = p.skip_kv_update ? 0 : p.T;
  const int64_t nattend = p.prefill_on ? 0 : static_cast<int64_t>(p.T) * p.Hq;
  const int64_t total = static_cast<int64_t>(nmerge) + nwrite + nattend;

  const int64_t gw = static_cast<int64_t>(blockIdx.x) * kWaves + wave;
  const int64_t nw = static_cast<int64_t>(gridDim.x) * kWaves;
  for (int64_t it = gw; it < total; it += nw) {
    if (it < nmerge) {
      finish_merge_item<DP, OutS>(p, pv, static_cast<int32_t>(it), cu, part_o, part_ml, out);
      continue;
    }
    if (it < static_cast<int64_t>(nmerge) + nwrite) {
      finish_write_item<E>(p, decode_on, pv, &R, n, cu, kv_lens, cache, page_indices, keys,
                           values, static_cast<int32_t>(it - nmerge), lane);
      continue;
    }
    // Attend item (token row t, q head g).
    const int64_t a = it - nmerge - nwrite;
    const int32_t t = static_cast<int32_t>(a / p.Hq);
    const int32_t g = static_cast<int32_t>(a - static_cast<int64_t>(t) * p.Hq);
    RowOwner o;
    if (!row_owner(p, decode_on, pv, &R, n, cu, kv_lens, t, &o)) continue;
    wave_lds_sync();  // the previous item's reads of qs are complete
    const uint16_t* qrow = q + (static_cast<int64_t>(t) * p.Hq + g) * p.D;
    for (int d = lane; d < DP; d += 64) qs[wave][d] = d < p.D ? bf16_bits_to_f32(qrow[d]) : 0.0f;
    wave_lds_sync();
    generic_row<KVT, OutS>(p, qs[wave], cache, keys, values, p.skip_kv_update == 0, page_indices,
                           o.s, t, g, o.q_start, o.q_end - o.q_start, o.kv_len, out);
  }
}

template <typename KVT, typename OutS>
hipError_t launch_dp(const Params& p, const DecodeWorkspace& ws, const void* q, const void* k,
                     const void* v, void* cache, const int32_t* kv_lens,
                     const int32_t* page_indices, const int32_t* cu, const int32_t* dist,
                     void* out, int blocks, hipStream_t stream) {
  using E = typename KVT::storage;
  const dim3 grid(blocks), block(kThreads);
#define RPA_FINISH_LAUNCH(DPV)                                                                    \
  hipLaunchKernelGGL((finish_kernel<KVT, DPV, OutS>), grid, block, 0, stream, p,                  \
                     static_cast<const uint16_t*>(q), static_cast<const E*>(k),                   \
                     static_cast<const E*>(v), static_cast<E*>(cache), kv_lens, page_indices, cu, \
                     dist, static_cast<OutS*>(out), ws.part_o, ws.part_ml, ws.plan)
  if (p.Dp == 64) {
    RPA_FINISH_LAUNCH(64);
  } else if (p.Dp == 128) {
    RPA_FINISH_LAUNCH(128);
  } else if (p.Dp == 256) {
    RPA_FINISH_LAUNCH(256);
  } else {
    return hipErrorInvalidValue;
  }
#undef RPA_FINISH_LAUNCH
  return hipGetLastError();
}

template <typename OutS>
hipError_t launch_kv(const Params& p, int kv_dtype, const DecodeWorkspace& ws, const void* q,
                     const void* k, const void* v, void* cache, const int32_t* kv_lens,
                     const int32_t* page_indices, const int32_t* cu, const int32_t* dist,
                     void* out, int blocks, hipStream_t stream) {
  switch (kv_dtype) {
    case RPA_DTYPE_BF16:
      return launch_dp<TBF16, OutS>(p, ws, q, k, v, cache, kv_lens, page_indices, cu, dist, out, blocks, stream);
    case RPA_DTYPE_FP8_E4M3FN:
      return launch_dp<TE4M3, OutS>(p, ws, q, k, v, cache, kv_lens, page_indices, cu, dist, out, blocks, stream);
    case RPA_DTYPE_FP8_E5M2:
      return launch_dp<TE5M2, OutS>(p, ws, q, k, v, cache, kv_lens, page_indices, cu, dist, out, blocks, stream);
    default:
      return hipErrorInvalidValue;
  }
}

}  // namespace

bool finish_supported(const Params& p, int q_dtype, int kv_dtype, int out_dtype) {
  if (q_dtype != RPA_DTYPE_BF16) return false;
  if (kv_dtype != RPA_DTYPE_BF16 && kv_dtype != RPA_DTYPE_FP8_E4M3FN &&
      kv_dtype != RPA_DTYPE_FP8_E5M2)
    return false;
  if (out_dtype != RPA_DTYPE_BF16 && out_dtype != RPA_DTYPE_F32) return false;
  if (p.Dp != 64 && p.Dp != 128 && p.Dp != 256) return false;
  if (p.D % 8 != 0 || p.S > kMaxDecodeSeqs) return false;
  return true;
}

int finish_blocks(const Params& p, int num_cus) {
  (void)p;
  return 2 * num_cus;
}

hipError_t launch_finish(const Params& p, int kv_dtype, int out_dtype, const DecodeWorkspace& ws,
                         const void* q, const void* k, const void* v, void* cache,
                         const int32_t* kv_lens, const int32_t* page_indices, const int32_t* cu,
                         const int32_t* dist, void* out, int num_cus, hipStream_t stream) {
  const int blocks = finish_blocks(p, num_cus);
  if (out_dtype == RPA_DTYPE_F32)
    return launch_kv<float>(p, kv_dtype, ws, q, k, v, cache, kv_lens, page_indices, cu, dist, out, blocks, stream);
  return launch_kv<uint16_t>(p, kv_dtype, ws, q, k, v, cache, kv_lens, page_indices, cu, dist, out, blocks, stream);
}

}  // namespace rpa
