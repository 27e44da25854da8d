// Finish kernel: everything of a call that the decode kernel does not do.
//
// Launched right after the decode kernel on the same stream (or alone, when
// the decode kernel does not apply).  A persistent grid walks three kinds of
// items in grid-stride order:
//   merge   (decode sequence s, kv head h) with more than one unit: combine
//           the unit partials (m, l, O) the decode kernel wrote -- the
//           split-K form of the online softmax, out = sum_k 2^(m_k - M) O_k /
//           sum_k 2^(m_k - M) l_k * v_scale.  The kernel boundary makes the
//           partials visible; nothing waits on another wavefront.
//   write   token row t of a non-decode sequence: its new K/V record into
//           its cache page (kernel.py:154-166), unless skip_kv_update.
//   attend  (token row t, q head g) of a non-decode sequence: generic_row
//           attention, reading this call's new tokens from the k/v inputs
//           (the write items of the same launch may not have run yet).
// Every workgroup first derives the decode kernel's plan (rpa_plan.h) from
// the device-resident metadata.
#include "rpa_common.h"
#include "rpa_generic_row.h"
#include "rpa_internal.h"
#include "rpa_plan.h"

namespace rpa {

namespace {

constexpr int kWaves = kPlanWaves;
constexpr int kThreads = kPlanThreads;

// Merge the `nunits` partials of one (sequence, kv head) and write its output
// rows [0, rows).  The partial of unit k sits in slot first + k * Hkv: RP rows
// x DP floats of un-normalised O, and RP (m, l) pairs (log2 units).  One
// wavefront; lane e of load j covers element e + 64 j of a slot, so every
// load is a wave-wide contiguous 256-byte read and row (j * 64 / DP) is the
// same for the whole wavefront.  Loads are batched over UB units so that a
// merge costs a few memory round trips.  A NaN partial sum propagates.
__device__ __forceinline__ void ml_combine(float& M, float& L, float m, float l) {
  const float mn = fmaxf(M, m);
  const float a = (M == -INFINITY) ? 0.0f : exp2f(M - mn);
  const float b = (m == -INFINITY) ? 0.0f : exp2f(m - mn);
  L = L * a + l * b;
  M = mn;
}

template <int DP, int RP, typename OutS>
__device__ __forceinline__ void merge_partials(const Params& p, const float* __restrict__ part_o,
                                               const float* __restrict__ part_ml, int32_t first,
                                               int32_t nunits, int32_t rows,
                                               OutS* __restrict__ out, int64_t orow0) {
  constexpr int NDW = RP * DP / 64;             // dwords per lane per slot
  constexpr int UB = NDW >= 64 ? 1 : 64 / NDW;  // slots per load batch
  const int lane = threadIdx.x & 63;
  const int64_t stride = static_cast<int64_t>(p.Hkv);

  float M[RP], L[RP];
#pragma unroll
  for (int r = 0; r < RP; ++r) {
    M[r] = -INFINITY;
    L[r] = 0.0f;
  }
  for (int32_t k = lane; k < nunits; k += 64) {
    const float2* ml = reinterpret_cast<const float2*>(part_ml + (first + k * stride) * (2 * RP));
    float2 v[RP];
#pragma unroll
    for (int r = 0; r < RP; ++r) v[r] = ml[r];
#pragma unroll
    for (int r = 0; r < RP; ++r) ml_combine(M[r], L[r], v[r].x, v[r].y);
  }
#pragma unroll
  for (int r = 0; r < RP; ++r) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const float mo = __shfl_xor(M[r], o, 64);
      const float lo = __shfl_xor(L[r], o, 64);
      ml_combine(M[r], L[r], mo, lo);
    }
  }
  float scale[RP];
#pragma unroll
  for (int r = 0; r < RP; ++r) scale[r] = (L[r] == 0.0f) ? 0.0f : p.v_scale / L[r];

  float acc[NDW];
#pragma unroll
  for (int j = 0; j < NDW; ++j) acc[j] = 0.0f;
  for (int32_t k0 = 0; k0 < nunits; k0 += 64) {
    const int32_t kn = min(64, nunits - k0);
    // Weight of unit k0 + lane for every row (0 for lanes past the end).
    float w[RP];
    {
      const int32_t k = k0 + min(lane, kn - 1);
      const float* ml = part_ml + (first + k * stride) * (2 * RP);
#pragma unroll
      for (int r = 0; r < RP; ++r) {
        const float m = ml[2 * r];
        w[r] = (lane >= kn || m == -INFINITY) ? 0.0f : exp2f(m - M[r]) * scale[r];
      }
    }
    for (int32_t kb = 0; kb < kn; kb += UB) {
      float v[UB][NDW];
#pragma unroll
      for (int u = 0; u < UB; ++u) {
        const int32_t k = k0 + min(kb + u, kn - 1);  // in-bounds; weight 0 past kn
        const float* po = part_o + (first + k * stride) * (RP * DP) + lane;
#pragma unroll
        for (int j = 0; j < NDW; ++j) v[u][j] = po[64 * j];
      }
#pragma unroll
      for (int u = 0; u < UB; ++u) {
        const int src = min(kb + u, 63);
        const bool live = kb + u < kn;
#pragma unroll
        for (int j = 0; j < NDW; ++j) {
          const float wr = live ? __shfl(w[j * 64 / DP], src, 64) : 0.0f;
          acc[j] += wr * v[u][j];
        }
      }
    }
  }
#pragma unroll
  for (int j = 0; j < NDW; ++j) {
    const int r = j * 64 / DP;
    const int d = lane + 64 * (j % (DP / 64));
    if (r < rows && d < p.D) store_out(out, (orow0 + r) * p.D + d, acc[j]);
  }
}

// New K/V record of token row t (logical position j of sequence s) into its
// cache page: merge_kv(k, v)[t] (kernel.py:1140-1168) -- combined head 2h is
// K_h, 2h + 1 is V_h, heads >= 2 Hkv and dims >= D are zero.  Bits are
// copied as they are.  8-byte pieces (D * element bytes is a multiple of 8).
template <typename E>
__device__ __forceinline__ void write_record(const Params& p, E* __restrict__ cache,
                                             const int32_t* __restrict__ page_indices,
                                             const E* __restrict__ keys,
                                             const E* __restrict__ values, int32_t s, int32_t j,
                                             int32_t t, int lane) {
  constexpr int EPP = 8 / sizeof(E);
  const int32_t pg = page_indices[static_cast<int64_t>(s) * p.pps + j / p.ps];
  if (pg < 0 || pg >= p.P) return;
  E* rec = cache + (static_cast<int64_t>(pg) * p.ps + j % p.ps) * p.rec;
  const int64_t src_row = static_cast<int64_t>(t) * p.Hkv * p.D;
  const int32_t per_head = p.Dp / EPP;
  const int32_t pieces = p.Kx2 * per_head;
  for (int32_t i = lane; i < pieces; i += 64) {
    const int32_t c = i / per_head;
    const int32_t e0 = (i - c * per_head) * EPP;
    uint2 v = make_uint2(0u, 0u);
    if (c < 2 * p.Hkv && e0 < p.D)
      v = *reinterpret_cast<const uint2*>(((c & 1) ? values : keys) + src_row +
                                          static_cast<int64_t>(c >> 1) * p.D + e0);
    *reinterpret_cast<uint2*>(rec + static_cast<int64_t>(c) * p.Dp + e0) = v;
  }
}

template <typename KVT, int DP, typename OutS>
__global__ void __launch_bounds__(kThreads)
finish_kernel(Params p, const uint16_t* __restrict__ q, const typename KVT::storage* __restrict__ keys,
              const typename KVT::storage* __restrict__ values,
              typename KVT::storage* __restrict__ cache, const int32_t* __restrict__ kv_lens,
              const int32_t* __restrict__ page_indices, const int32_t* __restrict__ cu,
              const int32_t* __restrict__ dist, OutS* __restrict__ out,
              const float* __restrict__ part_o, const float* __restrict__ part_ml,
              int32_t max_units) {
  using E = typename KVT::storage;
  __shared__ PlanLds L;
  __shared__ float qs[kWaves][DP];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const bool decode_on = p.decode_waves > 0;
  const Plan pl = build_plan(p, kv_lens, cu, dist, decode_tile_tokens(DP, sizeof(E)), max_units,
                             decode_on, L);
  const int32_t n = pl.num_seqs;
  const int32_t nrows = max(0, min(L.cu[n], p.T));
  const int32_t nmerge = decode_on ? n * p.Hkv : 0;
  const int32_t nwrite = p.skip_kv_update ? 0 : nrows;
  const int64_t total = static_cast<int64_t>(nmerge) + nwrite + static_cast<int64_t>(nrows) * p.Hq;
  const int32_t rows = min(p.qpk, 16);
  const int32_t rp = decode_slot_rows(p.qpk);

  const int64_t gw = static_cast<int64_t>(blockIdx.x) * kWaves + wave;
  const int64_t nw = static_cast<int64_t>(gridDim.x) * kWaves;
  for (int64_t it = gw; it < total; it += nw) {
    if (it < nmerge) {
      const int32_t s = static_cast<int32_t>(it / p.Hkv);
      const int32_t h = static_cast<int32_t>(it - static_cast<int64_t>(s) * p.Hkv);
      const int32_t nunits = L.units[s + 1] - L.units[s];
      if (L.nt[s] == 0 || nunits <= 1) continue;
      const int32_t first = L.units[s] * p.Hkv + h;
      const int64_t orow0 = static_cast<int64_t>(L.tq[s]) * p.Hq + h * p.qpk;
      switch (rp) {
        case 1: merge_partials<DP, 1>(p, part_o, part_ml, first, nunits, rows, out, orow0); break;
        case 2: merge_partials<DP, 2>(p, part_o, part_ml, first, nunits, rows, out, orow0); break;
        case 4: merge_partials<DP, 4>(p, part_o, part_ml, first, nunits, rows, out, orow0); break;
        case 8: merge_partials<DP, 8>(p, part_o, part_ml, first, nunits, rows, out, orow0); break;
        default: merge_partials<DP, 16>(p, part_o, part_ml, first, nunits, rows, out, orow0); break;
      }
      continue;
    }
    // Row items: find the sequence of token row t.
    const bool is_write = it < static_cast<int64_t>(nmerge) + nwrite;
    const int64_t a = it - nmerge - (is_write ? 0 : nwrite);
    const int32_t t = static_cast<int32_t>(is_write ? a : a / p.Hq);
    const int32_t s = find_seq(L.cu, n + 1, t);
    if (s < 0 || s >= n || L.nt[s] != 0) continue;  // padding, or a decode row
    const int32_t q_start = L.cu[s];
    const int32_t q_len = L.cu[s + 1] - q_start;
    if (t >= q_start + q_len) continue;
    const int32_t kv_len = L.kvlen[s];
    if (is_write) {
      const int32_t j = kv_len - q_len + (t - q_start);
      if (j >= 0) write_record<E>(p, cache, page_indices, keys, values, s, j, t, lane);
      continue;
    }
    const int32_t g = static_cast<int32_t>(a - static_cast<int64_t>(t) * p.Hq);
    wave_lds_sync();  // the previous item's reads of qs are complete
    const uint16_t* qrow = q + (static_cast<int64_t>(t) * p.Hq + g) * p.D;
    for (int d = lane; d < DP; d += 64) qs[wave][d] = d < p.D ? bf16_bits_to_f32(qrow[d]) : 0.0f;
    wave_lds_sync();
    generic_row<KVT, OutS>(p, qs[wave], cache, keys, values, p.skip_kv_update == 0, page_indices,
                           s, t, g, q_start, q_len, kv_len, out);
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
                     dist, static_cast<OutS*>(out), ws.part_o, ws.part_ml, ws.max_units)
  if (p.Dp == 128) {
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
  if (p.Dp != 128 && p.Dp != 256) return false;
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
