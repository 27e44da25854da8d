// Shape-generic attention of one (token row, q head): one wavefront.
//
// Semantics follow ref_ragged_paged_attention (kernel.py:74-214): for q row i
// of sequence s at logical position p = kv_len - q_len + i and q head g,
//   s_j = (q_g . k_{g/qpk, j}) * sm_scale * k_scale * q_scale,
//   s_j = cap * tanh(s_j / cap)                 (soft cap, kernel.py:193-194)
//   keys with j > p, or j <= p - W under a window, are excluded
//   (causal mask kernel.py:196-204); without the causal mask, a window with
//   window_nc set excludes j <= p - W alone (kernel_hd64.py:155-158)
//   out = softmax(s) . v * v_scale               (kernel.py:205-209)
// Masked keys get weight exactly 0 (mask_value = finfo.min underflows).
//
// Work split inside the wavefront: lane j scores key (k0 + j) of a 64-key
// tile against the q row held in LDS, the wavefront reduces max/sum with
// shuffles, and for P.V each lane owns head dims {lane, lane + 64, ...}.
#pragma once

#include "rpa_common.h"

namespace rpa {

constexpr int kGenericMaxDp = 512;
constexpr int kGenericMaxChunks = kGenericMaxDp / 64;

// Where key j of the row's sequence lives.  New tokens (j >= kv_len - q_len)
// come from the k/v inputs when `new_from_input` (the cache write of this call
// may not have happened yet); every other key from its cache page.
struct KeySource {
  int64_t k_off;       // element offset of K_h in the cache, or in the k input
  int64_t v_off;       // element offset of V_h in the cache, or in the v input
  int32_t from_input;  // 1: offsets index the k/v inputs
};

template <typename KVT>
__device__ __forceinline__ KeySource key_source(const Params& p, const int32_t* ptab, int32_t h,
                                                int32_t j, int32_t new_start, int32_t q_start,
                                                bool new_from_input) {
  KeySource ks;
  if (new_from_input && j >= new_start) {
    const int64_t row = min(q_start + (j - new_start), p.T - 1);
    ks.k_off = (row * p.Hkv + h) * p.D;
    ks.v_off = ks.k_off;
    ks.from_input = 1;
  } else {
    int32_t page = ptab[page_of(p, j)];
    page = min(max(page, 0), p.P - 1);
    const int64_t rec_base = (static_cast<int64_t>(page) * p.ps + slot_of(p, j)) * p.rec;
    ks.k_off = rec_base + static_cast<int64_t>(2 * h) * p.Dp;
    ks.v_off = ks.k_off + p.Dp;
    ks.from_input = 0;
  }
  return ks;
}

// qs: this wavefront's q row (Dp floats, zero beyond D) in LDS.
template <typename KVT, typename OutS>
__device__ __forceinline__ void generic_row(const Params& p, const float* qs,
                                            const typename KVT::storage* __restrict__ cache,
                                            const typename KVT::storage* __restrict__ keys,
                                            const typename KVT::storage* __restrict__ values,
                                            bool new_from_input, const int32_t* page_indices,
                                            int32_t s, int32_t t, int32_t g, int32_t q_start,
                                            int32_t q_len, int32_t kv_len, OutS* __restrict__ out) {
  using E = typename KVT::storage;
  const int lane = threadIdx.x & 63;
  const int32_t pos = kv_len - q_len + (t - q_start);
  int32_t hi = kv_len, lo = 0;
  if (p.causal) {
    hi = min(kv_len, pos + 1);
    if (p.window > 0) lo = max(0, pos - p.window + 1);
  } else if (p.window_nc) {
    lo = max(0, pos - p.window + 1);  // kernel_hd64.py:155-158: window without causality
  }
  const int32_t h = g / p.qpk;
  const int32_t new_start = kv_len - q_len;
  const int32_t* ptab = page_indices + static_cast<int64_t>(s) * p.pps;

  float m_run = -INFINITY, l_run = 0.0f;
  float acc[kGenericMaxChunks];
#pragma unroll
  for (int c = 0; c < kGenericMaxChunks; ++c) acc[c] = 0.0f;

  for (int32_t k0 = lo; k0 < hi; k0 += 64) {
    const int32_t j = k0 + lane;
    const bool kvalid = j < hi;
    KeySource ks{0, 0, 0};
    float sc = -INFINITY;
    if (kvalid) {
      ks = key_source<KVT>(p, ptab, h, j, new_start, q_start, new_from_input);
      const E* krow = (ks.from_input ? keys : cache) + ks.k_off;
      float dot = 0.0f;
      for (int d = 0; d < p.D; ++d) dot += qs[d] * KVT::load(krow, d);
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
    for (int c = 0; c < kGenericMaxChunks; ++c) acc[c] *= alpha;
    const int nkeys = min(64, hi - k0);
    for (int jj = 0; jj < nkeys; ++jj) {
      const float pw = __shfl(pj, jj, 64);
      const int64_t vo = __shfl(ks.v_off, jj, 64);
      const int32_t fi = __shfl(ks.from_input, jj, 64);
      const E* vrow = (fi ? values : cache) + vo;
#pragma unroll
      for (int c = 0; c < kGenericMaxChunks; ++c) {
        const int d = lane + 64 * c;
        if (d < p.D) acc[c] += pw * KVT::load(vrow, d);
      }
    }
  }

  // The attention sink (a logit with value 0) joins the sum.
  const float l_s = p.sink != nullptr ? l_run + __expf(p.sink[g] - m_run) : l_run;
  const float inv_l = l_s > 0.0f ? p.v_scale / l_s : 0.0f;
  if (p.lse != nullptr && lane == 0)
    p.lse[static_cast<int64_t>(t) * p.Hq + g] = l_run > 0.0f ? m_run + __logf(l_run) : -INFINITY;
  OutS* orow = out + (static_cast<int64_t>(t) * p.Hq + g) * p.D;
#pragma unroll
  for (int c = 0; c < kGenericMaxChunks; ++c) {
    const int d = lane + 64 * c;
    if (d < p.D) store_out(orow, d, acc[c] * inv_l);
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
  if (j < 0 || j >= p.pps * p.ps) return;  // outside the sequence's page table
  const int32_t pg = page_indices[static_cast<int64_t>(s) * p.pps + page_of(p, j)];
  if (pg < 0 || pg >= p.P) return;
  E* rec = cache + (static_cast<int64_t>(pg) * p.ps + slot_of(p, j)) * p.rec;
  const int64_t src_row = static_cast<int64_t>(t) * p.Hkv * p.D;
  const int32_t per_head = p.Dp / EPP;
  const int32_t pieces = p.Kx2 * per_head;
  // Batches of kBatch pieces per lane: all loads, then all stores (one memory
  // round trip per batch instead of one per piece).
  constexpr int kBatch = 8;
  for (int32_t i0 = lane; i0 < pieces; i0 += 64 * kBatch) {
    uint2 v[kBatch];
    int32_t dst[kBatch];
#pragma unroll
    for (int b = 0; b < kBatch; ++b) {
      const int32_t i = i0 + 64 * b;
      const int32_t c = i / per_head;
      const int32_t e0 = (i - c * per_head) * EPP;
      v[b] = make_uint2(0u, 0u);
      dst[b] = i < pieces ? c * p.Dp + e0 : -1;
      if (i < pieces && c < 2 * p.Hkv && e0 < p.D)
        v[b] = *reinterpret_cast<const uint2*>(((c & 1) ? values : keys) + src_row +
                                               static_cast<int64_t>(c >> 1) * p.D + e0);
    }
#pragma unroll
    for (int b = 0; b < kBatch; ++b)
      if (dst[b] >= 0) *reinterpret_cast<uint2*>(rec + dst[b]) = v[b];
  }
}

}  // namespace rpa
