// Split-K merge of decode partials (the finish kernel's merge items).
//
// Each wavefront k that touched a (sequence, kv head) pair left (m_k, l_k, O_k):
// row max of its scores (log2 units), row sum of 2^(s - m_k), and sum of
// 2^(s - m_k) v.  The merged row is out = sum_k 2^(m_k - M) O_k /
// sum_k 2^(m_k - M) l_k * v_scale with M = max_k m_k -- the online-softmax
// recurrence of kernel.py:486-557 applied across key ranges.  The partials
// were written by the previous launch, so plain loads see them.
#pragma once

#include "rpa_common.h"

namespace rpa {

// Merge the `nunits` partials of one (sequence, kv head) and write its output
// rows [0, rows): row r is token tq + r / qpk, q head h * qpk + r % qpk.  Partial k sits in slot first + k: RP rows
// x DP floats of un-normalised O, and RP (m, l) pairs (log2 units).  One
// wavefront; lane e of load j covers element e + 64 j of a slot, so every
// load is a wave-wide contiguous 256-byte read and row (j * 64 / DP) is the
// same for the whole wavefront.  The (m, l) pairs (lane k: unit k) and the O
// rows of the first UB units are issued together, so a merge of up to UB
// units costs one memory round trip.  A NaN partial sum propagates.
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
                                               OutS* __restrict__ out, int32_t tq, int32_t h) {
  constexpr int NDW = RP * DP / 64;  // dwords per lane per slot
  constexpr int UB = NDW >= 64 ? 1 : (64 / NDW > 16 ? 16 : 64 / NDW);  // units per batch
  const int lane = threadIdx.x & 63;
  // Element offsets of unit k's O row block (this lane's first element) and of
  // its (m, l) pairs.
  auto off_o = [&](int32_t k) { return (static_cast<int64_t>(first) + k) * (RP * DP) + lane; };
  auto off_ml = [&](int32_t k) { return (static_cast<int64_t>(first) + k) * (2 * RP); };
  auto ld_o = [&](int64_t e) __attribute__((always_inline)) -> float { return part_o[e]; };
  auto ld_ml = [&](int64_t e) __attribute__((always_inline)) -> float { return part_ml[e]; };

  // Issue the (m, l) pairs of unit `lane` and the first batch of O rows.
  float2 ml0[RP];
  {
    const int64_t ml = off_ml(min(lane, nunits - 1));
#pragma unroll
    for (int r = 0; r < RP; ++r) ml0[r] = make_float2(ld_ml(ml + 2 * r), ld_ml(ml + 2 * r + 1));
  }
  float v[UB][NDW];  // one batch of O rows; batch 0 is in flight during the reduction
#pragma unroll
  for (int u = 0; u < UB; ++u) {
    const int64_t po = off_o(min(u, nunits - 1));
#pragma unroll
    for (int j = 0; j < NDW; ++j) v[u][j] = ld_o(po + 64 * j);
  }

  // Row max and sum over all units.
  float M[RP], L[RP];
#pragma unroll
  for (int r = 0; r < RP; ++r) {
    M[r] = lane < nunits ? ml0[r].x : -INFINITY;
    L[r] = lane < nunits ? ml0[r].y : 0.0f;
  }
  for (int32_t k = lane + 64; k < nunits; k += 64) {
    const int64_t ml = off_ml(k);
#pragma unroll
    for (int r = 0; r < RP; ++r) ml_combine(M[r], L[r], ld_ml(ml + 2 * r), ld_ml(ml + 2 * r + 1));
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
  // Output row and q head of row r (one-token groups: rows r < qpk).
  // Token of row r within the group (wavefront-uniform; 0 for one-token
  // groups, where the division is skipped).
  int32_t tokr[RP];
#pragma unroll
  for (int r = 0; r < RP; ++r) tokr[r] = 0;
  if (p.dq > 1) {
#pragma unroll
    for (int r = 0; r < RP; ++r) tokr[r] = r / p.qpk;
  }
  const int64_t row0 = static_cast<int64_t>(tq) * p.Hq + h * p.qpk;
  auto qhead = [&](int r) __attribute__((always_inline)) -> int32_t {
    return h * p.qpk + r - tokr[r] * p.qpk;
  };
  auto orow = [&](int r) __attribute__((always_inline)) -> int64_t {
    return row0 + r + static_cast<int64_t>(tokr[r]) * (p.Hq - p.qpk);
  };
  float scale[RP];
#pragma unroll
  for (int r = 0; r < RP; ++r) {
    const float ls = r < rows ? sum_with_sink(p, qhead(r), M[r], L[r]) : L[r];
    scale[r] = ls > 0.0f ? p.v_scale / ls : 0.0f;
  }
  if (p.lse != nullptr) {
#pragma unroll
    for (int r = 0; r < RP; ++r)
      if (lane == r && r < rows) p.lse[orow(r)] = lse_from_log2(M[r], L[r]);
  }

  float acc[NDW];
#pragma unroll
  for (int j = 0; j < NDW; ++j) acc[j] = 0.0f;
  for (int32_t k0 = 0; k0 < nunits; k0 += 64) {
    const int32_t kn = min(64, nunits - k0);
    // Weight of unit k0 + lane for every row (0 for lanes past the end).
    float w[RP];
    if (k0 == 0) {
#pragma unroll
      for (int r = 0; r < RP; ++r)
        w[r] = (lane >= kn || ml0[r].x == -INFINITY) ? 0.0f : exp2f(ml0[r].x - M[r]) * scale[r];
    } else {
      const int64_t ml = off_ml(k0 + min(lane, kn - 1));
#pragma unroll
      for (int r = 0; r < RP; ++r) {
        const float m = ld_ml(ml + 2 * r);
        w[r] = (lane >= kn || m == -INFINITY) ? 0.0f : exp2f(m - M[r]) * scale[r];
      }
    }
    for (int32_t kb = 0; kb < kn; kb += UB) {
      if (k0 != 0 || kb != 0) {
#pragma unroll
        for (int u = 0; u < UB; ++u) {
          const int64_t po = off_o(k0 + min(kb + u, kn - 1));  // in-bounds; weight 0 past kn
#pragma unroll
          for (int j = 0; j < NDW; ++j) v[u][j] = ld_o(po + 64 * j);
        }
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
    if (r < rows && d < p.D) store_out(out, orow(r) * p.D + d, acc[j]);
  }
}

}  // namespace rpa
