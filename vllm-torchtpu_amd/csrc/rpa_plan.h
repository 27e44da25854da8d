// Work plan shared by the decode kernel and the finish kernel.
//
// Every workgroup of both kernels derives the same plan from the
// device-resident metadata (kv_lens, cu_q_lens, distribution), so nothing is
// read back to the host and a call stays graph-capturable.
//
//   decode sequence  q_len == 1 and kv_len >= 1 (kernel.py:1345-1349 allows
//                    0 < q_len <= kv_len); its key range [lo, hi) is the whole
//                    history, or the last W keys under a causal window
//                    (kernel.py:196-204 with p = kv_len - 1).
//   tile             TT consecutive keys of one sequence (one kv head).
//   pair             (decode sequence s, kv head h), numbered p = s * Hkv + h.
//   work order       every tile of every pair on one line, pair-major:
//                    g = Hkv * base[s] + h * nt_s + t for tile t of pair
//                    (s, h), with nt_s the sequence's tiles and base[s] their
//                    exclusive prefix.
//   stream-K split   wavefront w of the decode kernel's persistent grid walks
//                    tiles [w * tpw, (w + 1) * tpw) of that line, tpw =
//                    cdiv(G, W) for G tiles and W wavefronts: every wavefront
//                    gets the same number of tiles.  A pair that lies inside
//                    one wavefront's range is finished there; a pair cut by
//                    range ends leaves one partial per wavefront that touched
//                    it, in slot w + p.  Slots never collide: wavefronts and
//                    pairs are both ordered intervals of the line, so
//                    w1 < w2 with both touching pairs p1, p2 forces p1 <= p2.
//                    The partials of pair p are slots w_a + p .. w_b + p with
//                    w_a, w_b the wavefronts owning its first and last tile.
#pragma once

#include "rpa_common.h"
#include "rpa_internal.h"

namespace rpa {

constexpr int kPlanThreads = 256;
constexpr int kPlanWaves = kPlanThreads / 64;

struct Plan {
  int32_t num_seqs;     // min(distribution[2], S)
  int32_t tpw;          // tiles per wavefront (>= 1)
  int32_t total_tiles;  // G: tiles of all pairs
  int32_t n_other;      // sequences with rows that are not decode rows
  int32_t cu_end;       // cu_q_lens[num_seqs]
};

// Per-sequence plan arrays in LDS (kMaxDecodeSeqs entries each).  The
// decode kernel needs only the core; the finish kernel also keeps every
// sequence's kv_len and cu_q_lens.
template <int N>
struct PlanCoreT {
  static constexpr int kCap = N;  // sequences the plan holds
  int32_t base[N + 1];   // exclusive prefix of tiles per sequence; base[n] = total
  int32_t dkv[N];        // kv_len of a decode sequence (clamped), else 0
  int32_t tq[N];         // q row of the sequence (cu_q_lens[s], clamped)
  int32_t ql[N];         // q_len of a decode sequence, else 0
  int32_t cu[N + 1];     // cu_q_lens[0 .. num_seqs] as read
  int32_t red[3 * kPlanWaves];
};
using PlanCore = PlanCoreT<kMaxDecodeSeqs>;
struct PlanRows {
  int32_t kvlen[kMaxDecodeSeqs];      // kv_len clamped to the page table (every sequence)
  int32_t cu[kMaxDecodeSeqs + 1];     // cu_q_lens[0 .. num_seqs]
};

// Keys [lo, hi) that some row of a decode group of q_len tokens attends:
// under a causal window the first token (position kv_len - q_len) sees back
// to kv_len - q_len - W + 1.
__device__ __forceinline__ void decode_range(const Params& p, int32_t kv_len, int32_t q_len,
                                             int32_t* lo, int32_t* hi) {
  *hi = kv_len;
  *lo = (p.causal && p.window > 0) ? max(0, kv_len - q_len - p.window + 1) : 0;
}

// A decode sequence has 1 <= q_len <= dq new tokens (their q_len * qpk rows
// fit the decode kernel's 16 MFMA columns), inside the token and key ranges.
// c0, c1 = cu_q_lens[s], cu_q_lens[s + 1]; kv = kv_lens[s].
__device__ __forceinline__ bool is_decode_seq(const Params& p, int32_t c0, int32_t c1, int32_t kv,
                                              int32_t* kv_len_out, int32_t* q_len_out) {
  const int32_t q_len = c1 - c0;
  const int32_t kv_len = min(kv, p.pps * p.ps);
  *kv_len_out = kv_len;
  *q_len_out = q_len;
  return q_len >= 1 && q_len <= p.dq && kv_len >= q_len && c0 >= 0 && c0 + q_len <= p.T;
}
__device__ __forceinline__ bool is_decode_seq(const Params& p, const int32_t* cu,
                                              const int32_t* kv_lens, int32_t s,
                                              int32_t* kv_len_out, int32_t* q_len_out) {
  return is_decode_seq(p, cu[s], cu[s + 1], kv_lens[s], kv_len_out, q_len_out);
}

// In-place exclusive scan of a[0..n) (values >= 0); a[n] = total.
__device__ __forceinline__ void block_exclusive_scan(int32_t* a, int32_t n, int32_t* red) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int32_t per = (n + kPlanThreads - 1) / kPlanThreads;
  const int32_t s0 = min(n, tid * per), s1 = min(n, s0 + per);
  int32_t local = 0;
  for (int32_t i = s0; i < s1; ++i) local += a[i];
  int32_t x = local;
  for (int o = 1; o < 64; o <<= 1) {
    const int32_t y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  if (lane == 63) red[wave] = x;
  __syncthreads();
  int32_t run = x - local;
  for (int w = 0; w < wave; ++w) run += red[w];
  for (int32_t i = s0; i < s1; ++i) {
    const int32_t v = a[i];
    a[i] = run;
    run += v;
  }
  if (tid == kPlanThreads - 1) a[n] = run;
  __syncthreads();
}

// Tiles of a decode sequence with kv_len dkv and q_len ql (0 for a
// non-decode sequence).
__device__ __forceinline__ int32_t decode_tiles(const Params& p, int32_t dkv, int32_t ql,
                                                int32_t tile) {
  if (dkv <= 0) return 0;
  int32_t lo, hi;
  decode_range(p, dkv, ql, &lo, &hi);
  return (hi - lo + tile - 1) / tile;
}

// Builds the plan in LDS (every thread of a workgroup of at least
// kPlanThreads threads calls it; ends with a barrier).  With decode_enabled
// false no sequence is a decode sequence (every row belongs to the finish
// kernel).  R, when given,
// receives every sequence's kv_len and cu_q_lens.
template <typename PlanLds>
__device__ __forceinline__ Plan build_plan(const Params& p, const int32_t* kv_lens,
                                           const int32_t* cu, const int32_t* dist, int32_t tile,
                                           bool decode_enabled, PlanLds& L, PlanRows* R) {
  Plan pl;
  const int tid = threadIdx.x;
  // The metadata of every sequence slot below min(S, capacity) is loaded
  // without waiting for distribution[2]: the two loads are independent, so
  // the plan costs one memory round trip instead of two.  Slots at or past
  // num_seqs are then treated as empty.
  const int32_t n_cap = min(p.S, PlanLds::kCap);
  const int32_t n = min(num_seqs_of(dist, p.S), PlanLds::kCap);
  pl.num_seqs = n;
  int32_t tiles = 0, seqs = 0, others = 0;
  // Wider workgroups (the prefill kernel's 512 threads) take part with their
  // first kPlanThreads threads only: the reduction slots hold kPlanWaves waves.
  const bool planner = tid < kPlanThreads;
  for (int32_t s = planner ? tid : n_cap; s < n_cap; s += kPlanThreads) {
    const int32_t c0 = cu[s], c1 = cu[s + 1], kv = kv_lens[s];
    const bool live = s < n;
    // Always evaluated: kl (the clamped kv_len) feeds the row plan R too.
    int32_t kl, ql;
    const bool dseq = is_decode_seq(p, c0, c1, kv, &kl, &ql);
    const bool dec = live && decode_enabled && dseq;
    const int32_t nt = dec ? decode_tiles(p, kl, ql, tile) : 0;
    seqs += dec ? 1 : 0;
    others += (live && !dec && c1 > c0) ? 1 : 0;
    L.dkv[s] = dec ? kl : 0;
    L.ql[s] = dec ? ql : 0;
    L.tq[s] = min(max(c0, 0), max(p.T - 1, 0));
    L.cu[s] = c0;
    L.base[s] = live ? nt : 0;  // scanned into the prefix below
    if (live && R != nullptr) {
      R->kvlen[s] = kl;
      R->cu[s] = c0;
    }
    // cu_q_lens[num_seqs]: the end of the last sequence's rows.
    if (s + 1 == n) {
      L.cu[n] = c1;
      if (R != nullptr) R->cu[n] = c1;
    }
    tiles += nt;
  }
  if (n == 0 && tid == 0) {
    L.cu[0] = cu[0];
    if (R != nullptr) R->cu[0] = L.cu[0];
  }
  for (int o = 32; o > 0; o >>= 1) {
    tiles += __shfl_xor(tiles, o, 64);
    seqs += __shfl_xor(seqs, o, 64);
    others += __shfl_xor(others, o, 64);
  }
  if (planner && (tid & 63) == 0) {
    L.red[tid >> 6] = tiles;
    L.red[kPlanWaves + (tid >> 6)] = seqs;
    L.red[2 * kPlanWaves + (tid >> 6)] = others;
  }
  __syncthreads();
  int64_t total_tiles = 0;
  int32_t nseq = 0, nother = 0;
  for (int w = 0; w < kPlanWaves; ++w) {
    total_tiles += L.red[w];
    nseq += L.red[kPlanWaves + w];
    nother += L.red[2 * kPlanWaves + w];
  }
  pl.n_other = nother;
  pl.cu_end = L.cu[n];
  (void)nseq;
  __syncthreads();
  block_exclusive_scan(L.base, n, L.red);
  const int64_t g = total_tiles * p.Hkv;
  pl.total_tiles = static_cast<int32_t>(g);
  const int64_t w = max(p.decode_waves, 1);
  pl.tpw = static_cast<int32_t>(max<int64_t>(1, (g + w - 1) / w));
  return pl;
}

// Publishes the plan for the finish kernel (every thread of the workgroup
// takes part; workgroup b writes the row map of sequences b, b + G, ...).
// The row map takes cu_q_lens from the plan in LDS, so publishing issues
// stores only and never waits on memory.
template <typename PlanLds>
__device__ __forceinline__ void publish_plan(const Params& p, const Plan& pl, const PlanLds& L,
                                             int32_t* plan) {
  const PlanView v = plan_view(plan, p.S);
  int32_t* base = const_cast<int32_t*>(v.base);
  int32_t* dkv = const_cast<int32_t*>(v.dkv);
  int32_t* tq = const_cast<int32_t*>(v.tq);
  int32_t* rowseq = const_cast<int32_t*>(v.rowseq);
  const int tid = threadIdx.x;
  const int32_t n = pl.num_seqs;
  if (blockIdx.x == 0) {
    if (tid == 0) {
      plan[0] = n;
      plan[1] = pl.tpw;
      plan[2] = pl.total_tiles;
      plan[3] = pl.n_other;
    }
    for (int32_t s = tid; s <= n; s += kPlanThreads) base[s] = L.base[s];
    for (int32_t s = tid; s < n; s += kPlanThreads) {
      dkv[s] = L.dkv[s];
      tq[s] = L.tq[s];
    }
  }
  const int32_t G = static_cast<int32_t>(gridDim.x);
  for (int32_t s = static_cast<int32_t>(blockIdx.x); s < n; s += G) {
    const int32_t r0 = min(max(L.cu[s], 0), p.T), r1 = min(max(L.cu[s + 1], r0), p.T);
    const int32_t val = L.dkv[s] > 0 ? -1 : s;
    for (int32_t t = r0 + tid; t < r1; t += kPlanThreads) rowseq[t] = val;
  }
  // Padding rows.
  const int32_t pad0 = min(max(L.cu[n], 0), p.T);
  for (int32_t t = pad0 + static_cast<int32_t>(blockIdx.x) * kPlanThreads + tid; t < p.T;
       t += G * kPlanThreads)
    rowseq[t] = -1;
}

// Largest s in [0, n) with prefix[s] <= x.
__device__ __forceinline__ int32_t find_prefix(const int32_t* prefix, int32_t n, int32_t x) {
  int32_t lo = 0, hi = n;
  while (hi - lo > 1) {
    const int32_t mid = (lo + hi) >> 1;
    if (prefix[mid] <= x) lo = mid; else hi = mid;
  }
  return lo;
}

// Rows of a partial slot: the largest decode row group, min(dq * qpk, 16),
// rounded up to a power of two (padding rows are never written and never
// output).
__host__ __device__ constexpr int decode_slot_rows(int group_rows) {
  int r = group_rows < 16 ? group_rows : 16;
  int rp = 1;
  while (rp < r) rp *= 2;
  return rp;
}

// Keys per tile: 16 KiB of one kv head's K|V bytes (16 x 16-byte loads per
// lane): 32 keys at head_dim 128 bf16, 64 for fp8.
__host__ __device__ constexpr int decode_tile_tokens(int dp, int kv_bytes) {
  return 16384 / (2 * dp * kv_bytes);
}
}  // namespace rpa
