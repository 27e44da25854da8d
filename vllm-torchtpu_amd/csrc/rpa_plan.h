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
//   unit             up to `tpu` consecutive tiles of one decode sequence;
//                    units of all sequences are numbered in sequence order.
//   item             (unit, kv head) = unit * Hkv + h: the decode kernel's
//                    work granule, walked in grid-stride order so that
//                    concurrent wavefronts read the kv heads of the same
//                    tokens (adjacent bytes of a page).
#pragma once

#include "rpa_common.h"
#include "rpa_internal.h"

namespace rpa {

constexpr int kPlanThreads = 256;
constexpr int kPlanWaves = kPlanThreads / 64;

struct Plan {
  int32_t num_seqs;     // min(distribution[2], S)
  int32_t tpu;          // tiles per unit
  int32_t total_units;  // (sequence, unit) pairs over all decode sequences
};

// Per-sequence plan arrays in LDS (kMaxDecodeSeqs entries each).
struct PlanLds {
  int32_t nt[kMaxDecodeSeqs];         // decode tiles (0: not a decode sequence)
  int32_t units[kMaxDecodeSeqs + 1];  // exclusive prefix of units; units[n] = total
  int32_t kvlen[kMaxDecodeSeqs];      // kv_len clamped to the page table (every sequence)
  int32_t tq[kMaxDecodeSeqs];         // q row of the sequence (cu_q_lens[s], clamped)
  int32_t cu[kMaxDecodeSeqs + 1];     // cu_q_lens[0 .. num_seqs]
  int32_t red[2 * kPlanWaves];
};

__device__ __forceinline__ void decode_range(const Params& p, int32_t kv_len, int32_t* lo,
                                             int32_t* hi) {
  *hi = kv_len;
  *lo = (p.causal && p.window > 0) ? max(0, kv_len - p.window) : 0;
}

__device__ __forceinline__ bool is_decode_seq(const Params& p, const int32_t* cu,
                                              const int32_t* kv_lens, int32_t s,
                                              int32_t* kv_len_out) {
  const int32_t q_len = cu[s + 1] - cu[s];
  int32_t kv_len = kv_lens[s];
  kv_len = min(kv_len, p.pps * p.ps);
  *kv_len_out = kv_len;
  return q_len == 1 && kv_len >= 1 && cu[s] >= 0 && cu[s] < p.T;
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

// Tiles per unit: about four items per decode wavefront (so the grid-stride
// walk ends evenly), at most kMaxTilesPerUnit (a unit's partial is a few KiB
// against 100+ KiB of keys), and at least what the partial-slot capacity
// (max_units) requires.
constexpr int kMaxTilesPerUnit = 8;

__device__ __forceinline__ int32_t plan_tiles_per_unit(int64_t total_tiles, int32_t nseq,
                                                       int32_t hkv, int32_t decode_waves,
                                                       int32_t max_units) {
  int64_t tpu = (total_tiles * hkv) / (4 * static_cast<int64_t>(max(decode_waves, 1)));
  tpu = tpu < 1 ? 1 : (tpu > kMaxTilesPerUnit ? kMaxTilesPerUnit : tpu);
  const int64_t budget = max<int64_t>(1, static_cast<int64_t>(max_units) - nseq);
  const int64_t need = (total_tiles + budget - 1) / budget;
  return static_cast<int32_t>(tpu > need ? tpu : need);
}

// Builds the plan in LDS (all threads of a kPlanThreads-wide workgroup take
// part; ends with a barrier).  With decode_enabled false no sequence is a
// decode sequence (every row belongs to the finish kernel).
__device__ __forceinline__ Plan build_plan(const Params& p, const int32_t* kv_lens,
                                           const int32_t* cu, const int32_t* dist, int32_t tile,
                                           int32_t max_units, bool decode_enabled, PlanLds& L) {
  Plan pl;
  const int tid = threadIdx.x;
  const int32_t n = num_seqs_of(dist, p.S);
  pl.num_seqs = n;
  int32_t tiles = 0, seqs = 0;
  for (int32_t s = tid; s < n; s += kPlanThreads) {
    int32_t kl, lo, hi, nt = 0;
    if (is_decode_seq(p, cu, kv_lens, s, &kl) && decode_enabled) {
      decode_range(p, kl, &lo, &hi);
      nt = (hi - lo + tile - 1) / tile;
      seqs += 1;
    }
    L.kvlen[s] = kl;
    L.tq[s] = min(max(cu[s], 0), max(p.T - 1, 0));
    L.cu[s] = cu[s];
    L.nt[s] = nt;
    tiles += nt;
  }
  if (tid == 0) L.cu[n] = cu[n];
  for (int o = 32; o > 0; o >>= 1) {
    tiles += __shfl_xor(tiles, o, 64);
    seqs += __shfl_xor(seqs, o, 64);
  }
  if ((tid & 63) == 0) {
    L.red[tid >> 6] = tiles;
    L.red[kPlanWaves + (tid >> 6)] = seqs;
  }
  __syncthreads();
  int64_t total_tiles = 0;
  int32_t nseq = 0;
  for (int w = 0; w < kPlanWaves; ++w) {
    total_tiles += L.red[w];
    nseq += L.red[kPlanWaves + w];
  }
  __syncthreads();
  pl.tpu = plan_tiles_per_unit(total_tiles, nseq, p.Hkv, p.decode_waves, max_units);
  for (int32_t s = tid; s < n; s += kPlanThreads) L.units[s] = (L.nt[s] + pl.tpu - 1) / pl.tpu;
  __syncthreads();
  block_exclusive_scan(L.units, n, L.red);
  pl.total_units = L.units[n];
  return pl;
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

// Rows of a partial slot: min(q_heads_per_kv_head, 16) rounded up to a power
// of two (padding rows are never written and never output).
__host__ __device__ constexpr int decode_slot_rows(int qpk) {
  int r = qpk < 16 ? qpk : 16;
  int rp = 1;
  while (rp < r) rp *= 2;
  return rp;
}

// Keys per tile: 16 KiB of one kv head's K|V bytes (16 x 16-byte loads per
// lane); 32 keys at head_dim 128 bf16.
__host__ __device__ constexpr int decode_tile_tokens(int dp, int kv_bytes) {
  return 16384 / (2 * dp * kv_bytes);
}

}  // namespace rpa
