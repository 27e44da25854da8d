// Prefill attention for bf16 KV at head_dim 128 and 256 (unpadded): key
// tiles copied straight from HBM into LDS (gfx950's global_load_lds_dwordx4),
// no register staging.
//
// Included by rpa_prefill.hip, whose prefill_kernel it replaces for these
// shapes.  The item decomposition, row layout and math are the same: a
// workgroup of 8 wavefronts owns 256 q rows at head_dim 128 (BQ = rows / qpk
// query tokens of one sequence times the qpk q heads of one kv head),
// wavefront w owns rows [32w, 32w + 32), lane l owns MFMA column l % 32, and
// per 32-key sub-block
//   S^T[key, row] = K[key, :] . Q^T[:, row]          (v_mfma_f32_32x32x16_bf16)
//   O^T[dim, row] += V^T[dim, key] . P^T[key, row]    (V^T via ds_read_b64_tr_b16)
// with an online softmax in the column layout.  At head_dim 256 the 8
// wavefronts own 16 rows each (128 rows, v_mfma_f32_16x16x32_bf16): 32-row
// blocks would need 192 registers for O and Q, i.e. one wavefront per SIMD.
// Each attention workgroup also writes its q block's new K/V records for its
// kv head into the cache (it is the only workgroup holding those tokens for
// that head); merge workgroups at the front of the grid combine the decode
// kernel's split-K partials.
//
// What changes is the tile path:
//   * Three LDS tile buffers (16 KiB of K and 16 KiB of V each: 64 keys at
//     head_dim 128, 32 at 256), filled by LDS-DMA: each wavefront issues
//     16 / WAVES 1-KiB copies per K (and per V) tile (64 lanes x
//     16 bytes land contiguously), so no VGPRs hold tiles in flight and no
//     ds_write is issued.  A wavefront issues its copies of tile t + 2 after
//     computing tile t (issued before the compute, as the measured variants
//     with three or four buffers did, they slowed it: C3 prefill 443-452 us
//     against 430 us).
//   * Rows are stored unpadded (2 x head_dim bytes) with an XOR swizzle of their
//     16-byte chunks, chosen per operand read pattern:
//       K: chunk c of key k sits at chunk c ^ (k & 15): the 16 lanes that read
//          chunk c of 16 consecutive keys hit 16 distinct chunks (all 64 banks).
//       V: chunk c of key k sits at chunk c ^ 4 (k & 3): a transposing read
//          takes 4 keys x 2 chunks per 16-lane group, 4 aligned chunks per
//          32 lanes; the XOR moves each key's 4 chunks to a distinct group of 4.
//          16-row blocks read 8 keys x 2 chunks per 32 lanes and add 2 to the
//          XOR for keys 4 .. 7 of each 8 (c ^ (4 (k & 3) + 2 ((k >> 2) & 1))).
//     The swizzle is applied on the global side of the copy (lane l of a copy
//     loads the global chunk that belongs at its fixed LDS slot).
//   * One barrier per tile; the copies are issued as inline asm and waited for
//     explicitly (s_waitcnt vmcnt), so the compiler adds no waits of its own
//     on the buffers being filled while the current one is read.
//   * The cross-half exchanges of the softmax use v_permlane32_swap (VALU)
//     instead of LDS permutes.
//
// (Textually included inside rpa_prefill.hip's anonymous namespace, after the
// helpers it shares with prefill_kernel.)
#pragma once

// Largest soft cap (in log2 units of the logits) for which the fixed
// reference max keeps every P in the normal range (see FIXREF below).
constexpr float kFixRefMaxLog2 = 87.0f;

template <int DP_, int RW_ = 32>
struct DmaCfg {
  static constexpr int DP = DP_;
  // Rows per wavefront: 32 (32x32x16 MFMAs) or 16 (16x16x32 MFMAs).
  static constexpr int RW = RW_;
  // 32 rows: head_dim 128: 8 wavefronts, two per SIMD (256 registers each);
  // head_dim 256: 4 wavefronts, one per SIMD (the O and Q operands alone take
  // 192).  16 rows at head_dim 256: 8 wavefronts, two per SIMD (O and Q take
  // 96): one wavefront issues MFMAs at half the pipe's rate, two fill it.
  static constexpr int THREADS = RW == 32 ? (DP <= 128 ? 512 : 256) : (DP <= 128 ? 1024 : 512);
  static constexpr int WAVES = THREADS / 64;
  static constexpr int ROWS = RW * WAVES;          // q rows per item
  static constexpr int ROWB = 2 * DP;              // bytes of one key's K (or V) row
  static constexpr int BK = 16384 / ROWB;          // keys per tile: 16 KiB of K, 16 KiB of V
  static constexpr int NSB = BK / 32;              // 32-key sub-blocks per tile
  static constexpr int TILE = BK * ROWB;           // 16 KiB
  static constexpr int CHUNKS = TILE / 1024;       // 1-KiB copies per K (or V) tile
  static constexpr int CPW = CHUNKS / WAVES;       // per wavefront
  static constexpr int CPR = ROWB / 16;            // 16-byte chunks per row
  static constexpr int KSTEPS = DP / (512 / RW);   // QK^T k-steps (16 or 32 dims each)
  static constexpr int NT = DP / RW;               // RW-dim output blocks
  static constexpr int PLAN_BYTES = static_cast<int>(sizeof(PlanCore) + sizeof(PlanRows));
  static_assert(CHUNKS % WAVES == 0 && NSB >= 1, "whole copies per wavefront");
  static_assert(PLAN_BYTES >= 4 * (kMaxDecodeSeqs + 1), "block prefix fits the plan scratch");
};

typedef __attribute__((address_space(3))) unsigned char lds_u8_t;

__device__ __forceinline__ uint32_t lds_offset(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const lds_u8_t*)p));
}

// 16 bytes per lane from global address g to LDS byte lds + 16 * lane (lds is
// wavefront-uniform, in M0).  Counted by vmcnt.
__device__ __forceinline__ void dma16(const void* g, uint32_t lds) {
  asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(g), "{m0}"(lds) : "memory");
}
// Waits until at most N of this wavefront's vector-memory operations are
// outstanding.
template <int N>
__device__ __forceinline__ void vm_wait() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
// This wavefront's LDS operations complete, then the workgroup barrier.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// max(x, x of lane l ^ 32) and x + (x of lane l ^ 32): one v_permlane32_swap.
__device__ __forceinline__ float xmax32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return __builtin_fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xmax16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return __builtin_fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xsum16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xsum32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Tiles (of BK keys) of block b (query tokens [b bq, b bq + bq)) of sequence
// s: the key range its rows attend, as the kernel computes it.
template <int BK>
__device__ __forceinline__ int32_t item_tiles(const Params& p, const int32_t* cu,
                                              const int32_t* kv_lens, int32_t s, int32_t b,
                                              int32_t bq) {
  const int32_t q_len = cu[s + 1] - cu[s];
  const int32_t kv_len = min(kv_lens[s], p.pps * p.ps);
  const int32_t new_start = kv_len - q_len;
  const int32_t tok0 = b * bq;
  const int32_t ntok = min(bq, q_len - tok0);
  int32_t lo = 0, hi = kv_len;
  if (p.causal) {
    hi = min(kv_len, new_start + tok0 + ntok);
    if (p.window > 0) lo = max(0, new_start + tok0 - p.window + 1);
  }
  return hi > lo ? (hi - lo + BK - 1) / BK : 0;
}

// The block of rank `rank` when the item blocks (blk: exclusive prefix of
// blocks per sequence, in LDS, total = blk[n]) are ordered by tile count,
// longest first, ties in block order: the hardware dispatches workgroups in
// index order to whichever CU frees up, so the longest items start first
// and the short ones fill the tail (longest-processing-time-first).  A
// counting sort in LDS behind the prefix (kLenBuckets buckets of tile
// counts; longer items share the last bucket).  Every thread of the
// workgroup calls it; it ends with a barrier.  When the LDS scratch behind
// the prefix is too small it falls back to the last block first.
constexpr int kLenBuckets = 2048;
template <int BK, int THREADS, int SCRATCH_INTS>
__device__ __forceinline__ int32_t longest_first_block(const Params& p, const int32_t* cu,
                                                       const int32_t* kv_lens, int32_t* blk,
                                                       int32_t n, int32_t total, int32_t rank,
                                                       int32_t bq, int32_t* red) {
  const int tid = threadIdx.x;
  if (n + 1 + total + kLenBuckets + 1 > SCRATCH_INTS) return total - 1 - rank;
  int32_t* blen = blk + n + 1;      // tile count of each block, then flags
  int32_t* hist = blen + total;     // blocks per tile count, longest first
  for (int32_t i = tid; i < kLenBuckets; i += THREADS) hist[i] = 0;
  for (int32_t k = tid; k < total; k += THREADS) {
    const int32_t s = find_prefix(blk, n, k);
    blen[k] = min(item_tiles<BK>(p, cu, kv_lens, s, k - blk[s], bq), kLenBuckets - 1);
  }
  __syncthreads();
  for (int32_t k = tid; k < total; k += THREADS) atomicAdd(&hist[kLenBuckets - 1 - blen[k]], 1);
  __syncthreads();
  block_exclusive_scan(hist, kLenBuckets, red);
  const int32_t bi = find_prefix(hist, kLenBuckets, rank);  // a non-empty bucket
  const int32_t tc = kLenBuckets - 1 - bi;
  const int32_t j = rank - hist[bi];  // rank within the bucket
  __syncthreads();                    // every thread has read hist
  for (int32_t k = tid; k < total; k += THREADS) blen[k] = blen[k] == tc ? 1 : 0;
  __syncthreads();
  block_exclusive_scan(blen, total, red);
  // The j-th block with tile count tc: the last k whose prefix count is j.
  return find_prefix(blen, total, j);
}

// CAP: the logit soft cap is on (a template parameter, so the score
// transform has no per-element branches).
// FIXREF (soft-capped logits, |y| <= b = cap * log2 e <= kFixRefMaxLog2): each
// row's reference max is fixed at its first attended tile, m = max(tile max,
// b - 64), and never moves, so P = 2^(y - m) stays within [2^(64 - 2b), 2^64]
// (normal in bf16 and fp32, no overflow of P, l or O) and the accumulators are
// never rescaled.  At head_dim 256 that keeps the compiler from moving the
// 128 accumulator registers between AGPRs and VGPRs on every tile (the rescale
// is a VALU use of them); results equal the rescaling kernel's up to rounding.
template <int DP_, typename OutS, bool CAP, bool FIXREF = false, int RW_ = 32>
__global__ void __launch_bounds__((DmaCfg<DP_, RW_>::THREADS))
__attribute__((amdgpu_waves_per_eu((DmaCfg<DP_, RW_>::THREADS) / 256)))
prefill_dma_kernel(Params p, const uint16_t* __restrict__ q, const uint16_t* __restrict__ keys,
                   const uint16_t* __restrict__ values, uint16_t* __restrict__ cache,
                   const int32_t* __restrict__ kv_lens, const int32_t* __restrict__ page_indices,
                   const int32_t* __restrict__ cu, const int32_t* __restrict__ dist,
                   OutS* __restrict__ out, const int32_t* __restrict__ plan,
                   const float* __restrict__ part_o, const float* __restrict__ part_ml,
                   int32_t nfm, int32_t nfw) {
  using C = DmaCfg<DP_, RW_>;
  constexpr int DP = C::DP, BK = C::BK, RW = C::RW;
  static_assert(RW == 32 || C::THREADS <= 512, "the plan scan's reduction slots hold 8 waves");
  using Acc = typename std::conditional<RW == 32, f32x16_t, f32x4_t>::type;
  // Separate arrays per buffer: reads of one are never ordered after copies
  // into another.
  __shared__ __align__(1024) unsigned char kt0[C::TILE], kt1[C::TILE], kt2[C::TILE];
  __shared__ __align__(1024) unsigned char vt0[C::TILE], vt1[C::TILE], vt2[C::TILE];
  __shared__ __align__(16) unsigned char aux[C::PLAN_BYTES];
  __shared__ int32_t pages[kItemPages];
  __shared__ int32_t red[3 * kPlanWaves];
  // Key address table, three tiles: [t % 3][key] = {K row, V row}.
  __shared__ __align__(16) uint64_t ktab[3][BK][2];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int col = lane & 31;
  const int half = lane >> 5;
  // 16-row blocks: lane = 16 g + rn holds row rn (k-slots / output rows 4g ..).
  const int rn = lane & 15;
  const int g4l = lane >> 4;
  const bool decode_on = p.decode_waves > 0;
  const int32_t bq = C::ROWS / p.qpk;
  // ---- finish workgroups: [0, nfm) merge items, the last nfw write items.
  const int32_t blk_id = static_cast<int32_t>(blockIdx.x);
  const int32_t nattn = static_cast<int32_t>(gridDim.x) - nfm - nfw;
  {
    if (blk_id < nfm || blk_id >= nfm + nattn) {
      const bool merges = blk_id < nfm;
      prefill_finish_role<uint16_t, DP, OutS>(p, aux, keys, values, cache, kv_lens,
                                              page_indices, cu, dist, out, plan, part_o, part_ml,
                                              merges, merges ? nfm : nfw,
                                              merges ? blk_id : blk_id - nfm - nattn, C::WAVES);
      return;
    }
  }
  const int32_t bid = blk_id - nfm;
  if (decode_on && plan[3] == 0) return;

  // ---- item (block kb over all owned sequences, kv head h), longest first.
  int32_t* blk = reinterpret_cast<int32_t*>(aux);
  const int32_t n = min(num_seqs_of(dist, p.S), kMaxDecodeSeqs);
  for (int32_t s = tid; s < n; s += C::THREADS)
    blk[s] = prefill_blocks(p, cu, kv_lens, s, bq, decode_on);
  __syncthreads();
  block_exclusive_scan(blk, n, red);
  const int32_t total = blk[n];
  const int32_t h = bid % p.Hkv;
  const int32_t rank = bid / p.Hkv;
  if (rank >= total) return;
  const int32_t kb = longest_first_block<BK, C::THREADS, C::PLAN_BYTES / 4>(
      p, cu, kv_lens, blk, n, total, rank, bq, red);
  const int32_t s = find_prefix(blk, n, kb);
  const int32_t b = kb - blk[s];
  const int32_t q_start = cu[s];
  const int32_t q_len = cu[s + 1] - q_start;
  if (q_start < 0 || q_len <= 0 || q_start + q_len > p.T) return;
  const int32_t kv_cap = p.pps * p.ps;
  const int32_t kv_len = min(kv_lens[s], kv_cap);
  const int32_t new_start = kv_len - q_len;
  const bool new_from_input = p.skip_kv_update == 0;
  const int32_t* ptab = page_indices + static_cast<int64_t>(s) * p.pps;

  const int32_t tok0 = b * bq;
  const int32_t ntok = min(bq, q_len - tok0);
  int32_t lo = 0, hi = kv_len;
  if (p.causal) {
    hi = min(kv_len, new_start + tok0 + ntok);
    if (p.window > 0) lo = max(0, new_start + tok0 - p.window + 1);
  }
  const int32_t ntiles = hi > lo ? (hi - lo + BK - 1) / BK : 0;

  const int32_t r = wave * RW + (RW == 32 ? col : rn);
  const int32_t ti = r / p.qpk;
  const bool row_ok = ti < ntok && r < bq * p.qpk;
  const int32_t tok = tok0 + min(ti, ntok - 1);
  const int32_t qhead = h * p.qpk + r % p.qpk;
  auto key_range = [&](int32_t token, int32_t* klo, int32_t* khi) {
    const int32_t pos = new_start + token;
    *klo = 0;
    *khi = kv_len;
    if (p.causal) {
      *khi = min(kv_len, pos + 1);
      if (p.window > 0) *klo = max(0, pos - p.window + 1);
    }
  };
  int32_t row_lo, row_hi;
  key_range(tok, &row_lo, &row_hi);
  const bool wave_live = wave * RW < bq * p.qpk && wave * RW / p.qpk < ntok;
  const int32_t wt0 = tok0 + min(wave * RW / p.qpk, ntok - 1);
  const int32_t wt1 = tok0 + min(min(wave * RW + RW - 1, bq * p.qpk - 1) / p.qpk, ntok - 1);
  int32_t w_lo0, w_hi0, w_lo1, w_hi1;
  key_range(wt0, &w_lo0, &w_hi0);
  key_range(wt1, &w_lo1, &w_hi1);

  // ---- page ids of the item's keys into LDS (longer ranges read the table).
  const int32_t pg0 = hi > lo ? page_of(p, lo) : 0;
  const int32_t npg = hi > lo ? page_of(p, hi - 1) - pg0 + 1 : 0;
  const bool lds_pages = npg <= kItemPages;
  if (lds_pages)
    for (int32_t i = tid; i < npg; i += C::THREADS) pages[i] = min(max(ptab[pg0 + i], 0), p.P - 1);
  __syncthreads();

  // ---- address table: K and V row of every key of tile t (its cache
  // record, or its k/v input row for this call's new tokens), by threads
  // 0 .. BK - 1.
  auto fill_tab = [&](int32_t t, int slot) __attribute__((always_inline)) {
    if (tid < BK) {
      const int32_t j = min(lo + t * BK + tid, hi - 1);  // past the range: a valid key
      const uint16_t* kr;
      const uint16_t* vr;
      if (new_from_input && j >= new_start) {
        const int64_t row = min(q_start + (j - new_start), p.T - 1);
        kr = keys + (row * p.Hkv + h) * DP;
        vr = values + (row * p.Hkv + h) * DP;
      } else {
        const int32_t pg = lds_pages ? pages[page_of(p, j) - pg0]
                                     : min(max(ptab[page_of(p, j)], 0), p.P - 1);
        kr = cache + (static_cast<int64_t>(pg) * p.ps + slot_of(p, j)) * p.rec +
             static_cast<int64_t>(2 * h) * DP;
        vr = kr + DP;
      }
      ktab[slot][tid][0] = reinterpret_cast<uint64_t>(kr);
      ktab[slot][tid][1] = reinterpret_cast<uint64_t>(vr);
    }
  };
  // V chunk c of key k sits at chunk c ^ vswz(k).  16-row blocks read 8 keys
  // (2 chunks each) per 32 lanes: bit 1 of the XOR separates keys 4 .. 7 of
  // each 8 from keys 0 .. 3, so the 32 lanes cover all 64 banks.
  auto vswz = [](int key) __attribute__((always_inline)) -> int {
    return RW == 32 ? 4 * (key & 3) : 4 * (key & 3) + 2 * ((key >> 2) & 1);
  };
  // ---- copies of tile t into buffer B: this wavefront's 1-KiB chunks
  // c = wave + WAVES i hold keys 4c .. 4c + 3; lane l lands at chunk l % 16 of
  // key 4c + l / 16 and loads the global chunk the swizzle puts there.
  auto issue = [&](int32_t t, uint32_t kbuf, uint32_t vbuf) __attribute__((always_inline)) {
    const int slot = t % 3;
#pragma unroll
    for (int i = 0; i < C::CPW; ++i) {
      const int c = wave + C::WAVES * i;
      const int key = (1024 / C::ROWB) * c + lane / C::CPR;
      const int j = lane % C::CPR;
      const unsigned char* ka = reinterpret_cast<const unsigned char*>(ktab[slot][key][0]);
      const unsigned char* va = reinterpret_cast<const unsigned char*>(ktab[slot][key][1]);
      const uint32_t kl = __builtin_amdgcn_readfirstlane(kbuf + 1024 * c);
      const uint32_t vl = __builtin_amdgcn_readfirstlane(vbuf + 1024 * c);
      dma16(ka + 16 * (j ^ (key & 15)), kl);
      dma16(va + 16 * (j ^ vswz(key)), vl);
    }
  };

  // ---- Q^T operand (B of S^T): column = row, k-slots 8 half .. + 7 of each
  // 16-dim k-step (head_dim == 128: no padding).
  uint4 qop[C::KSTEPS];
  {
    const uint16_t* qrow = q + (static_cast<int64_t>(q_start + tok) * p.Hq + qhead) * DP;
#pragma unroll
    for (int kk = 0; kk < C::KSTEPS; ++kk)
      qop[kk] = *reinterpret_cast<const uint4*>(
          qrow + (RW == 32 ? 16 * kk + 8 * half : 32 * kk + 8 * g4l));
  }

  // Swizzled operand offsets (ROWB-byte rows).  K: key 32 sb + col, chunk
  // 2 kk + half at chunk (2 kk + half) ^ (col & 15): byte (kbase ^ 32 kk) +
  // 32 ROWB sb.
  const uint32_t kbase = col * C::ROWB + 16 * (half ^ (col & 15));
  // V (ds_read_b64_tr_b16, 16-lane group G, lane jl): key 32 sb + 16 ks +
  // 4 (G >> 1) + jl / 4 (+ 8 for the second read), dims 32 tt + 16 (G & 1) +
  // 4 (jl & 3): chunk 4 tt + 2 (G & 1) + ((jl >> 1) & 1) at chunk ^ 4 (jl >> 2),
  // byte (vbase ^ 64 tt) + 32 ROWB sb + 16 ROWB ks (+ 8 ROWB).
  const int G = lane >> 4, jl = lane & 15;
  const uint32_t vbase = (4 * (G >> 1) + (jl >> 2)) * C::ROWB + 64 * (jl >> 2) +
                         16 * (2 * (G & 1) + ((jl >> 1) & 1)) + 8 * (jl & 1);

  const float cm = CAP ? 1.0f : p.score_scale * kLog2e;
  const SoftCapLog2 capk = soft_cap_log2_consts(p);
  Acc oacc[C::NT];
#pragma unroll
  for (int t = 0; t < C::NT; ++t) oacc[t] = Acc{};
  float m_ref = -INFINITY;
  float l_run = 0.0f;

  // ---- 16-row blocks (16x16x32 MFMAs).  Lane 16 g + rn: row rn.  Per 32-key
  // sub-block: S^T for key groups x = 0, 1 (keys 32 sb + 16 x + ...):
  //   A = K[key 32 sb + 16 x + rn][dims 32 kk + 8 g ..], B = Q^T (qop[kk]),
  //   lane holds S^T[key 32 sb + 16 x + 4 g + i][row rn], i < 4;
  // P^T k-slot 8 g + 4 x + i <-> key 32 sb + 16 x + 4 g + i, and the V^T
  // operand (two ds_read_b64_tr_b16, x = 0, 1) follows the same key order:
  //   A = V^T[dims 16 tt + rn][those 8 keys]; O^T[dim 16 tt + 4 g + i][row rn].
  // K chunk c of key k at c ^ (k & 15); V chunk c at c ^ vswz(k).
  auto compute16 = [&](int32_t t, const unsigned char* kbuf, const unsigned char* vbuf,
                       int32_t k0, bool need_mask) __attribute__((always_inline)) {
    if constexpr (RW == 16) {
#pragma unroll
      for (int sb = 0; sb < C::NSB; ++sb) {
        constexpr int KS = C::KSTEPS;
        auto kread = [&](int x, int kk) __attribute__((always_inline)) -> uint4 {
          const int key = 32 * sb + 16 * x + rn;
          return *reinterpret_cast<const uint4*>(kbuf + key * C::ROWB +
                                                 16 * ((4 * kk + g4l) ^ rn));
        };
        f32x4_t sacc[2] = {f32x4_t{}, f32x4_t{}};
        constexpr int kRA = 4;  // K operand reads in flight (of 2 KS)
        uint4 kb[kRA];
#pragma unroll
        for (int i = 0; i < kRA; ++i) kb[i] = kread(i & 1, i >> 1);
#pragma unroll
        for (int i = 0; i < 2 * KS; ++i) {
          const uint4 kv = kb[i % kRA];
          if (i + kRA < 2 * KS) kb[i % kRA] = kread((i + kRA) & 1, (i + kRA) >> 1);
          sacc[i & 1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
              __builtin_bit_cast(bf16x8_t, kv), __builtin_bit_cast(bf16x8_t, qop[i >> 1]),
              sacc[i & 1], 0, 0, 0);
        }
        // Scores: y[4 x + i] -> key k0 + 32 sb + 16 x + 4 g + i.
        float y[8];
#pragma unroll
        for (int x = 0; x < 2; ++x)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            float v = sacc[x][i];
            if constexpr (CAP) v = soft_cap_log2(v, capk.a, capk.b);
            y[4 * x + i] = v;
          }
        float cme = cm;
        if (!(cm > 0.0f)) {
#pragma unroll
          for (int i = 0; i < 8; ++i) y[i] *= cm;
          cme = 1.0f;
        }
        if (need_mask) {
          // Key j = jb + c with a compile-time c: compare c against the
          // range shifted by jb (no per-score offset registers).
          const int32_t jb = k0 + 32 * sb + 4 * g4l;
          const int32_t dlo = row_lo - jb, dhi = row_hi - jb;
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const int32_t c = 16 * (i >> 2) + (i & 3);
            if (c < dlo || c >= dhi) y[i] = -INFINITY;
          }
        }
        float tmax = -INFINITY;
#pragma unroll
        for (int i = 0; i < 8; ++i) tmax = __builtin_fmaxf(tmax, y[i]);
        tmax = xmax32(xmax16(tmax));
        const float m_tile = tmax * cme;
        if constexpr (FIXREF) {
          if (m_ref == -INFINITY && m_tile != -INFINITY)
            m_ref = __builtin_fmaxf(m_tile, capk.b - 64.0f);
        } else if (__any(m_tile > m_ref + kRescaleLog2)) {
          const float m_new = __builtin_fmaxf(m_ref, m_tile);
          const float alpha = (m_ref == -INFINITY) ? 0.0f : exp2f(m_ref - m_new);
          l_run *= alpha;
#pragma unroll
          for (int tt = 0; tt < C::NT; ++tt) oacc[tt] *= alpha;
          m_ref = m_new;
        }
        const float m_use = (m_ref == -INFINITY) ? 0.0f : m_ref;
#pragma unroll
        for (int i = 0; i < 8; ++i) y[i] = __builtin_amdgcn_exp2f(fmaf(y[i], cme, -m_use));
        const uint4 pop = make_uint4(pack_bf16x2_rne(y[0], y[1]), pack_bf16x2_rne(y[2], y[3]),
                                     pack_bf16x2_rne(y[4], y[5]), pack_bf16x2_rne(y[6], y[7]));
        float psum = sum_bf16x2(pop.x, sum_bf16x2(pop.y, 0.0f));
        psum = sum_bf16x2(pop.z, sum_bf16x2(pop.w, psum));
        l_run += psum;
        // V^T reads: in 16-lane group g, lane jl (= rn) points at key
        // 32 sb + 16 x + 4 g + jl / 4, dims 16 tt + 4 (jl & 3): chunk
        // 2 tt + ((jl >> 1) & 1) at chunk ^ vswz(key), byte 8 (jl & 1).
        auto vread = [&](int tt) __attribute__((always_inline)) -> uint4 {
          const int kq = 4 * g4l + (rn >> 2);
          const int off = 16 * ((2 * tt + ((rn >> 1) & 1)) ^ vswz(kq)) + 8 * (rn & 1);
          const unsigned char* ra = vbuf + (32 * sb + kq) * C::ROWB + off;
          const v4i16 va = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (__attribute__((address_space(3))) v4i16*)ra);
          const v4i16 vb = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (__attribute__((address_space(3))) v4i16*)(ra + 16 * C::ROWB));
          const uint2 ua = __builtin_bit_cast(uint2, va), ub = __builtin_bit_cast(uint2, vb);
          return make_uint4(ua.x, ua.y, ub.x, ub.y);
        };
        constexpr int kVR = 2;
        uint4 vb2[kVR];
#pragma unroll
        for (int i = 0; i < kVR; ++i) vb2[i] = vread(i);
#pragma unroll
        for (int tt = 0; tt < C::NT; ++tt) {
          const uint4 vop = vb2[tt % kVR];
          if (tt + kVR < C::NT) vb2[tt % kVR] = vread(tt + kVR);
          oacc[tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
              __builtin_bit_cast(bf16x8_t, vop), __builtin_bit_cast(bf16x8_t, pop), oacc[tt], 0,
              0, 0);
        }
      }
    }
  };
  auto compute = [&](int32_t t, const unsigned char* kbuf, const unsigned char* vbuf)
                     __attribute__((always_inline)) {
    const int32_t k0 = lo + t * BK;
    if (!(wave_live && k0 < w_hi1 && k0 + BK > w_lo0)) return;
    const bool need_mask = !(k0 >= w_lo1 && k0 + BK <= w_hi0);
    if constexpr (RW == 16) {
      compute16(t, kbuf, vbuf, k0, need_mask);
      return;
    } else {
    // One 32-key sub-block; sb is a compile-time constant so that each
    // sub-block's scheduling groups get SyncIDs of their own.
    auto sub_block = [&](auto sbc) __attribute__((always_inline)) {
      constexpr int sb = decltype(sbc)::value;
      constexpr int kSyncS = 2 * sb, kSyncPV = 2 * sb + 1;
      __builtin_amdgcn_sched_barrier(0);
      constexpr int kRA = 4;  // K operand reads in flight
      auto kread = [&](int kk) __attribute__((always_inline)) -> uint4 {
        return *reinterpret_cast<const uint4*>(kbuf + 32 * C::ROWB * sb + (kbase ^ (32u * kk)));
      };
      f32x16_t sacc = f32x16_t{};
      uint4 kb[kRA];
#pragma unroll
      for (int i = 0; i < kRA; ++i) kb[i] = kread(i);
#pragma unroll
      for (int kk = 0; kk < C::KSTEPS; ++kk) {
        const uint4 kv = kb[kk % kRA];
        if (kk + kRA < C::KSTEPS) kb[kk % kRA] = kread(kk + kRA);
        sacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
            __builtin_bit_cast(bf16x8_t, kv), __builtin_bit_cast(bf16x8_t, qop[kk]), sacc, 0, 0,
            0);
      }
      __builtin_amdgcn_sched_group_barrier(0x100, kRA, kSyncS);
#pragma unroll
      for (int i = 0; i < C::KSTEPS - kRA; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, kSyncS);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, kSyncS);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, kRA, kSyncS);
      // Scores: register i -> key k0 + 32 sb + 8 (i / 4) + 4 half + i % 4.
      float y[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        float x = sacc[i];
        if constexpr (CAP) x = soft_cap_log2(x, capk.a, capk.b);
        y[i] = x;
      }
      float cme = cm;
      if (!(cm > 0.0f)) {
#pragma unroll
        for (int i = 0; i < 16; ++i) y[i] *= cm;
        cme = 1.0f;
      }
      if (need_mask) {
        // Key j = jb + c with a compile-time c: compare c against the range
        // shifted by jb (no per-score offset registers).
        const int32_t jb = k0 + 32 * sb + 4 * half;
        const int32_t dlo = row_lo - jb, dhi = row_hi - jb;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int32_t c = 8 * (i >> 2) + (i & 3);
          if (c < dlo || c >= dhi) y[i] = -INFINITY;
        }
      }
      float tmax = -INFINITY;
#pragma unroll
      for (int i = 0; i < 16; ++i) tmax = __builtin_fmaxf(tmax, y[i]);
      tmax = xmax32(tmax);
      const float m_tile = tmax * cme;
      if constexpr (FIXREF) {
        if (m_ref == -INFINITY && m_tile != -INFINITY)
          m_ref = __builtin_fmaxf(m_tile, capk.b - 64.0f);
      } else if (__any(m_tile > m_ref + kRescaleLog2)) {
        const float m_new = __builtin_fmaxf(m_ref, m_tile);
        const float alpha = (m_ref == -INFINITY) ? 0.0f : exp2f(m_ref - m_new);
        l_run *= alpha;
#pragma unroll
        for (int tt = 0; tt < C::NT; ++tt) oacc[tt] *= alpha;
        m_ref = m_new;
      }
      const float m_use = (m_ref == -INFINITY) ? 0.0f : m_ref;
#pragma unroll
      for (int i = 0; i < 16; ++i) y[i] = __builtin_amdgcn_exp2f(fmaf(y[i], cme, -m_use));
      uint4 pops[2];
      float psum = 0.0f;
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const float* pv = y + 8 * ks;
        pops[ks] = make_uint4(pack_bf16x2_rne(pv[0], pv[1]), pack_bf16x2_rne(pv[2], pv[3]),
                              pack_bf16x2_rne(pv[4], pv[5]), pack_bf16x2_rne(pv[6], pv[7]));
        psum = sum_bf16x2(pops[ks].x, sum_bf16x2(pops[ks].y, psum));
        psum = sum_bf16x2(pops[ks].z, sum_bf16x2(pops[ks].w, psum));
      }
      l_run += psum;
      constexpr int kP = 2 * C::NT;
      auto vread = [&](int i) __attribute__((always_inline)) -> uint4 {
        const int ks = i / C::NT, tt = i % C::NT;
        const unsigned char* ra =
            vbuf + 32 * C::ROWB * sb + 16 * C::ROWB * ks + (vbase ^ (64u * tt));
        const v4i16 va = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) v4i16*)ra);
        const v4i16 vb = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) v4i16*)(ra + 8 * C::ROWB));
        const uint2 ua = __builtin_bit_cast(uint2, va), ub = __builtin_bit_cast(uint2, vb);
        return make_uint4(ua.x, ua.y, ub.x, ub.y);
      };
      uint4 vb2[2];
      vb2[0] = vread(0);
      vb2[1] = vread(1);
#pragma unroll
      for (int i = 0; i < kP; ++i) {
        const uint4 vop = vb2[i & 1];
        if (i + 2 < kP) vb2[i & 1] = vread(i + 2);
        const int tt = i % C::NT;
        oacc[tt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
            __builtin_bit_cast(bf16x8_t, vop), __builtin_bit_cast(bf16x8_t, pops[i / C::NT]),
            oacc[tt], 0, 0, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x100, 4, kSyncPV);
#pragma unroll
      for (int i = 0; i < kP - 2; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, kSyncPV);
        __builtin_amdgcn_sched_group_barrier(0x100, 2, kSyncPV);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, 2, kSyncPV);
    };
    static_assert(C::NSB <= 2, "sub-blocks per tile");
    sub_block(std::integral_constant<int, 0>{});
    if constexpr (C::NSB > 1) sub_block(std::integral_constant<int, 1>{});
    }
  };

  // ---- pipeline.  Prologue: address tables of tiles 0..2, copies of tiles
  // 0 and 1, then everything (the q operand too) lands before the loop.
  // Iteration t: wait for this wavefront's copies of tile t (those of tile
  // t + 1 may stay in flight), barrier (every wavefront's copies of tile t
  // and the table of tile t + 2 have landed; every wavefront is done with
  // tile t - 1), write the table of tile t + 3 into the slot tile t used,
  // compute tile t, then issue the copies of tile t + 2 into the buffer tile
  // t - 1 used.
  if (ntiles > 0)
    for (int i = 0; i < 3; ++i) fill_tab(min(i, ntiles - 1), i);
  __syncthreads();
  // LDS byte offsets of the buffers (the copies' destinations).
  const uint32_t ko0 = lds_offset(kt0), ko1 = lds_offset(kt1), ko2 = lds_offset(kt2);
  const uint32_t vo0 = lds_offset(vt0), vo1 = lds_offset(vt1), vo2 = lds_offset(vt2);
  if (ntiles > 0) issue(0, ko0, vo0);
  if (ntiles > 1) issue(1, ko1, vo1);
  // A wait the compiler sees: it then knows the q operand has landed (it
  // cannot count the copies, which are inline asm).
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  auto iter = [&](int32_t t, const unsigned char* kc, const unsigned char* vc, uint32_t kn,
                  uint32_t vn) __attribute__((always_inline)) {
    if (t > 0) {
      if (t + 1 < ntiles)
        vm_wait<2 * C::CPW>();
      else
        vm_wait<0>();
      lds_barrier();
    }
    if (t + 3 < ntiles) fill_tab(t + 3, t % 3);
    compute(t, kc, vc);
    if (t + 2 < ntiles) issue(t + 2, kn, vn);
  };
  for (int32_t t = 0; t < ntiles; t += 3) {
    iter(t, kt0, vt0, ko2, vo2);
    if (t + 1 < ntiles) iter(t + 1, kt1, vt1, ko0, vo0);
    if (t + 2 < ntiles) iter(t + 2, kt2, vt2, ko1, vo1);
  }

  // ---- this item's new tokens into the cache (kernel.py:154-166): token
  // rows tok0 .. tok0 + ntok - 1 of the sequence are keys new_start + tok0 ..,
  // and this workgroup is the only one holding them for kv head h, so it
  // writes their K and V rows from the inputs (16-byte chunks; all loads of a
  // batch before its stores).  Overlaps other workgroups' MFMA work instead of
  // running in write workgroups at the launch's tail.
  if (new_from_input) {
    constexpr int CH = DP / 8;  // 16-byte chunks per K (or V) row
    constexpr int kB = 8;
    const int32_t nchunk = ntok * 2 * CH;
    for (int32_t c0 = tid; c0 < nchunk; c0 += C::THREADS * kB) {
      uint4 v[kB];
      int32_t pgv[kB];
      int32_t rowj[kB], part[kB];
#pragma unroll
      for (int b = 0; b < kB; ++b) {
        const int32_t c = c0 + b * C::THREADS;
        const int32_t i = c / (2 * CH);
        const int32_t r = c - i * 2 * CH;  // K chunks, then V chunks
        const int32_t j = new_start + tok0 + i;
        rowj[b] = (c < nchunk && j >= 0 && j < kv_cap) ? j : -1;
        part[b] = r;
        pgv[b] = -1;
        v[b] = make_uint4(0u, 0u, 0u, 0u);
        if (rowj[b] >= 0) {
          pgv[b] = ptab[page_of(p, j)];
          const uint16_t* src = (r < CH ? keys : values) +
                                (static_cast<int64_t>(q_start + tok0 + i) * p.Hkv + h) * DP +
                                8 * (r < CH ? r : r - CH);
          v[b] = *reinterpret_cast<const uint4*>(src);
        }
      }
#pragma unroll
      for (int b = 0; b < kB; ++b) {
        if (rowj[b] < 0 || pgv[b] < 0 || pgv[b] >= p.P) continue;
        uint16_t* dst = cache + (static_cast<int64_t>(pgv[b]) * p.ps + slot_of(p, rowj[b])) * p.rec +
                        static_cast<int64_t>(2 * h) * DP + 8 * part[b];
        *reinterpret_cast<uint4*>(dst) = v[b];
      }
    }
  }

  if constexpr (RW == 16) {
    // ---- output: lane 16 g + rn, block tt, register i -> dim 16 tt + 4 g + i.
    const float lsum = xsum32(xsum16(l_run));
    if (!row_ok) return;
    const float lsum_s = sum_with_sink(p, qhead, m_ref, lsum);
    const float inv = lsum_s > 0.0f ? p.v_scale / lsum_s : 0.0f;
    const int64_t orow_i = static_cast<int64_t>(q_start + tok) * p.Hq + qhead;
    if (p.lse != nullptr && g4l == 0) p.lse[orow_i] = lse_from_log2(m_ref, lsum);
    OutS* orow = out + orow_i * DP;
#pragma unroll
    for (int tt = 0; tt < C::NT; ++tt) {
      const int d = 16 * tt + 4 * g4l;
      const float v0 = oacc[tt][0] * inv, v1 = oacc[tt][1] * inv;
      const float v2 = oacc[tt][2] * inv, v3 = oacc[tt][3] * inv;
      if constexpr (sizeof(OutS) == 4) {
        *reinterpret_cast<float4*>(orow + d) = make_float4(v0, v1, v2, v3);
      } else {
        *reinterpret_cast<uint2*>(orow + d) =
            make_uint2(static_cast<uint32_t>(f32_to_bf16_bits(v0)) |
                           (static_cast<uint32_t>(f32_to_bf16_bits(v1)) << 16),
                       static_cast<uint32_t>(f32_to_bf16_bits(v2)) |
                           (static_cast<uint32_t>(f32_to_bf16_bits(v3)) << 16));
      }
    }
    return;
  } else {
    // ---- output: lane l, block tt, register i -> dim 32 tt + 8 (i / 4) + 4 half + i % 4.
    const float lsum = xsum32(l_run);
    if (!row_ok) return;
    const float lsum_s = sum_with_sink(p, qhead, m_ref, lsum);
    const float inv = lsum_s > 0.0f ? p.v_scale / lsum_s : 0.0f;
    const int64_t orow_i = static_cast<int64_t>(q_start + tok) * p.Hq + qhead;
    if (p.lse != nullptr && half == 0) p.lse[orow_i] = lse_from_log2(m_ref, lsum);
    OutS* orow = out + orow_i * DP;
#pragma unroll
    for (int tt = 0; tt < C::NT; ++tt)
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        const int d = 32 * tt + 8 * g4 + 4 * half;
        const float v0 = oacc[tt][4 * g4 + 0] * inv, v1 = oacc[tt][4 * g4 + 1] * inv;
        const float v2 = oacc[tt][4 * g4 + 2] * inv, v3 = oacc[tt][4 * g4 + 3] * inv;
        if constexpr (sizeof(OutS) == 4) {
          *reinterpret_cast<float4*>(orow + d) = make_float4(v0, v1, v2, v3);
        } else {
          *reinterpret_cast<uint2*>(orow + d) =
              make_uint2(static_cast<uint32_t>(f32_to_bf16_bits(v0)) |
                             (static_cast<uint32_t>(f32_to_bf16_bits(v1)) << 16),
                         static_cast<uint32_t>(f32_to_bf16_bits(v2)) |
                             (static_cast<uint32_t>(f32_to_bf16_bits(v3)) << 16));
        }
      }
  }
}
