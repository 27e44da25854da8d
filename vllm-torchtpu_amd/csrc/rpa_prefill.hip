// Prefill attention (rows of sequences with several query tokens) for gfx950.
//
// MFMA flash attention over the paged cache.  A workgroup (8 wavefronts at
// head_dim 128, 4 at 256) owns one item: 32 q rows per wavefront of one
// sequence and one kv head -- BQ = rows / qpk consecutive query tokens times
// the qpk q heads that share the kv head (GQA packing: the K/V tiles of the
// kv head are read once for all of them).
// Wavefront w owns rows [32w, 32w + 32).  Keys are streamed in 64-key tiles
// (32 at head_dim 256),
// staged through double-buffered LDS as bf16 (fp8 KV converted on the way),
// the next tile's global loads in flight in registers while the current one
// is consumed.
//
// Per tile a wavefront computes, with v_mfma_f32_32x32x16_bf16,
//   S^T[key, row] = K[key, :] . Q^T[:, row]          (A = K from LDS, B = Q^T in registers)
//   O^T[dim, row] += V^T[dim, key] . P^T[key, row]    (A = V^T via ds_read_b64_tr_b16, B = P^T)
// Lane l owns MFMA column l % 32 -- one q row -- in every accumulator, so the
// online softmax needs one cross-lane exchange (lanes l and l ^ 32) per tile
// and P feeds the PV product straight from the S^T accumulator registers.
// The accumulator holds, for lane half c = l / 32, keys 8(i / 4) + 4c + i % 4
// (register i); the PV k-step built from registers 0..7 therefore covers keys
// {0-3, 8-11} (c = 0) and {4-7, 12-15} (c = 1), and the V^T operand is read
// with the same key permutation (two 4-key transposing reads per k-step).
//
// Extra workgroups do the work that follows the decode kernel
// (rpa_finish_items.h), independent of the attention blocks (which read new
// tokens from the k/v inputs, never from the pages being written): the first
// `nfm` workgroups merge the decode partials (short, latency-bound: dispatched
// first), the last `nfw` write the new K/V records of the non-decode rows
// into their pages (bandwidth filler for the tail of the launch).
//
// Semantics (ref_ragged_paged_attention, kernel.py:185-209): row i of
// sequence s sits at position p = kv_len - q_len + i; keys j <= p (and
// j > p - W under a window) with s_j = q . k_j * sm_scale * k_scale * q_scale,
// optional soft cap, softmax, out = P . V * v_scale.  New tokens (positions
// >= kv_len - q_len) are read from the k/v inputs unless skip_kv_update, as
// the Pallas kernel does (kernel.py:634-641); the finish kernel, launched
// after this one, writes them into their pages.  P is rounded to bf16 for
// the PV product (kernel.py:553); everything else accumulates in fp32.
#include <type_traits>

#include "rpa_common.h"
#include "rpa_finish_items.h"
#include "rpa_internal.h"
#include "rpa_plan.h"

namespace rpa {

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef short v4i16 __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;

// KV element types: 8 elements per load piece, converted to 8 bf16.
// Loads through global (address space 1) pointers, as native vectors.
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
struct PKvBF16 {
  using storage = uint16_t;
  static __device__ __forceinline__ uint4 load8g(const __attribute__((address_space(1))) storage* p) {
    const u32x4_t r = *reinterpret_cast<const __attribute__((address_space(1))) u32x4_t*>(p);
    return make_uint4(r.x, r.y, r.z, r.w);
  }
};
template <bool kE5M2>
struct PKvFP8 {
  using storage = uint8_t;
  static __device__ __forceinline__ uint4 load8g(const __attribute__((address_space(1))) storage* p) {
    const u32x2_t r = *reinterpret_cast<const __attribute__((address_space(1))) u32x2_t*>(p);
    const uint2 a = fp8x4_to_bf16x4<kE5M2>(r.x), b = fp8x4_to_bf16x4<kE5M2>(r.y);
    return make_uint4(a.x, a.y, b.x, b.y);
  }
};

// Round-to-nearest-even pair of f32 -> packed bf16 (the hardware conversion).
__device__ __forceinline__ uint32_t pack_bf16x2_rne(float lo, float hi) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  const bf16x2_t r = __builtin_convertvector(f32x2_t{lo, hi}, bf16x2_t);
  return __builtin_bit_cast(uint32_t, r);
}

// Sum of a packed bf16 pair added to acc (v_dot2 with (1, 1)).
__device__ __forceinline__ float sum_bf16x2(uint32_t pair, float acc) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  const bf16x2_t ones = {static_cast<__bf16>(1.0f), static_cast<__bf16>(1.0f)};
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, pair), ones, acc, false);
}

template <int DP>
struct PrefillCfg {
  // head_dim 128: 8 wavefronts (256 q rows), one workgroup per CU with two
  // wavefronts per SIMD -- each K|V tile staged once feeds twice the rows of
  // a 4-wavefront workgroup.  head_dim 256: 4 wavefronts, one per SIMD.
  static constexpr int THREADS = DP <= 128 ? 512 : 256;
  static constexpr int ROWS = 32 * THREADS / 64;   // q rows per item (32 per wavefront)
  static constexpr int BK = DP <= 128 ? 64 : 32;   // keys per tile
  static constexpr int NSB = BK / 32;              // 32-key S^T blocks per tile
  // LDS row strides.  K rows (read 16 bytes per lane, 16 consecutive keys
  // per access) are padded by 16 bytes, 4 banks apart; V rows (read with
  // ds_read_b64_tr_b16: 4 keys x 32 bytes per 16-lane group, two groups 32
  // bytes apart per access) by 64 bytes, which puts the 4 keys 16 banks
  // apart so both groups' 8 rows of 8 banks are disjoint.  A 32-byte pad
  // makes those reads 2-way conflicted.
  static constexpr int KS = 2 * DP + 16;
  static constexpr int VS = 2 * DP + 64;
  static constexpr int BUF = BK * (KS + VS);       // one K|V tile buffer
  static constexpr int PPK = 2 * DP / 8;           // 8-element pieces per key (K then V)
  static constexpr int KPI = THREADS / PPK;        // keys covered per staging step
  static constexpr int PPT = BK / KPI;             // pieces per thread per tile
  static constexpr int KSTEPS = DP / 16;           // QK^T k-steps over head_dim
  static constexpr int NT = DP / 32;               // 32-dim output blocks
  static_assert(THREADS % PPK == 0 && BK % KPI == 0, "whole pieces per thread");
  static_assert(THREADS >= kPlanThreads && 3 * kPlanWaves >= THREADS / 64, "plan scan fits");
  // LDS of the tile buffers, which also hold the block prefix of the
  // attention role and the plan of the finish role (at least that much).
  static constexpr int PLAN_BYTES = static_cast<int>(sizeof(PlanCore) + sizeof(PlanRows));
  static constexpr int SMEM = 2 * BUF > PLAN_BYTES ? 2 * BUF : PLAN_BYTES;
  static_assert(SMEM >= 4 * (kMaxDecodeSeqs + 1), "plan scratch fits the tile buffers");
};

// Page ids of an item's key range kept in LDS (longer ranges read the page
// table directly).
constexpr int kItemPages = 512;

// Which sequences this kernel owns: every sequence with rows, except the
// decode sequences when the decode kernel runs.
__device__ __forceinline__ int32_t prefill_blocks(const Params& p, const int32_t* cu,
                                                  const int32_t* kv_lens, int32_t s, int32_t bq,
                                                  bool decode_on) {
  int32_t kl, ql;
  if (decode_on && is_decode_seq(p, cu, kv_lens, s, &kl, &ql)) return 0;
  const int32_t q_len = cu[s + 1] - cu[s];
  if (q_len <= 0) return 0;
  return (q_len + bq - 1) / bq;
}

// Finish workgroup `fb` of `nfin` (pw wavefronts each) walks the merge items
// (merges) or the write items (!merges) of rpa_finish_items.h, grid-stride
// over the group's wavefronts.  `smem` (the tile buffers, unused here) holds
// the plan when the decode kernel did not publish one.
template <typename E, int DP, typename OutS>
__device__ __forceinline__ void prefill_finish_role(
    const Params& p, unsigned char* smem, const E* __restrict__ keys,
    const E* __restrict__ values, E* __restrict__ cache, const int32_t* __restrict__ kv_lens,
    const int32_t* __restrict__ page_indices, const int32_t* __restrict__ cu,
    const int32_t* __restrict__ dist, OutS* __restrict__ out, const int32_t* __restrict__ plan,
    const float* __restrict__ part_o, const float* __restrict__ part_ml, bool merges,
    int32_t nfin, int32_t fb, int pw) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const bool decode_on = p.decode_waves > 0;
  const PlanView pv = plan_view(plan, p.S);
  const int32_t nw = nfin * pw;
  if (merges) {
    // Bounded by S * Hkv: each item loads the sequence count n with its own
    // plan entries, and the loop ends at the first item past n.
    if (!decode_on) return;
    for (int32_t it = fb * pw + wave; it < p.S * p.Hkv; it += nw)
      if (!finish_merge_item<DP, OutS>(p, pv, it, cu, part_o, part_ml, out)) break;
    return;
  }
  PlanCore& pl_core = *reinterpret_cast<PlanCore*>(smem);
  PlanRows* pl_rows = reinterpret_cast<PlanRows*>(smem + sizeof(PlanCore));
  int32_t n;
  if (decode_on) {
    n = min(max(pv.hdr[0], 0), p.S);
  } else {
    n = build_plan(p, kv_lens, cu, dist, 16, false, pl_core, pl_rows).num_seqs;
  }
  const int32_t total = p.skip_kv_update ? 0 : p.T;
  for (int32_t it = fb * pw + wave; it < total; it += nw)
    finish_write_item<E>(p, decode_on, pv, pl_rows, n, cu, kv_lens, cache, page_indices, keys,
                         values, it, lane);
}

// Two wavefronts per SIMD at head_dim 128 (256 registers per lane), one at 256.
// FULL_D: head_dim == Dp (no zero-padded dims to skip).
template <typename KV, int DP, typename OutS, bool FULL_D>
__global__ void __launch_bounds__(PrefillCfg<DP>::THREADS) __attribute__((amdgpu_waves_per_eu(DP <= 128 ? 2 : 1)))
prefill_kernel(Params p, const uint16_t* __restrict__ q,
               const typename KV::storage* __restrict__ keys,
               const typename KV::storage* __restrict__ values,
               typename KV::storage* __restrict__ cache,
               const int32_t* __restrict__ kv_lens, const int32_t* __restrict__ page_indices,
               const int32_t* __restrict__ cu, const int32_t* __restrict__ dist,
               OutS* __restrict__ out, const int32_t* __restrict__ plan,
               const float* __restrict__ part_o, const float* __restrict__ part_ml,
               int32_t nfm, int32_t nfw) {
  using C = PrefillCfg<DP>;
  using E = typename KV::storage;
  constexpr int BK = C::BK;
  __shared__ __align__(16) unsigned char smem[C::SMEM];
  __shared__ int32_t pages[kItemPages];
  __shared__ int32_t red[3 * kPlanWaves];
  // Key address table, three tiles: [t % 3][key] = {K row, V row}.
  __shared__ __align__(16) uint64_t ktab[3][BK][2];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int col = lane & 31;  // MFMA column: this lane's q row within the wavefront
  const int half = lane >> 5;
  const bool decode_on = p.decode_waves > 0;
  const int32_t bq = C::ROWS / p.qpk;  // query tokens per item
  // ---- finish workgroups: [0, nfm) merge items, the last nfw write items.
  const int32_t blk_id = static_cast<int32_t>(blockIdx.x);
  const int32_t nattn = static_cast<int32_t>(gridDim.x) - nfm - nfw;
  // At head_dim 256 the finish work runs in the finish kernel instead: inlined
  // here it costs the attention loop of that instance about 10% (measured).
  if constexpr (kPrefillFinishRoles<DP>) {
    if (blk_id < nfm || blk_id >= nfm + nattn) {
      const bool merges = blk_id < nfm;
      prefill_finish_role<E, DP, OutS>(p, smem, keys, values, cache, kv_lens, page_indices, cu,
                                       dist, out, plan, part_o, part_ml, merges,
                                       merges ? nfm : nfw, merges ? blk_id : blk_id - nfm - nattn,
                                       C::THREADS / 64);
      return;
    }
  }
  // Attention block index (nfm is a multiple of 8, so bid % 8 and blockIdx.x
  // % 8 -- the XCD the dispatcher picks -- agree).
  const int32_t bid = blk_id - nfm;
  // The decode kernel counted the sequences with non-decode rows.
  if (decode_on && plan[3] == 0) return;

  // ---- item: (block kb over all owned sequences, kv head h).  The block
  // prefix lives in the (not yet used) tile buffers.
  int32_t* blk = reinterpret_cast<int32_t*>(smem);
  const int32_t n = min(num_seqs_of(dist, p.S), kMaxDecodeSeqs);
  for (int32_t s = tid; s < n; s += C::THREADS)
    blk[s] = prefill_blocks(p, cu, kv_lens, s, bq, decode_on);
  __syncthreads();
  block_exclusive_scan(blk, n, red);
  const int32_t total = blk[n];
  const int32_t h = bid % p.Hkv;
  // Later blocks of a sequence attend to more keys: walk blocks from the
  // last one so the longest items start first.
  const int32_t kb_rev = bid / p.Hkv;
  if (kb_rev >= total) return;
  const int32_t kb = total - 1 - kb_rev;
  const int32_t s = find_prefix(blk, n, kb);
  const int32_t b = kb - blk[s];
  const int32_t q_start = cu[s];
  const int32_t q_len = cu[s + 1] - q_start;
  // Rows outside [0, T) are never read or written (metadata out of contract).
  if (q_start < 0 || q_len <= 0 || q_start + q_len > p.T) return;
  const int32_t kv_cap = p.pps * p.ps;
  const int32_t kv_len = min(kv_lens[s], kv_cap);
  const int32_t new_start = kv_len - q_len;
  const bool new_from_input = p.skip_kv_update == 0;
  const int32_t* ptab = page_indices + static_cast<int64_t>(s) * p.pps;

  // Rows of this item: row r -> query token i = b * bq + r / qpk, q head
  // h * qpk + r % qpk; valid when r < bq * qpk and i < q_len.
  const int32_t tok0 = b * bq;
  const int32_t ntok = min(bq, q_len - tok0);
  // Key range of the whole item.
  int32_t lo = 0, hi = kv_len;
  if (p.causal) {
    hi = min(kv_len, new_start + tok0 + ntok);
    if (p.window > 0) lo = max(0, new_start + tok0 - p.window + 1);
  }
  const int32_t ntiles = hi > lo ? (hi - lo + BK - 1) / BK : 0;

  // This lane's row, and the range of keys it attends: [row_lo, row_hi).
  const int32_t r = wave * 32 + col;
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
  // The wavefront's rows span tokens [wt0, wt1]: tiles outside the union of
  // their ranges are skipped, tiles inside the intersection need no mask.
  const bool wave_live = wave * 32 < bq * p.qpk && wave * 32 / p.qpk < ntok;
  const int32_t wt0 = tok0 + min(wave * 32 / p.qpk, ntok - 1);
  const int32_t wt1 = tok0 + min(min(wave * 32 + 31, bq * p.qpk - 1) / p.qpk, ntok - 1);
  int32_t w_lo0, w_hi0, w_lo1, w_hi1;  // ranges of the first and last token
  key_range(wt0, &w_lo0, &w_hi0);
  key_range(wt1, &w_lo1, &w_hi1);

  // ---- page ids of the item's keys into LDS.
  const int32_t pg0 = hi > lo ? page_of(p, lo) : 0;
  const int32_t npg = hi > lo ? page_of(p, hi - 1) - pg0 + 1 : 0;
  const bool lds_pages = npg <= kItemPages;
  if (lds_pages)
    for (int32_t i = tid; i < npg; i += C::THREADS) pages[i] = min(max(ptab[pg0 + i], 0), p.P - 1);
  __syncthreads();  // the plan scratch is dead; the page ids are visible

  // ---- Q^T operand (B of S^T): column = row, k-slots 8 * half .. + 7 of
  // each 16-dim k-step.
  uint4 qop[C::KSTEPS];
  {
    const uint16_t* qrow = q + (static_cast<int64_t>(q_start + tok) * p.Hq + qhead) * p.D;
#pragma unroll
    for (int kk = 0; kk < C::KSTEPS; ++kk) {
      const int d0 = 16 * kk + 8 * half;
      qop[kk] = d0 < p.D ? *reinterpret_cast<const uint4*>(qrow + d0) : make_uint4(0u, 0u, 0u, 0u);
    }
  }

  // ---- tile staging.  The address of every key's K and V row (its cache
  // record, or its k/v input row for this call's new tokens) is computed
  // once per tile by threads 0 .. BK-1, three tiles ahead, into ktab.  Thread
  // tid always moves piece c = tid % PPK (K for c < Dp / 8, else V; elements
  // e0 .. e0 + 7) of keys tid / PPK + KPI * i.  Tile loads are issued two
  // tiles ahead into two register stages.
  auto fill_tab = [&](int32_t t, int slot) __attribute__((always_inline)) {
    if (tid < BK) {
      const int32_t j = min(lo + t * BK + tid, hi - 1);  // past the range: a valid key
      const E* kr;
      const E* vr;
      if (new_from_input && j >= new_start) {
        const int64_t row = min(q_start + (j - new_start), p.T - 1);
        kr = keys + (row * p.Hkv + h) * p.D;
        vr = values + (row * p.Hkv + h) * p.D;
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
  const int pc = tid % C::PPK;
  const int pkey = tid / C::PPK;
  const int isv = pc >= DP / 8;
  const int e0 = (pc - isv * (DP / 8)) * 8;
  const bool piece_live = FULL_D || e0 < p.D;
  // The table holds plain addresses; they are global memory, so the loads are
  // global (not flat) loads and count only against vmcnt -- a flat load would
  // also hold up every LDS wait of the compute phase.
  typedef const __attribute__((address_space(1))) E* GlobalPtr;
  auto load_tile = [&](int32_t t, uint4* stage) __attribute__((always_inline)) {
    const int slot = t % 3;
#pragma unroll
    for (int i = 0; i < C::PPT; ++i) {
      const GlobalPtr src =
          reinterpret_cast<GlobalPtr>(ktab[slot][pkey + C::KPI * i][isv]) + e0;
      uint4 v = make_uint4(0u, 0u, 0u, 0u);
      if (piece_live) v = KV::load8g(src);
      stage[i] = v;
    }
  };
  auto store_tile = [&](unsigned char* buf, const uint4* stage) __attribute__((always_inline)) {
    unsigned char* dst0 = isv ? buf + BK * C::KS + pkey * C::VS + 2 * e0
                              : buf + pkey * C::KS + 2 * e0;
    const int rstride = isv ? C::VS : C::KS;
#pragma unroll
    for (int i = 0; i < C::PPT; ++i)
      *reinterpret_cast<uint4*>(dst0 + C::KPI * i * rstride) = stage[i];
  };

  const float cm = p.has_cap ? 1.0f : p.score_scale * kLog2e;  // multiplier into log2 units
  const SoftCapLog2 capk = soft_cap_log2_consts(p);
  f32x16_t oacc[C::NT];
#pragma unroll
  for (int t = 0; t < C::NT; ++t) oacc[t] = f32x16_t{};
  float m_ref = -INFINITY;  // reference max of the row (log2 units)
  float l_run = 0.0f;       // this lane's share of the row sum (relative to m_ref)

  // Attention of tile t (in LDS buffer t & 1).
  auto compute_tile = [&](int32_t t) __attribute__((always_inline)) {
    const unsigned char* kbuf = smem + (t & 1) * C::BUF;
    const unsigned char* vbuf = kbuf + BK * C::KS;
    const int32_t k0 = lo + t * BK;
    if (!(wave_live && k0 < w_hi1 && k0 + BK > w_lo0)) return;
    {
      // S^T = K . Q^T per 32-key sub-block (A lane l -> key l % 32, dims
      // 16kk + 8 half ..).  With several sub-blocks (head_dim <= 128, two
      // wavefronts per SIMD) each sub-block runs S^T, its softmax, then
      // O^T += V^T . P^T: one 16-VGPR score accumulator is live, which leaves
      // room for the K operand reads to run kRA k-steps ahead of their MFMAs.
      // With one sub-block (head_dim 256) S^T comes first, as a whole.
      constexpr int kRA = 4;  // K operand reads in flight
      f32x16_t sacc1 = f32x16_t{};
      if constexpr (C::NSB == 1) {
#pragma unroll
        for (int kk = 0; kk < C::KSTEPS; ++kk) {
          const uint4 kv = *reinterpret_cast<const uint4*>(
              kbuf + col * C::KS + 2 * (16 * kk + 8 * half));
          sacc1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
              __builtin_bit_cast(bf16x8_t, kv), __builtin_bit_cast(bf16x8_t, qop[kk]), sacc1,
              0, 0, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x100, kRA, 0);
#pragma unroll
        for (int i = 0; i < C::KSTEPS - kRA; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, kRA, 0);
      }
      // Masks only where some row of the wavefront does not see the whole tile.
      const bool need_mask = !(k0 >= w_lo1 && k0 + BK <= w_hi0);
      const int G = lane >> 4, jl = lane & 15;
#pragma unroll
      for (int sb = 0; sb < C::NSB; ++sb) {
        f32x16_t sacc = sacc1;
        if constexpr (C::NSB > 1) {
          // Explicit ring of kRA operands (two wavefronts per SIMD: registers
          // are short, and without it the reads end up one MFMA ahead).
          auto kread = [&](int kk) __attribute__((always_inline)) -> uint4 {
            return *reinterpret_cast<const uint4*>(kbuf + (32 * sb + col) * C::KS +
                                                   2 * (16 * kk + 8 * half));
          };
          uint4 kb[kRA];
#pragma unroll
          for (int i = 0; i < kRA; ++i) kb[i] = kread(i);
#pragma unroll
          for (int kk = 0; kk < C::KSTEPS; ++kk) {
            const uint4 kv = kb[kk % kRA];
            if (kk + kRA < C::KSTEPS) kb[kk % kRA] = kread(kk + kRA);
            sacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                __builtin_bit_cast(bf16x8_t, kv), __builtin_bit_cast(bf16x8_t, qop[kk]), sacc,
                0, 0, 0);
          }
          __builtin_amdgcn_sched_group_barrier(0x100, kRA, 0);
#pragma unroll
          for (int i = 0; i < C::KSTEPS - kRA; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
          }
          __builtin_amdgcn_sched_group_barrier(0x008, kRA, 0);
        }
        // Scores y (raw logits, or soft-capped logits in log2 units); register
        // i -> key k0 + 32 sb + 8(i/4) + 4 half + i%4.
        float y[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          float x = sacc[i];
          if (p.has_cap) x = soft_cap_log2(x, capk.a, capk.b);
          y[i] = x;
        }
        // A non-positive multiplier is applied before masking (the max and
        // the exp argument below assume cme > 0).
        float cme = cm;
        if (!(cm > 0.0f)) {
#pragma unroll
          for (int i = 0; i < 16; ++i) y[i] *= cm;
          cme = 1.0f;
        }
        if (need_mask) {
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const int32_t j = k0 + 32 * sb + 8 * (i >> 2) + 4 * half + (i & 3);
            if (j < row_lo || j >= row_hi) y[i] = -INFINITY;
          }
        }
        float tmax = -INFINITY;
#pragma unroll
        for (int i = 0; i < 16; ++i) tmax = fmaxf(tmax, y[i]);
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
        const float m_tile = tmax * cme;  // -inf stays -inf (cme > 0)
        // Move the reference max only when it grew by more than 2^8 somewhere.
        if (__any(m_tile > m_ref + kRescaleLog2)) {
          const float m_new = fmaxf(m_ref, m_tile);
          const float alpha = (m_ref == -INFINITY) ? 0.0f : exp2f(m_ref - m_new);
          l_run *= alpha;
#pragma unroll
          for (int tt = 0; tt < C::NT; ++tt) oacc[tt] *= alpha;
          m_ref = m_new;
        }
        const float m_use = (m_ref == -INFINITY) ? 0.0f : m_ref;
#pragma unroll
        for (int i = 0; i < 16; ++i)
          y[i] = __builtin_amdgcn_exp2f(fmaf(y[i], cme, -m_use));  // masked: exp2(-inf) = 0
        // P^T operands (bf16, round to nearest even); the row sum adds the
        // same rounded values the PV product uses (v_dot2 with (1, 1)).
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
        // O^T += V^T . P^T.  P^T k-step ks is registers 8 ks .. + 7; the V^T
        // operand: lane l -> dim 32 tt + l % 32, k-slots 0..3 -> keys
        // 32 sb + 16 ks + 4 half + 0..3, slots 4..7 -> the same + 8.
        // ds_read_b64_tr_b16 in 16-lane group G: source lane j points at key
        // kbase + j / 4, dims d0 + 4 (j % 4); lane n receives V[kbase + 0..3][d0 + n].
        constexpr int kP = 2 * C::NT;  // PV MFMAs per sub-block: (ks, tt)
        auto vread = [&](int i) __attribute__((always_inline)) -> uint4 {
          const int ks = i / C::NT, tt = i % C::NT;
          const int key_a = 32 * sb + 16 * ks + 4 * (G >> 1) + (jl >> 2);
          const unsigned char* ra =
              vbuf + key_a * C::VS + 2 * (16 * (G & 1) + 4 * (jl & 3)) + 64 * tt;
          const v4i16 va = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (__attribute__((address_space(3))) v4i16*)ra);
          const v4i16 vb = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (__attribute__((address_space(3))) v4i16*)(ra + 8 * C::VS));
          const uint2 ua = __builtin_bit_cast(uint2, va), ub = __builtin_bit_cast(uint2, vb);
          return make_uint4(ua.x, ua.y, ub.x, ub.y);
        };
        if constexpr (C::NSB > 1) {
          // The V^T operands of MFMA i + 2 are read before MFMA i issues.
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
        } else {
#pragma unroll
          for (int i = 0; i < kP; ++i) {
            const int tt = i % C::NT;
            oacc[tt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                __builtin_bit_cast(bf16x8_t, vread(i)),
                __builtin_bit_cast(bf16x8_t, pops[i / C::NT]), oacc[tt], 0, 0, 0);
          }
        }
        // Schedule: the V^T reads (two per MFMA) run two MFMAs ahead.
        __builtin_amdgcn_sched_group_barrier(0x100, 4, 1);
#pragma unroll
        for (int i = 0; i < kP - 2; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);
          __builtin_amdgcn_sched_group_barrier(0x100, 2, 1);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, 2, 1);
      }
    }
  };

  // ---- pipeline: iteration t issues the loads of tile t + 2 (register
  // stage t & 1) and the address table of tile t + 3, computes tile t, then
  // stores tile t + 1 (stage (t + 1) & 1) into LDS buffer (t + 1) & 1.
  uint4 stage0[C::PPT], stage1[C::PPT];
  // Every slot gets valid addresses (tiles past the end repeat the last
  // one), so the unconditional prefetch below never reads an unset entry.
  if (ntiles > 0)
    for (int i = 0; i < 3; ++i) fill_tab(min(i, ntiles - 1), i);
  __syncthreads();
  if (ntiles > 0) load_tile(0, stage0);
  if (ntiles > 1) load_tile(1, stage1);
  if (ntiles > 0) store_tile(smem, stage0);
  // Every load issued so far (the q operand included) completes here, so no
  // load from before the loop is still pending inside it: otherwise each
  // iteration would wait for all loads -- the prefetched tiles too -- before
  // its first use of the q operand.
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  auto iter = [&](int32_t t, uint4* st_t, uint4* st_t1) __attribute__((always_inline)) {
    // st_t held tile t (already in LDS); it now receives tile t + 2.  The
    // load is unconditional (past the end: a re-read of the last tile, never
    // stored), so the wait before storing st_t1 counts exactly these loads.
    load_tile(min(t + 2, ntiles - 1), st_t);
    // Slot t % 3 was last read by load_tile(t), two barriers ago.
    if (t + 3 < ntiles) fill_tab(t + 3, t % 3);
    compute_tile(t);
    if (t + 1 < ntiles) store_tile(smem + ((t + 1) & 1) * C::BUF, st_t1);
    __syncthreads();
  };
  for (int32_t t = 0; t < ntiles; t += 2) {
    iter(t, stage0, stage1);
    if (t + 1 < ntiles) iter(t + 1, stage1, stage0);
  }

  // ---- output: lane l, block tt, register i -> dim 32tt + 8(i/4) + 4 half + i%4.
  const float lsum = l_run + __shfl_xor(l_run, 32, 64);
  if (!row_ok) return;
  const float lsum_s = sum_with_sink(p, qhead, m_ref, lsum);
  const float inv = lsum_s > 0.0f ? p.v_scale / lsum_s : 0.0f;
  const int64_t orow_i = static_cast<int64_t>(q_start + tok) * p.Hq + qhead;
  // Lanes l and l + 32 hold the same row.
  if (p.lse != nullptr && half == 0) p.lse[orow_i] = lse_from_log2(m_ref, lsum);
  OutS* orow = out + orow_i * p.D;
#pragma unroll
  for (int tt = 0; tt < C::NT; ++tt)
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      const int d = 32 * tt + 8 * g4 + 4 * half;
      if (d >= p.D) continue;
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

#include "rpa_prefill_dma.h"

// The grid below is sized with PrefillCfg's rows per item; the LDS-DMA
// instances must cover the same rows per item.
static_assert(DmaCfg<128>::ROWS == PrefillCfg<128>::ROWS &&
                  DmaCfg<256, 16>::ROWS == PrefillCfg<256>::ROWS,
              "LDS-DMA and register-staged kernels share the item size");

template <typename KV, typename OutS>
hipError_t launch_dp(const Params& p, const void* q, const void* k, const void* v, void* cache,
                     const int32_t* kv_lens, const int32_t* page_indices, const int32_t* cu,
                     const int32_t* dist, void* out, const DecodeWorkspace& ws, int num_cus,
                     hipStream_t stream) {
  using E = typename KV::storage;
  // Upper bound on attention items: every sequence adds at most one partial
  // block.
  const int32_t bq = (p.Dp <= 128 ? PrefillCfg<128>::ROWS : PrefillCfg<256>::ROWS) / p.qpk;
  const int64_t blocks = (static_cast<int64_t>(p.T) + bq - 1) / bq + p.S;
  const int32_t nfm = prefill_merge_blocks(p, num_cus);
  const int32_t nfw = prefill_write_blocks(p, num_cus);
  const int64_t grid = blocks * p.Hkv + nfm + nfw;
  if (grid > 0x7fffffff) return hipErrorInvalidValue;
  const dim3 g(static_cast<uint32_t>(grid));
#define RPA_PREFILL_LAUNCH(DPV, FULL)                                                        \
  hipLaunchKernelGGL((prefill_kernel<KV, DPV, OutS, FULL>), g,                             \
                     dim3(PrefillCfg<DPV>::THREADS), 0, stream, p,                           \
                     static_cast<const uint16_t*>(q), static_cast<const E*>(k),             \
                     static_cast<const E*>(v), static_cast<E*>(cache), kv_lens,             \
                     page_indices, cu, dist, static_cast<OutS*>(out), ws.plan, ws.part_o,    \
                     ws.part_ml, nfm, nfw)
  const bool full = p.D == p.Dp;
  if constexpr (sizeof(E) == 2) {
    // bf16 KV at head_dim 128 and 256: the LDS-DMA kernel (rpa_prefill_dma.h).
    if (prefill_dma_path(p)) {
#define RPA_DMA_LAUNCH16(DPV, CAP, FIX)                                                          \
  hipLaunchKernelGGL((prefill_dma_kernel<DPV, OutS, CAP, FIX, 16>), g,                           \
                     dim3(DmaCfg<DPV, 16>::THREADS), 0, stream, p,                               \
                     static_cast<const uint16_t*>(q), static_cast<const uint16_t*>(k),          \
                     static_cast<const uint16_t*>(v), static_cast<uint16_t*>(cache), kv_lens,   \
                     page_indices, cu, dist, static_cast<OutS*>(out), ws.plan, ws.part_o,       \
                     ws.part_ml, nfm, nfw)
#define RPA_DMA_LAUNCH(DPV, CAP, FIX)                                                            \
  hipLaunchKernelGGL((prefill_dma_kernel<DPV, OutS, CAP, FIX>), g, dim3(DmaCfg<DPV>::THREADS), 0,\
                     stream, p,                                                                  \
                     static_cast<const uint16_t*>(q), static_cast<const uint16_t*>(k),          \
                     static_cast<const uint16_t*>(v), static_cast<uint16_t*>(cache), kv_lens,   \
                     page_indices, cu, dist, static_cast<OutS*>(out), ws.plan, ws.part_o,       \
                     ws.part_ml, nfm, nfw)
      if (p.Dp == 128) {
        if (p.has_cap) RPA_DMA_LAUNCH(128, true, false); else RPA_DMA_LAUNCH(128, false, false);
      } else {
        // Soft-capped logits are bounded: a fixed reference max (no rescale).
        if (p.has_cap && p.cap * kLog2e <= kFixRefMaxLog2) RPA_DMA_LAUNCH16(256, true, true);
        else if (p.has_cap) RPA_DMA_LAUNCH16(256, true, false);
        else RPA_DMA_LAUNCH16(256, false, false);
      }
#undef RPA_DMA_LAUNCH
#undef RPA_DMA_LAUNCH16
      return hipGetLastError();
    }
  }
  if (p.Dp == 64) {
    if (full) RPA_PREFILL_LAUNCH(64, true); else RPA_PREFILL_LAUNCH(64, false);
  } else if (p.Dp == 128) {
    if (full) RPA_PREFILL_LAUNCH(128, true); else RPA_PREFILL_LAUNCH(128, false);
  } else if (p.Dp == 256) {
    if (full) RPA_PREFILL_LAUNCH(256, true); else RPA_PREFILL_LAUNCH(256, false);
  } else {
    return hipErrorInvalidValue;
  }
#undef RPA_PREFILL_LAUNCH
  return hipGetLastError();
}

template <typename OutS>
hipError_t launch_kv(const Params& p, int kv_dtype, const void* q, const void* k, const void* v,
                     void* cache, const int32_t* kv_lens, const int32_t* page_indices,
                     const int32_t* cu, const int32_t* dist, void* out, const DecodeWorkspace& ws,
                     int num_cus, hipStream_t stream) {
  switch (kv_dtype) {
    case RPA_DTYPE_BF16:
      return launch_dp<PKvBF16, OutS>(p, q, k, v, cache, kv_lens, page_indices, cu, dist, out, ws, num_cus, stream);
    case RPA_DTYPE_FP8_E4M3FN:
      return launch_dp<PKvFP8<false>, OutS>(p, q, k, v, cache, kv_lens, page_indices, cu, dist, out, ws, num_cus, stream);
    case RPA_DTYPE_FP8_E5M2:
      return launch_dp<PKvFP8<true>, OutS>(p, q, k, v, cache, kv_lens, page_indices, cu, dist, out, ws, num_cus, stream);
    default:
      return hipErrorInvalidValue;
  }
}

}  // namespace

bool prefill_supported(const Params& p, int q_dtype, int kv_dtype, int out_dtype) {
  if (q_dtype != RPA_DTYPE_BF16) return false;
  if (kv_dtype != RPA_DTYPE_BF16 && kv_dtype != RPA_DTYPE_FP8_E4M3FN &&
      kv_dtype != RPA_DTYPE_FP8_E5M2)
    return false;
  if (out_dtype != RPA_DTYPE_BF16 && out_dtype != RPA_DTYPE_F32) return false;
  if (p.Dp != 64 && p.Dp != 128 && p.Dp != 256) return false;
  // 8-element pieces of q / k / v rows; at least one query token per item.
  if (p.D % 8 != 0 || p.qpk > (p.Dp <= 128 ? PrefillCfg<128>::ROWS : PrefillCfg<256>::ROWS))
    return false;
  if (p.S > kMaxDecodeSeqs) return false;
  return true;
}

// Merge workgroups (front of the grid): one merge item per wavefront for
// every possible pair, at most two per CU (the kernel's occupancy), a
// multiple of 8 so the attention blocks keep their XCD placement.
int prefill_merge_blocks(const Params& p, int num_cus) {
  if (p.decode_waves <= 0 || !prefill_has_finish_roles(p)) return 0;
  int64_t b = (static_cast<int64_t>(p.S) * p.Hkv + 3) / 4;
  b = b > 2 * num_cus ? 2 * num_cus : b;
  return static_cast<int>((b + 7) / 8 * 8);
}

// Write workgroups (end of the grid): about 16 token rows each, at most one
// per CU.  The LDS-DMA kernel needs none: each attention workgroup writes its
// own block's new tokens for its kv head.
int prefill_write_blocks(const Params& p, int num_cus) {
  if (p.skip_kv_update || p.T == 0 || !prefill_has_finish_roles(p) || prefill_dma_path(p))
    return 0;
  int64_t b = (static_cast<int64_t>(p.T) + 15) / 16;
  return static_cast<int>(b > num_cus ? num_cus : b);
}

hipError_t launch_prefill(const Params& p, int kv_dtype, int out_dtype, const void* q,
                          const void* k, const void* v, void* cache, const int32_t* kv_lens,
                          const int32_t* page_indices, const int32_t* cu, const int32_t* dist,
                          void* out, const DecodeWorkspace& ws, int num_cus, hipStream_t stream) {
  if (p.decode_waves > 0 && ws.plan == nullptr) return hipErrorInvalidValue;
  if (out_dtype == RPA_DTYPE_F32)
    return launch_kv<float>(p, kv_dtype, q, k, v, cache, kv_lens, page_indices, cu, dist, out, ws, num_cus, stream);
  return launch_kv<uint16_t>(p, kv_dtype, q, k, v, cache, kv_lens, page_indices, cu, dist, out, ws, num_cus, stream);
}

}  // namespace rpa
