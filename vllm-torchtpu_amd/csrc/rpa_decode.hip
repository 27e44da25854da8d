// Decode attention (q_len <= dq query tokens per sequence) for gfx950.
//
// Bandwidth-bound GQA split-K with a stream-K split (rpa_plan.h): the tiles
// of every (decode sequence, kv head) pair lie on one line, pair-major, and
// each wavefront of the persistent grid walks an equal contiguous stretch of
// it, so every wavefront streams the same number of bytes.  A pair inside one
// wavefront's stretch gets its output rows directly; a pair cut between
// wavefronts gets one un-normalised partial (m, l, O) per wavefront, which the
// finish kernel (rpa_finish.hip), launched next on the same stream, merges.
// The kernel boundary orders the partial writes before the merge reads, so no
// wavefront ever waits for another.  Concurrent wavefronts sit at the same
// offset of consecutive pairs -- the kv heads of the same tokens, adjacent
// bytes of the same pages.
//
// New tokens.  The keys at positions [kv_len - q_len, kv_len) of a decode
// sequence are its own new tokens: unless skip_kv_update, the wavefront that
// owns a tile holding some of them reads them from the k/v inputs (patched
// into its LDS tile) and writes their K|V bytes for that kv head into the
// cache pages (kernel.py:154-166).
//
// Memory path.  Each global load instruction moves 8 tokens x 128 bytes of
// one kv head (whole cache lines); a tile is 16 KiB of one head's K|V bytes,
// and each wavefront keeps two tiles in flight in registers (ping-pong
// buffers, one loading while the other is consumed).  K goes through a padded
// LDS tile into the MFMA operand layout; V is stored row-major and read back
// with ds_read_b64_tr_b16, which returns four tokens of one head dim per lane
// -- exactly the V^T operand of v_mfma_f32_16x16x16_bf16 -- so no register
// transpose is needed.
//
// Per 16-token group of a tile a wavefront computes
//   S^T[token, row] = K[token, :] . Q^T[:, row]      (16x16x32, A = K, B = Q^T)
//   O^T[dim, row]  += V^T[dim, token] . P^T[token, row] (16x16x16, A = V^T, B = P^T)
// where the 16 MFMA columns ("rows") are the (token, q head) pairs of this kv
// head: column n is token n / qpk of the sequence's q_len (spec-verify windows
// of several tokens, batched_rpa/wrapper.py:549 decode_query_size) and q head
// n % qpk; columns past q_len * qpk repeat the last token and are not output.  Lane l owns row l % 16 in all
// three accumulators, so the online softmax needs two cross-lane shuffles per
// tile and P feeds the PV product with no shuffle.
//
// Semantics match ref_ragged_paged_attention (kernel.py:185-209):
// s_j = (q . k_j) * sm_scale * k_scale * q_scale, optional soft cap; token i
// of q_len at position p_i = kv_len - q_len + i attends keys j <= p_i (all
// j < kv_len without the causal mask) and j > p_i - W under a causal window;
// softmax, out = P . V * v_scale.  P is rounded to bf16 for the PV product, as the
// Pallas kernel does (kernel.py:553); everything else accumulates in fp32.
#include "rpa_common.h"
#include "rpa_internal.h"
#include "rpa_plan.h"

namespace rpa {

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kWaves = kPlanWaves;
constexpr int kThreads = kPlanThreads;
constexpr float kLog2e = 1.4426950408889634f;

// ---------------------------------------------------------------------------
// KV element loaders producing bf16 MFMA operands.
// ---------------------------------------------------------------------------
struct KvBF16 {
  using storage = uint16_t;
  using raw_t = uint4;  // 8 elements as loaded
  static __device__ __forceinline__ raw_t zero() { return make_uint4(0u, 0u, 0u, 0u); }
  // 8 consecutive elements starting at p (16-byte aligned).
  static __device__ __forceinline__ raw_t load8(const storage* p) {
    return *reinterpret_cast<const uint4*>(p);
  }
  static __device__ __forceinline__ uint4 to_bf16(raw_t r) { return r; }
};

template <bool kE5M2>
struct KvFP8 {
  static constexpr bool kIsE5M2 = kE5M2;
  using storage = uint8_t;
  using raw_t = uint2;  // 8 fp8 elements as loaded
  static __device__ __forceinline__ raw_t zero() { return make_uint2(0u, 0u); }
  static __device__ __forceinline__ raw_t load8(const storage* p) {
    return *reinterpret_cast<const uint2*>(p);
  }
  static __device__ __forceinline__ uint4 to_bf16(raw_t raw) {
    const uint2 a = fp8x4_to_bf16x4<kE5M2>(raw.x), b = fp8x4_to_bf16x4<kE5M2>(raw.y);
    return make_uint4(a.x, a.y, b.x, b.y);
  }
};

__device__ __forceinline__ bf16x8_t as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8_t, v); }

// Two floats -> packed bf16 pair, round to nearest even (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{lo, hi}, bf16x2_t));
}


// Store one 16-byte load piece (raw KV bytes) as bf16 into an LDS row at
// element offset e0.
template <typename KV>
__device__ __forceinline__ void store_piece_bf16(unsigned char* row, int e0, uint4 raw) {
  if constexpr (sizeof(typename KV::storage) == 2) {
    *reinterpret_cast<uint4*>(row + 2 * e0) = raw;
  } else {
    const uint4 a = KV::to_bf16(make_uint2(raw.x, raw.y));
    const uint4 b = KV::to_bf16(make_uint2(raw.z, raw.w));
    *reinterpret_cast<uint4*>(row + 2 * e0) = a;
    *reinterpret_cast<uint4*>(row + 2 * e0 + 16) = b;
  }
}


typedef short v4i16 __attribute__((ext_vector_type(4)));

template <typename KV, int DP>
struct DecodeCfg {
  static constexpr int EB = sizeof(typename KV::storage);   // KV element bytes
  static constexpr int HB = 2 * DP * EB;                    // one head of a token: K then V
  static constexpr int NPART = HB / 128;                    // 128-byte parts per head
  static constexpr int TT = decode_tile_tokens(DP, EB);    // tokens per tile
  static constexpr int NOCT = TT / 8;                       // 8-token octets per tile
  static constexpr int NG = TT / 16;                        // 16-token MFMA groups
  static constexpr int KS = DP * 2 + 16;                    // LDS K row stride (bytes)
  static constexpr int VS = DP * 2 + 32;                    // LDS V row stride (bytes)
  static constexpr int WAVE_LDS = TT * VS;                  // per wavefront (K, then V)
  static_assert(TT >= 16 && TT % 16 == 0, "a tile holds whole 16-token groups");
  static_assert(NOCT * NPART == 16, "16 loads per lane per tile");
};

// One tile of the wavefront's walk (wavefront-uniform).
struct TileInfo {
  int32_t g;    // position on the work line; >= the stretch's end => none
  int32_t s;    // sequence
  int32_t h;    // kv head
  int32_t lt;   // tile index within the pair
  int32_t lt0;  // first tile of this wavefront's segment of the pair
  int32_t nt;   // tiles of the pair
  int32_t lo;   // first key of the sequence's range
  int32_t hi;   // end of the sequence's range (kv_len)
  int32_t ql;   // q_len of the sequence (its new tokens are keys [hi - ql, hi))
};

__device__ __forceinline__ int32_t uni(int32_t x) { return __builtin_amdgcn_readfirstlane(x); }

// LDS tile rows of stride RS bytes (bf16).  Rows [r0, r1) hold new tokens:
// row r0 + k is replaced by the k/v input row src + k * src_stride.
template <typename KV, int DP>
__device__ __forceinline__ void patch_rows(unsigned char* buf, int rs, int32_t r0, int32_t r1,
                                           const typename KV::storage* src, int64_t src_stride,
                                           int32_t D, int lane) {
  constexpr int PIECES = DP / 8;  // 16-byte bf16 pieces per row
  for (int32_t i = lane; i < (r1 - r0) * PIECES; i += 64) {
    const int32_t k = i / PIECES, e0 = (i - k * PIECES) * 8;
    uint4 v = make_uint4(0u, 0u, 0u, 0u);
    if (e0 < D) v = KV::to_bf16(KV::load8(src + k * src_stride + e0));  // D % 8 == 0
    *reinterpret_cast<uint4*>(buf + (r0 + k) * rs + 2 * e0) = v;
  }
}

// Rows [r0, TT) of a sequence's last tile (keys >= kv_len; the loads clamped
// them to copies of key kv_len - 1) are zeroed, so that their P = 0 never
// meets a NaN.
template <int DP, int TT>
__device__ __forceinline__ void zero_rows(unsigned char* buf, int rs, int32_t r0, int lane) {
  constexpr int PIECES = DP / 8;
  for (int32_t i = lane; i < (TT - r0) * PIECES; i += 64) {
    const int32_t r = r0 + i / PIECES, pc = i % PIECES;
    *reinterpret_cast<uint4*>(buf + r * rs + 16 * pc) = make_uint4(0u, 0u, 0u, 0u);
  }
}

// Cache write of a one-token decode row's new token (position j, input row
// tq) for kv head h (kernel.py:154-166): combined heads 2h (K) and 2h + 1
// (V), head dims >= D zero; the wavefront of the last kv head also zeroes the
// padding heads [2 Hkv, Kx2).
template <typename KV, int DP>
__device__ __forceinline__ void write_new_token(const Params& p, typename KV::storage* cache,
                                                const int32_t* page_indices,
                                                const typename KV::storage* keys,
                                                const typename KV::storage* values, int32_t s,
                                                int32_t h, int32_t j, int32_t tq, int lane) {
  using E = typename KV::storage;
  constexpr int EPP = 8 / sizeof(E);             // elements per 8-byte piece
  constexpr int PIECES = DP / EPP;               // pieces per head chunk
  const int32_t pg = page_indices[static_cast<int64_t>(s) * p.pps + page_of(p, j)];
  if (pg < 0 || pg >= p.P) return;
  E* rec = cache + (static_cast<int64_t>(pg) * p.ps + slot_of(p, j)) * p.rec;
  const int64_t src = (static_cast<int64_t>(tq) * p.Hkv + h) * p.D;
  for (int i = lane; i < 2 * PIECES; i += 64) {
    const int c = i / PIECES, e0 = (i % PIECES) * EPP;
    uint2 v = make_uint2(0u, 0u);
    if (e0 < p.D) v = *reinterpret_cast<const uint2*>((c ? values : keys) + src + e0);
    *reinterpret_cast<uint2*>(rec + static_cast<int64_t>(2 * h + c) * DP + e0) = v;
  }
  if (h == p.Hkv - 1) {
    const int32_t npad = (p.Kx2 - 2 * p.Hkv) * PIECES;
    for (int i = lane; i < npad; i += 64)
      *reinterpret_cast<uint2*>(rec + static_cast<int64_t>(2 * p.Hkv) * DP + i * EPP) =
          make_uint2(0u, 0u);
  }
}

// The same from registers (unpadded head_dim): page id pg of position j, and
// lane l < 2 DP EB / 16 holding bytes [16 l, 16 l + 16) of the token's K|V
// chunk of kv head h (K then V, as in the record).
template <typename KV, int DP>
__device__ __forceinline__ void write_new_token_regs(const Params& p, typename KV::storage* cache,
                                                     int32_t pg, int32_t h, int32_t j, uint4 v,
                                                     int lane) {
  using E = typename KV::storage;
  constexpr int EPP = 8 / sizeof(E);  // elements per 8-byte piece
  constexpr int PIECES = DP / EPP;    // pieces per head chunk
  constexpr int NEWP = 2 * DP * sizeof(E) / 16;
  if (pg < 0 || pg >= p.P) return;
  E* rec = cache + (static_cast<int64_t>(pg) * p.ps + slot_of(p, j)) * p.rec;
  if (lane < NEWP)
    *reinterpret_cast<uint4*>(reinterpret_cast<unsigned char*>(rec + static_cast<int64_t>(2 * h) * DP) +
                              16 * lane) = v;
  if (h == p.Hkv - 1) {
    const int32_t npad = (p.Kx2 - 2 * p.Hkv) * PIECES;
    for (int i = lane; i < npad; i += 64)
      *reinterpret_cast<uint2*>(rec + static_cast<int64_t>(2 * p.Hkv) * DP + i * EPP) =
          make_uint2(0u, 0u);
  }
}

// The same for a group's new tokens j0 <= j < j1 (input rows
// tq0 + j - j0) for kv head h (kernel.py:154-166): combined heads 2h (K) and
// 2h + 1 (V), head dims >= D zero; the wavefront of the last kv head also
// zeroes the padding heads [2 Hkv, Kx2).
template <typename KV, int DP>
__device__ __forceinline__ void write_new_tokens(const Params& p, typename KV::storage* cache,
                                                 const int32_t* page_indices,
                                                 const typename KV::storage* keys,
                                                 const typename KV::storage* values, int32_t s,
                                                 int32_t h, int32_t j0, int32_t j1, int32_t tq0,
                                                 int lane) {
  using E = typename KV::storage;
  constexpr int EPP = 8 / sizeof(E);             // elements per 8-byte piece
  constexpr int PIECES = DP / EPP;               // pieces per head chunk
  const int32_t npad = h == p.Hkv - 1 ? (p.Kx2 - 2 * p.Hkv) * PIECES : 0;
  const int32_t per_tok = 2 * PIECES + npad;
  for (int32_t i = lane; i < (j1 - j0) * per_tok; i += 64) {
    const int32_t k = i / per_tok, r = i - k * per_tok;
    const int32_t j = j0 + k;
    const int32_t pg = page_indices[static_cast<int64_t>(s) * p.pps + page_of(p, j)];
    if (pg < 0 || pg >= p.P) continue;
    E* rec = cache + (static_cast<int64_t>(pg) * p.ps + slot_of(p, j)) * p.rec;
    if (r < 2 * PIECES) {
      const int c = r / PIECES, e0 = (r - c * PIECES) * EPP;
      const int64_t src = (static_cast<int64_t>(tq0 + k) * p.Hkv + h) * p.D;
      uint2 v = make_uint2(0u, 0u);
      if (e0 < p.D) v = *reinterpret_cast<const uint2*>((c ? values : keys) + src + e0);
      *reinterpret_cast<uint2*>(rec + static_cast<int64_t>(2 * h + c) * DP + e0) = v;
    } else {
      *reinterpret_cast<uint2*>(rec + static_cast<int64_t>(2 * p.Hkv) * DP +
                                (r - 2 * PIECES) * EPP) = make_uint2(0u, 0u);
    }
  }
}

// ---------------------------------------------------------------------------
// The decode kernel (one wavefront per SIMD, two tile buffers in flight).
// ---------------------------------------------------------------------------
// MULTI: groups of several tokens (dq > 1); without it every group is one
// token and the per-token bookkeeping folds away.
template <typename KV, int DP, typename OutS, bool FULL_D, bool MULTI>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 1)))
decode_kernel(Params p, const uint16_t* __restrict__ q, const typename KV::storage* __restrict__ keys,
              const typename KV::storage* __restrict__ values,
              typename KV::storage* __restrict__ cache, const int32_t* __restrict__ kv_lens,
              const int32_t* __restrict__ page_indices, const int32_t* __restrict__ cu,
              const int32_t* __restrict__ dist, OutS* __restrict__ out,
              float* __restrict__ part_o, float* __restrict__ part_ml,
              int32_t* __restrict__ plan_ws) {
  using C = DecodeCfg<KV, DP>;
  constexpr int TT = C::TT, NOCT = C::NOCT, NPART = C::NPART, NG = C::NG;
  constexpr int KP = NPART / 2;        // K parts (then V parts)
  constexpr int EPP = 128 / C::EB;     // elements per part
  constexpr int KK = DP / 32;          // MFMA k-steps over head_dim
  constexpr int NT = DP / 16;          // PV output tiles over head_dim

  __shared__ __align__(16) unsigned char smem[kWaves * C::WAVE_LDS];
  __shared__ PlanCore L;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int g = lane >> 4;   // MFMA lane group
  const int n = lane & 15;   // MFMA column: q row within the kv head's group
  const int tl = lane >> 3;  // load shape: token within the octet
  const int ol = lane & 7;   // load shape: 16-byte column within a 128-byte part

  const Plan pl = build_plan(p, kv_lens, cu, dist, TT, true, L, nullptr);
  const int32_t gw = static_cast<int32_t>(blockIdx.x) * kWaves + wave;
  // This wavefront's stretch [g_begin, g_end) of the work line.
  const int64_t g_begin64 = static_cast<int64_t>(gw) * pl.tpw;
  if (g_begin64 >= pl.total_tiles) {  // no barrier follows the plan
    publish_plan(p, pl, L, plan_ws);
    return;
  }
  const int32_t g_begin = static_cast<int32_t>(g_begin64);
  const int32_t g_end = min(g_begin + pl.tpw, pl.total_tiles);
  unsigned char* buf = smem + wave * C::WAVE_LDS;
  const int32_t rp = decode_slot_rows(p.qpk * p.dq);
  // Column n: token n_tok of the group (clamped to the sequence's q_len), q
  // head n_head of the kv head.
  const int32_t n_tok = MULTI ? n / p.qpk : 0;
  const int32_t max_tok = p.pps * p.ps - 1;
  const bool write_kv = p.skip_kv_update == 0;

  // ---- walk of the stretch (wavefront-uniform) -----------------------------
  // Tile g: sequence s with Hkv * base[s] <= g < Hkv * base[s + 1] (the
  // largest such s is the non-empty one), then head and tile within it.
  auto locate = [&](int32_t g) __attribute__((always_inline)) {
    TileInfo ti;
    ti.g = g;
    if (g >= g_end) return ti;
    ti.s = uni(find_prefix(L.base, pl.num_seqs, g / p.Hkv));
    const int32_t dkv = uni(L.dkv[ti.s]);
    ti.nt = uni(L.base[ti.s + 1] - L.base[ti.s]);
    const int32_t r = g - p.Hkv * L.base[ti.s];
    ti.h = uni(r / ti.nt);
    ti.lt = uni(r - ti.h * ti.nt);
    ti.lt0 = ti.lt;
    ti.ql = MULTI ? uni(max(L.ql[ti.s], 1)) : 1;
    int32_t lo, hi;
    decode_range(p, dkv, ti.ql, &lo, &hi);
    ti.lo = uni(lo);
    ti.hi = uni(hi);
    return ti;
  };
  auto advance = [&](const TileInfo& c) __attribute__((always_inline)) {
    TileInfo ti = c;
    ti.g = c.g + 1;
    if (ti.g >= g_end) return ti;
    if (c.lt + 1 < c.nt) {
      ti.lt = c.lt + 1;
    } else if (c.h + 1 < p.Hkv) {
      ti.h = c.h + 1;
      ti.lt = 0;
      ti.lt0 = 0;
    } else {
      ti = locate(ti.g);
    }
    return ti;
  };

  // ---- addressing ------------------------------------------------------------
  // Lane (tl, ol) loads token base + 8o + tl of octet o (clamped into the key
  // range, so every address is inside the cache).  Its page id is a per-lane
  // vector load issued one pipeline step ahead of the tile load that uses it.
  auto clamp_tok = [&](const TileInfo& ti, int32_t j) __attribute__((always_inline)) -> int32_t {
    return min(max(min(j, ti.hi - 1), 0), max_tok);
  };
  struct Pages {
    int32_t pg[NOCT];
  };
  // Aligned tiles (power-of-two page size >= 8, tile start a multiple of
  // min(page size, TT)): each 8-token octet lies in one page, so its page id
  // and record address are wavefront-uniform (scalar loads and arithmetic;
  // the tile loads take a uniform base plus a per-lane 32-bit offset).  Lanes
  // past the key range then read other slots of an allocated page (page
  // index and page id clamped into the table and the cache), whose scores
  // the last tile's mask and zeroed V rows discard.  Other tiles use per-lane
  // tokens clamped into the range.
  auto aligned_tile = [&](int32_t base) __attribute__((always_inline)) -> bool {
    return p.ps_shift >= 3 && (base & (min(p.ps, TT) - 1)) == 0;
  };
  const int32_t lane_off = tl * static_cast<int32_t>(p.rec * C::EB) + 16 * ol;
  auto pages_of = [&](const TileInfo& ti, Pages& pp) __attribute__((always_inline)) {
    const int32_t sq = min(max(ti.s, 0), p.S - 1);
    const int32_t* ptab = page_indices + static_cast<int64_t>(sq) * p.pps;
    const int32_t base = ti.lo + ti.lt * TT;
    if (aligned_tile(base)) {
#pragma unroll
      for (int o = 0; o < NOCT; ++o)
        pp.pg[o] = ptab[min((base + 8 * o) >> p.ps_shift, p.pps - 1)];
    } else {
#pragma unroll
      for (int o = 0; o < NOCT; ++o)
        pp.pg[o] = ptab[page_of(p, clamp_tok(ti, base + 8 * o + tl))];
    }
  };
  // Tile loads: octet o, part pt -> bytes [128pt + 16ol, +16) of the head's
  // K|V chunk of that token.
  auto load_tile = [&](const TileInfo& ti, const Pages& pp, uint4 (*rb)[NPART])
                       __attribute__((always_inline)) {
    const int32_t base = ti.lo + ti.lt * TT;
    if (aligned_tile(base)) {
#pragma unroll
      for (int o = 0; o < NOCT; ++o) {
        const int32_t pg = min(max(uni(pp.pg[o]), 0), p.P - 1);
        const unsigned char* rec = reinterpret_cast<const unsigned char*>(
            cache + (static_cast<int64_t>(pg) * p.ps + ((base + 8 * o) & (p.ps - 1))) * p.rec +
            static_cast<int64_t>(2 * ti.h) * DP);
#pragma unroll
        for (int pt = 0; pt < NPART; ++pt)
          rb[o][pt] = *reinterpret_cast<const uint4*>(rec + lane_off + 128 * pt);
      }
    } else {
#pragma unroll
      for (int o = 0; o < NOCT; ++o) {
        const int32_t c = clamp_tok(ti, base + 8 * o + tl);
        const int32_t pg = min(max(pp.pg[o], 0), p.P - 1);
        const unsigned char* rec = reinterpret_cast<const unsigned char*>(
            cache + (static_cast<int64_t>(pg) * p.ps + slot_of(p, c)) * p.rec +
            static_cast<int64_t>(2 * ti.h) * DP);
#pragma unroll
        for (int pt = 0; pt < NPART; ++pt)
          rb[o][pt] = *reinterpret_cast<const uint4*>(rec + 128 * pt + 16 * ol);
      }
    }
  };
  // Q^T operand of (s, h): row n -> q head h*qpk + (n % qpk); dims 8g + 32kk
  // (clamped into the row; dims >= head_dim are zeroed where they are used).
  auto load_q = [&](const TileInfo& ti, uint4* qv) __attribute__((always_inline)) {
    const int32_t qh = ti.h * p.qpk + (n % p.qpk);
    const int32_t tq = L.tq[min(max(ti.s, 0), p.S - 1)] + (MULTI ? min(n_tok, ti.ql - 1) : 0);
    const uint16_t* qrow = q + (static_cast<int64_t>(tq) * p.Hq + qh) * p.D;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      const int d0 = FULL_D ? 8 * g + 32 * kk : min(8 * g + 32 * kk, p.D - 8);
      qv[kk] = *reinterpret_cast<const uint4*>(qrow + d0);
    }
  };

  // New token of a one-token group (kernel.py:154-166, :634-641): its K|V
  // bytes (HB = 2 * DP * EB, 16 bytes per lane for lanes < HB / 16: K, then
  // V) and its page id, loaded with the pair's last tile one pipeline step
  // ahead, so that the LDS patch and the cache write of the tile's owner
  // wait on no load.  Unpadded head_dim only (the input rows are the record's
  // chunks).
  constexpr bool kPrefetchNew = !MULTI && FULL_D;
  constexpr int NEWP = C::HB / 16;  // 16-byte pieces of the new token's K|V
  static_assert(NEWP <= 64, "one piece per lane");
  struct NewTok {
    uint4 v;
    int32_t pg;
  };
  auto load_new = [&](const TileInfo& ti, NewTok& nt) __attribute__((always_inline)) {
    if constexpr (kPrefetchNew) {
      if (write_kv && ti.lt + 1 == ti.nt) {
        const int32_t sq = min(max(ti.s, 0), p.S - 1);
        const int32_t j = ti.hi - 1;
        nt.pg = page_indices[static_cast<int64_t>(sq) * p.pps + page_of(p, min(max(j, 0), max_tok))];
        if (lane < NEWP) {
          const int c = lane / (NEWP / 2);
          const int64_t row = (static_cast<int64_t>(L.tq[sq]) * p.Hkv + ti.h) * DP;
          const unsigned char* src = reinterpret_cast<const unsigned char*>((c ? values : keys) + row);
          nt.v = *reinterpret_cast<const uint4*>(src + 16 * (lane - c * (NEWP / 2)));
        }
      }
    }
  };

  // ---- pipeline ----------------------------------------------------------------
  TileInfo cur = locate(g_begin);
  uint4 qbuf[2][KK];
  uint4 bufr[2][NOCT][NPART];
  Pages pbuf[2];
  NewTok nbuf[2];
  pages_of(cur, pbuf[0]);
  // The plan's stores go out while the first page ids are in flight.
  publish_plan(p, pl, L, plan_ws);
  load_tile(cur, pbuf[0], bufr[0]);
  load_q(cur, qbuf[0]);
  load_new(cur, nbuf[0]);
  TileInfo nxt = advance(cur);
  pages_of(nxt.g < g_end ? nxt : cur, pbuf[0]);

  const SoftCapLog2 capk = soft_cap_log2_consts(p);
  float m_run = -INFINITY;  // per row n, in log2 units
  float l_run = 0.0f;       // this lane's share of the row sum
  f32x4_t oacc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) oacc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // One pipeline step.  Issue, in this order, the page ids of the tile after
  // next (into page buffer NP), the tile `nxt` (into register buffer NB, with
  // page ids CP) and its q operand (NQ); then consume tile `cur` from CB/CQ.
  // A wavefront's last step re-reads its current, cache-resident tile, so
  // every load is unconditional.  All buffers alternate between the two call
  // sites, so no register copy forces an early wait on a prefetch.
  auto step = [&](uint4 (*CB)[NPART], uint4 (*NB)[NPART], const uint4* CQ, uint4* NQ,
                  const NewTok& CN, NewTok& NN,
                  const Pages& CP, Pages& NP) __attribute__((always_inline)) -> bool {
    const bool has_nxt = nxt.g < g_end;
    const TileInfo nn = has_nxt ? advance(nxt) : nxt;
    const TileInfo ldt = has_nxt ? nxt : cur;
    pages_of(nn.g < g_end ? nn : ldt, NP);
    load_tile(ldt, CP, NB);
    load_q(ldt, NQ);
    load_new(ldt, NN);

    const int32_t base = cur.lo + cur.lt * TT;
    const bool last_tile = cur.lt + 1 == cur.nt;
    const int32_t tq_cur = L.tq[cur.s];
    // This tile's rows [pr0, pr1) are new tokens (keys from new0 on).
    const int32_t ql = MULTI ? cur.ql : 1;
    const int32_t new0 = cur.hi - ql;
    int32_t pr0, pr1;
    bool patch;
    if constexpr (MULTI) {
      pr0 = max(new0 - base, 0);
      pr1 = min(cur.hi - base, TT);
      patch = write_kv && pr1 > pr0;
    } else {
      pr0 = cur.hi - 1 - base;
      pr1 = pr0 + 1;
      patch = write_kv && last_tile;
    }
    const int32_t tq_new = tq_cur + base + pr0 - new0;  // input row of row pr0
    const int64_t new_stride = static_cast<int64_t>(p.Hkv) * p.D;
    const typename KV::storage* knew =
        keys + (static_cast<int64_t>(tq_new) * p.Hkv + cur.h) * p.D;
    const typename KV::storage* vnew =
        values + (static_cast<int64_t>(tq_new) * p.Hkv + cur.h) * p.D;
    // Column n's token sits at key position pos; it sees keys [klo, pos].
    const int32_t pos = p.causal ? new0 + (MULTI ? min(n_tok, ql - 1) : 0) : cur.hi - 1;
    const int32_t klo = (p.causal && p.window > 0) ? pos - p.window + 1 : 0;

    // ---- K: registers -> LDS rows (stride KS) -> MFMA A operand.
    wave_lds_sync();  // the previous tile's V reads are complete
#pragma unroll
    for (int o = 0; o < NOCT; ++o)
#pragma unroll
      for (int pt = 0; pt < KP; ++pt)
        store_piece_bf16<KV>(buf + (8 * o + tl) * C::KS, pt * EPP + ol * (EPP / 8), CB[o][pt]);
    if (patch) {
      wave_lds_sync();
      if constexpr (kPrefetchNew) {
        if (lane < NEWP / 2) store_piece_bf16<KV>(buf + pr0 * C::KS, lane * (16 / C::EB), CN.v);
      } else {
        patch_rows<KV, DP>(buf, C::KS, pr0, pr1, knew, new_stride, p.D, lane);
      }
    }
    wave_lds_sync();
    f32x4_t sacc[NG];
#pragma unroll
    for (int r = 0; r < NG; ++r) sacc[r] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      const int d0 = 8 * g + 32 * kk;
      uint4 qv = CQ[kk];
      if constexpr (!FULL_D) {
        if (d0 >= p.D) qv = make_uint4(0u, 0u, 0u, 0u);
      }
      const bf16x8_t qop = as_bf16x8(qv);
      uint4 kv[NG];
#pragma unroll
      for (int r = 0; r < NG; ++r)
        kv[r] = *reinterpret_cast<const uint4*>(buf + (16 * r + n) * C::KS + 2 * d0);
#pragma unroll
      for (int r = 0; r < NG; ++r)
        sacc[r] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(kv[r]), qop, sacc[r], 0, 0, 0);
    }

    // ---- scores: reg i of group r -> token base + 16r + 4g + i.
    float sc[4 * NG];
#pragma unroll
    for (int r = 0; r < NG; ++r)
#pragma unroll
      for (int i = 0; i < 4; ++i) sc[4 * r + i] = sacc[r][i];
    if (p.has_cap) {
#pragma unroll
      for (int i = 0; i < 4 * NG; ++i)
        sc[i] = soft_cap_log2(sc[i], capk.a, capk.b);
    } else {
#pragma unroll
      for (int i = 0; i < 4 * NG; ++i) sc[i] *= p.score_scale * kLog2e;
    }
    // Masks: one-token groups only on a pair's last tile (keys past kv_len);
    // multi-token groups per column (causal position and window).
    if (MULTI || base + TT > cur.hi) {
#pragma unroll
      for (int i = 0; i < 4 * NG; ++i) {
        const int32_t j = base + 16 * (i >> 2) + 4 * g + (i & 3);
        if constexpr (MULTI)
          sc[i] = (j <= pos && j >= klo) ? sc[i] : -INFINITY;
        else
          sc[i] = (j < cur.hi) ? sc[i] : -INFINITY;
      }
    }
    float tmax = -INFINITY;
#pragma unroll
    for (int i = 0; i < 4 * NG; ++i) tmax = fmaxf(tmax, sc[i]);
    tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
    // The reference max m_run moves only when some column's max grew by more
    // than 2^kRescaleLog2 (a masked column's -inf never moves it).
    if (__any(tmax > m_run + kRescaleLog2)) {
      const float m_new = fmaxf(m_run, tmax);
      const float alpha =
          (m_run == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(m_run - m_new);
      l_run *= alpha;
#pragma unroll
      for (int t = 0; t < NT; ++t) oacc[t] *= alpha;
      m_run = m_new;
    }
    const float m_use = (m_run == -INFINITY) ? 0.0f : m_run;
    float psum = 0.0f;
#pragma unroll
    for (int i = 0; i < 4 * NG; ++i) {
      sc[i] = __builtin_amdgcn_exp2f(sc[i] - m_use);  // -inf -> 0
      psum += sc[i];
    }
    l_run += psum;

    // ---- V: registers -> LDS rows (stride VS) -> V^T operand via
    // ds_read_b64_tr_b16.  In 16-lane group g, source lane j points at token
    // 16r + 4g + j / 4, dims 16t + 4(j % 4); lane n then holds
    // V[16r + 4g + k][16t + n], k < 4 -- the A operand rows of the PV MFMA.
    wave_lds_sync();  // K reads are complete
#pragma unroll
    for (int o = 0; o < NOCT; ++o)
#pragma unroll
      for (int pt = KP; pt < NPART; ++pt) {
        uint4 vr = CB[o][pt];
        if constexpr (!FULL_D) {
          // dims of this piece: (pt - KP) * EPP + ol * EPP / 8 ...
          if ((pt - KP) * EPP + ol * (EPP / 8) >= p.D) vr = make_uint4(0u, 0u, 0u, 0u);
        }
        store_piece_bf16<KV>(buf + (8 * o + tl) * C::VS, (pt - KP) * EPP + ol * (EPP / 8), vr);
      }
    if (last_tile || patch) {
      wave_lds_sync();
      if (patch) {
        if constexpr (kPrefetchNew) {
          if (lane >= NEWP / 2 && lane < NEWP)
            store_piece_bf16<KV>(buf + pr0 * C::VS, (lane - NEWP / 2) * (16 / C::EB), CN.v);
        } else {
          patch_rows<KV, DP>(buf, C::VS, pr0, pr1, vnew, new_stride, p.D, lane);
        }
      }
      if (last_tile) zero_rows<DP, TT>(buf, C::VS, cur.hi - base, lane);
    }
    wave_lds_sync();
    // V^T operands of group r + 1 are read while group r's MFMAs run.
    auto read_va = [&](int r, v4i16* va) __attribute__((always_inline)) {
      const unsigned char* ra = buf + (16 * r + 4 * g + (n >> 2)) * C::VS + 8 * (n & 3);
#pragma unroll
      for (int t = 0; t < NT; ++t)
        va[t] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) v4i16*)(ra + 32 * t));
    };
    v4i16 va[2][NT];
    read_va(0, va[0]);
#pragma unroll
    for (int r = 0; r < NG; ++r) {
      if (r + 1 < NG) read_va(r + 1, va[(r + 1) & 1]);
      // P^T operand: k-slot k -> token 16r + 4g + k.
      const uint2 pw = make_uint2(pack_bf16x2(sc[4 * r + 0], sc[4 * r + 1]),
                                  pack_bf16x2(sc[4 * r + 2], sc[4 * r + 3]));
      const v4i16 pop = __builtin_bit_cast(v4i16, pw);
#pragma unroll
      for (int t = 0; t < NT; ++t)
        oacc[t] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(va[r & 1][t], pop, oacc[t], 0, 0, 0);
    }

    // ---- new tokens into the cache (owner of the tile that holds them).
    if (patch) {
      if constexpr (MULTI)
        write_new_tokens<KV, DP>(p, cache, page_indices, keys, values, cur.s, cur.h, base + pr0,
                                 base + pr1, tq_new, lane);
      else if constexpr (kPrefetchNew)
        write_new_token_regs<KV, DP>(p, cache, CN.pg, cur.h, cur.hi - 1, CN.v, lane);
      else
        write_new_token<KV, DP>(p, cache, page_indices, keys, values, cur.s, cur.h, cur.hi - 1,
                                tq_cur, lane);
    }

    // ---- end of this wavefront's segment of a pair: the output (the whole
    // pair was this wavefront's) or a partial in slot wavefront + pair.
    if (last_tile || cur.g + 1 >= g_end) {
      float lsum = l_run;
      lsum += __shfl_xor(lsum, 16, 64);
      lsum += __shfl_xor(lsum, 32, 64);
      const int32_t s = cur.s, h = cur.h;
      const int32_t rows = MULTI ? ql * p.qpk : min(p.qpk, 16);  // <= 16
      if (last_tile && cur.lt0 == 0) {
        if (n < rows) {
          const int32_t n_head = MULTI ? n - n_tok * p.qpk : n;
          const float lsum_s = sum_with_sink(p, h * p.qpk + n_head, m_run, lsum);
          const float inv = lsum_s > 0.0f ? p.v_scale / lsum_s : 0.0f;
          const int64_t orow_i =
              static_cast<int64_t>(tq_cur + (MULTI ? n_tok : 0)) * p.Hq + h * p.qpk + n_head;
          if (p.lse != nullptr && g == 0) p.lse[orow_i] = lse_from_log2(m_run, lsum);
          OutS* orow = out + orow_i * p.D;
#pragma unroll
          for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const int d = 16 * t + 4 * g + i;
              if (d < p.D) store_out(orow, d, oacc[t][i] * inv);
            }
        }
      } else if (n < rows) {
        const int64_t slot = static_cast<int64_t>(gw) + static_cast<int64_t>(s) * p.Hkv + h;
        float* po = part_o + (slot * rp + n) * DP;
#pragma unroll
        for (int t = 0; t < NT; ++t)
          *reinterpret_cast<f32x4_t*>(po + 16 * t + 4 * g) = oacc[t];
        if (g == 0)
          *reinterpret_cast<float2*>(part_ml + (slot * rp + n) * 2) = make_float2(m_run, lsum);
      }
      m_run = -INFINITY;
      l_run = 0.0f;
#pragma unroll
      for (int t = 0; t < NT; ++t) oacc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    }

    if (!has_nxt) return false;
    cur = nxt;
    nxt = nn;
    return true;
  };

  while (step(bufr[0], bufr[1], qbuf[0], qbuf[1], nbuf[0], nbuf[1], pbuf[0], pbuf[1]) &&
         step(bufr[1], bufr[0], qbuf[1], qbuf[0], nbuf[1], nbuf[0], pbuf[1], pbuf[0])) {
  }
}

template <typename KV, int DP, typename OutS>
hipError_t launch_typed(const Params& p, const DecodeWorkspace& ws, const void* q, const void* k,
                        const void* v, void* cache, const int32_t* kv_lens,
                        const int32_t* page_indices, const int32_t* cu, const int32_t* dist,
                        void* out, hipStream_t stream) {
  using E = typename KV::storage;
  const dim3 grid(p.decode_waves / kWaves), block(kThreads);
#define RPA_DECODE_LAUNCH(FULL, MULTI)                                                        \
  hipLaunchKernelGGL((decode_kernel<KV, DP, OutS, FULL, MULTI>), grid, block, 0, stream, p,   \
                     static_cast<const uint16_t*>(q), static_cast<const E*>(k),               \
                     static_cast<const E*>(v), static_cast<E*>(cache), kv_lens, page_indices, \
                     cu, dist, static_cast<OutS*>(out), ws.part_o, ws.part_ml, ws.plan)
  const bool full = p.D == DP, multi = p.dq > 1;
  if (full && !multi) RPA_DECODE_LAUNCH(true, false);
  else if (full) RPA_DECODE_LAUNCH(true, true);
  else if (!multi) RPA_DECODE_LAUNCH(false, false);
  else RPA_DECODE_LAUNCH(false, true);
#undef RPA_DECODE_LAUNCH
  return hipGetLastError();
}

template <typename KV, typename OutS>
hipError_t launch_dp(const Params& p, const DecodeWorkspace& ws, const void* q, const void* k,
                     const void* v, void* cache, const int32_t* kv_lens,
                     const int32_t* page_indices, const int32_t* cu, const int32_t* dist,
                     void* out, hipStream_t stream) {
  if (p.Dp == 64) {
    // A 128-byte load part holds K (or V) of one token only for 2-byte elements.
    if constexpr (sizeof(typename KV::storage) == 2)
      return launch_typed<KV, 64, OutS>(p, ws, q, k, v, cache, kv_lens, page_indices, cu, dist, out, stream);
    return hipErrorInvalidValue;
  }
  if (p.Dp == 128)
    return launch_typed<KV, 128, OutS>(p, ws, q, k, v, cache, kv_lens, page_indices, cu, dist, out, stream);
  if (p.Dp == 256)
    return launch_typed<KV, 256, OutS>(p, ws, q, k, v, cache, kv_lens, page_indices, cu, dist, out, stream);
  return hipErrorInvalidValue;
}

template <typename OutS>
hipError_t launch_kv(const Params& p, int kv_dtype, const DecodeWorkspace& ws, const void* q,
                     const void* k, const void* v, void* cache, const int32_t* kv_lens,
                     const int32_t* page_indices, const int32_t* cu, const int32_t* dist,
                     void* out, hipStream_t stream) {
  switch (kv_dtype) {
    case RPA_DTYPE_BF16:
      return launch_dp<KvBF16, OutS>(p, ws, q, k, v, cache, kv_lens, page_indices, cu, dist, out, stream);
    case RPA_DTYPE_FP8_E4M3FN:
      return launch_dp<KvFP8<false>, OutS>(p, ws, q, k, v, cache, kv_lens, page_indices, cu, dist, out, stream);
    case RPA_DTYPE_FP8_E5M2:
      return launch_dp<KvFP8<true>, OutS>(p, ws, q, k, v, cache, kv_lens, page_indices, cu, dist, out, stream);
    default:
      return hipErrorInvalidValue;
  }
}

}  // namespace

bool decode_supported(const Params& p, int q_dtype, int kv_dtype, int out_dtype) {
  if (q_dtype != RPA_DTYPE_BF16) return false;
  if (kv_dtype != RPA_DTYPE_BF16 && kv_dtype != RPA_DTYPE_FP8_E4M3FN &&
      kv_dtype != RPA_DTYPE_FP8_E5M2)
    return false;
  if (out_dtype != RPA_DTYPE_BF16 && out_dtype != RPA_DTYPE_F32) return false;
  if (p.Dp != 64 && p.Dp != 128 && p.Dp != 256) return false;
  if (p.Dp == 64 && kv_dtype != RPA_DTYPE_BF16) return false;
  if (p.D % 8 != 0 || p.qpk > 16) return false;
  if (p.S > kMaxDecodeSeqs) return false;
  // The work line (tiles of every pair) is indexed with 32-bit integers.
  const int64_t tiles = (static_cast<int64_t>(p.pps) * p.ps + 15) / 16;
  if (static_cast<int64_t>(p.S) * p.Hkv * tiles >= (int64_t(1) << 31)) return false;
  return true;
}

int decode_waves(const Params& p, int num_cus) {
  // Persistent grid at the kernel's occupancy: one workgroup of kWaves
  // wavefronts per CU (one wavefront per SIMD).
  (void)p;
  return num_cus * kWaves;
}

// Partial slots: one per (wavefront, pair) segment, indexed wavefront +
// pair (rpa_plan.h), so decode_waves + max_num_seqs * Hkv bound them.
static int64_t decode_slots(const Params& p) {
  return static_cast<int64_t>(p.decode_waves) + static_cast<int64_t>(p.S) * p.Hkv;
}

// Workspace layout: the partials, then the published plan.  Nothing in it
// needs initialising.
size_t decode_workspace_bytes(const Params& p) {
  const int64_t rows = decode_slot_rows(p.qpk * p.dq);
  const int64_t slots = decode_slots(p);
  size_t bytes = 256;
  bytes += static_cast<size_t>(slots) * rows * p.Dp * sizeof(float);  // part_o
  bytes += static_cast<size_t>(slots) * rows * 2 * sizeof(float);     // part_ml
  bytes += static_cast<size_t>(plan_ints(p.S, p.T)) * sizeof(int32_t);  // plan
  return bytes;
}

DecodeWorkspace carve_decode_workspace(const Params& p, void* base) {
  DecodeWorkspace ws;
  const int64_t rows = decode_slot_rows(p.qpk * p.dq);
  ws.slots = decode_slots(p);
  uintptr_t ptr = (reinterpret_cast<uintptr_t>(base) + 255) & ~static_cast<uintptr_t>(255);
  ws.part_o = reinterpret_cast<float*>(ptr);
  ptr += static_cast<size_t>(ws.slots) * rows * p.Dp * sizeof(float);
  ws.part_ml = reinterpret_cast<float*>(ptr);
  ptr += static_cast<size_t>(ws.slots) * rows * 2 * sizeof(float);
  ws.plan = reinterpret_cast<int32_t*>(ptr);
  return ws;
}

hipError_t launch_decode(const Params& p, int kv_dtype, int out_dtype, const DecodeWorkspace& ws,
                         const void* q, const void* k, const void* v, void* cache,
                         const int32_t* kv_lens, const int32_t* page_indices, const int32_t* cu,
                         const int32_t* dist, void* out, hipStream_t stream) {
  if (p.decode_waves <= 0 || p.decode_waves % kWaves != 0) return hipErrorInvalidValue;
  if (out_dtype == RPA_DTYPE_F32)
    return launch_kv<float>(p, kv_dtype, ws, q, k, v, cache, kv_lens, page_indices, cu, dist, out, stream);
  return launch_kv<uint16_t>(p, kv_dtype, ws, q, k, v, cache, kv_lens, page_indices, cu, dist, out, stream);
}

}  // namespace rpa
