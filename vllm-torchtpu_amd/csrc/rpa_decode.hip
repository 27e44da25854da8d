// Decode attention (one query token per sequence) for gfx950.
//
// Bandwidth-bound GQA split-K.  The key range of every decode sequence is cut
// into units of a few 64-token tiles; the (unit, kv head) work items are
// walked by a persistent grid in grid-stride order, so at any moment the
// wavefronts of the chip stream a compact window of the item list (measured
// on MI355X: ~1.3x the bandwidth of giving each wavefront a long private
// range).  Every unit writes an un-normalised partial (m, l, O) and the last
// wavefront to finish a (sequence, kv head) merges its partials (device-scope
// fences + an arrival counter that the merger resets to zero).  Every
// workgroup derives the same plan from the device-resident metadata, so
// nothing is read back to the host and the call stays graph-capturable.
//
// Memory path.  Each global load instruction moves 8 tokens x 128 bytes of
// one head (whole cache lines: 1.25x the bandwidth of the 16-token x 64-byte
// shape an MFMA operand would load directly).  K goes through a padded LDS tile
// into the MFMA operand layout; V is stored row-major and read back with
// ds_read_b64_tr_b16, which returns four tokens of one head dim per lane --
// exactly half of the V^T operand -- so no register transpose is needed.
//
// Per 64-token tile a wavefront computes, with v_mfma_f32_16x16x32_bf16,
//   S^T[token, row] = K[token, :] . Q^T[:, row]        (A = K tile, B = Q^T)
//   O^T[dim, row]  += V^T[dim, token] . P^T[token, row] (A = V^T,    B = P^T)
// where the 16 MFMA columns ("rows") are the q heads of this kv head,
// replicated when q_heads_per_kv_head < 16.  Lane l owns row l % 16 in all
// three accumulators, so the online softmax needs two cross-lane shuffles per
// tile and P feeds the PV product with no shuffle.
//
// Semantics match ref_ragged_paged_attention (kernel.py:185-209) for
// q_len == 1: s_j = (q . k_j) * sm_scale * k_scale * q_scale, optional soft
// cap, keys j < kv_len (and j >= kv_len - W under a causal window), softmax,
// out = P . V * v_scale.  P is rounded to bf16 for the PV product, as the
// Pallas kernel does (kernel.py:553); everything else accumulates in fp32.
#include "rpa_common.h"
#include "rpa_internal.h"

namespace rpa {

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;
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

// fp8 -> bf16 bits, exact (every e4m3/e5m2 value is representable in bf16).
__device__ __forceinline__ uint32_t e4m3_to_bf16_bits(uint32_t x) {
  const uint32_t sign = (x & 0x80u) << 8;
  const uint32_t mag = x & 0x7fu;
  uint32_t r;
  if (mag == 0x7fu) {
    r = 0x7fc0u;  // NaN
  } else if (mag >= 8u) {
    r = (mag << 4) + (120u << 7);  // normal: exponent rebias 7 -> 127
  } else {
    // subnormal m * 2^-9: exact through f32
    r = __float_as_uint(static_cast<float>(mag) * 0x1p-9f) >> 16;
  }
  return sign | r;
}
__device__ __forceinline__ uint32_t e5m2_to_bf16_bits(uint32_t x) {
  const float f = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(x << 8)));
  const uint32_t u = __float_as_uint(f);
  return ((u & 0x7fffffffu) > 0x7f800000u) ? ((u >> 16) | 0x40u) : (u >> 16);
}

template <bool kE5M2>
struct KvFP8 {
  static constexpr bool kIsE5M2 = kE5M2;
  using storage = uint8_t;
  using raw_t = uint2;  // 8 fp8 elements as loaded
  static __device__ __forceinline__ raw_t zero() { return make_uint2(0u, 0u); }
  static __device__ __forceinline__ raw_t load8(const storage* p) {
    return *reinterpret_cast<const uint2*>(p);
  }
  static __device__ __forceinline__ uint32_t cvt(uint32_t b) {
    return kE5M2 ? e5m2_to_bf16_bits(b) : e4m3_to_bf16_bits(b);
  }
  static __device__ __forceinline__ uint4 to_bf16(raw_t raw) {
    uint32_t w[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      w[i] = cvt((raw.x >> (8 * i)) & 0xffu);
      w[4 + i] = cvt((raw.y >> (8 * i)) & 0xffu);
    }
    return make_uint4(w[0] | (w[1] << 16), w[2] | (w[3] << 16), w[4] | (w[5] << 16),
                      w[6] | (w[7] << 16));
  }
};

__device__ __forceinline__ bf16x8_t as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8_t, v); }

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return static_cast<uint32_t>(f32_to_bf16_bits(lo)) |
         (static_cast<uint32_t>(f32_to_bf16_bits(hi)) << 16);
}

__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// ---------------------------------------------------------------------------
// Work plan, identical in every workgroup.
// ---------------------------------------------------------------------------
struct Plan {
  int32_t num_seqs;
  int32_t tpu;          // tiles per unit
  int32_t total_units;  // (sequence, unit) pairs
};

// Effective key range of a decode row: [lo, hi).
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
__device__ __forceinline__ void block_exclusive_scan(int32_t* a, int32_t n, int32_t* s_red) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int32_t per = (n + kThreads - 1) / kThreads;
  const int32_t s0 = min(n, tid * per), s1 = min(n, s0 + per);
  int32_t local = 0;
  for (int32_t i = s0; i < s1; ++i) local += a[i];
  int32_t x = local;
  for (int o = 1; o < 64; o <<= 1) {
    const int32_t y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  if (lane == 63) s_red[wave] = x;
  __syncthreads();
  int32_t run = x - local;
  for (int w = 0; w < wave; ++w) run += s_red[w];
  for (int32_t i = s0; i < s1; ++i) {
    const int32_t v = a[i];
    a[i] = run;
    run += v;
  }
  if (tid == kThreads - 1) a[n] = run;
  __syncthreads();
}

// s_nt[s]: tiles of sequence s (0 unless it is a decode row); s_units:
// exclusive prefix of units per sequence.  Units hold `tpu` tiles, chosen so
// that the unit count never exceeds max_units (the partial-slot capacity).
__device__ __forceinline__ Plan build_plan(const Params& p, const int32_t* kv_lens, const int32_t* cu,
                           const int32_t* dist, int32_t tile, int32_t max_units, int32_t* s_nt,
                           int32_t* s_units, int32_t* s_kvlen, int32_t* s_tq, int32_t* s_red) {
  Plan pl;
  const int tid = threadIdx.x;
  const int32_t n = num_seqs_of(dist, p.S);
  pl.num_seqs = n;
  int32_t tiles = 0, seqs = 0;
  for (int32_t s = tid; s < n; s += kThreads) {
    int32_t kl, lo, hi, nt = 0;
    if (is_decode_seq(p, cu, kv_lens, s, &kl)) {
      decode_range(p, kl, &lo, &hi);
      nt = (hi - lo + tile - 1) / tile;
      seqs += 1;
    } else {
      kl = 0;
    }
    s_kvlen[s] = kl;
    s_tq[s] = min(max(cu[s], 0), p.T - 1);
    s_nt[s] = nt;
    tiles += nt;
  }
  for (int o = 32; o > 0; o >>= 1) {
    tiles += __shfl_xor(tiles, o, 64);
    seqs += __shfl_xor(seqs, o, 64);
  }
  if ((tid & 63) == 0) {
    s_red[tid >> 6] = tiles;
    s_red[kWaves + (tid >> 6)] = seqs;
  }
  __syncthreads();
  int64_t total_tiles = 0;
  int32_t nseq = 0;
  for (int w = 0; w < kWaves; ++w) {
    total_tiles += s_red[w];
    nseq += s_red[kWaves + w];
  }
  __syncthreads();
  const int64_t budget = max<int64_t>(1, static_cast<int64_t>(max_units) - nseq);
  pl.tpu = static_cast<int32_t>(max<int64_t>(2, (total_tiles + budget - 1) / budget));
  for (int32_t s = tid; s < n; s += kThreads) s_units[s] = (s_nt[s] + pl.tpu - 1) / pl.tpu;
  __syncthreads();
  block_exclusive_scan(s_units, n, s_red);
  pl.total_units = s_units[n];
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

__device__ __forceinline__ int32_t uni(int32_t x) { return __builtin_amdgcn_readfirstlane(x); }

// One tile of the wavefront's item walk (wavefront-uniform).
struct TileInfo {
  int32_t unit;    // item index: (sequence unit) * Hkv + head; >= total => none
  int32_t s;       // sequence
  int32_t h;       // kv head
  int32_t lt;      // tile index within the sequence
  int32_t lt_end;  // end tile of the unit
  int32_t lo;      // first key of the sequence's range
  int32_t hi;      // end of the sequence's range
};

// Tokens per tile: 32 (one 32-token PV step).  Two tiles per wavefront in
// flight (one loading, one in use) keep ~16 MiB of reads outstanding
// chip-wide at head_dim 128 bf16, well above what hides HBM latency.
__host__ __device__ constexpr int decode_tile_tokens(int dp, int kv_bytes) {
  return (void)dp, (void)kv_bytes, 32;
}

template <typename KV, int DP>
struct DecodeCfg {
  static constexpr int EB = sizeof(typename KV::storage);   // KV element bytes
  static constexpr int HB = 2 * DP * EB;                    // one head of a token: K then V
  static constexpr int NPART = HB / 128;                    // 128-byte parts per head
  static constexpr int TT = decode_tile_tokens(DP, EB);    // tokens per tile
  static constexpr int NOCT = TT / 8;                       // 8-token octets per tile
  static constexpr int NG = TT / 16;                        // 16-token MFMA groups
  static constexpr int NU = TT / 32;                        // 32-token PV steps
  static constexpr int KS = DP * 2 + 16;                    // LDS K row stride (bytes)
  static constexpr int VS = DP * 2 + 32;                    // LDS V row stride (bytes)
  static constexpr int WAVE_LDS = TT * VS;                  // per wavefront (K, then V)
  static_assert(TT >= 32 && TT % 32 == 0, "a tile holds whole 32-token PV steps");
};

// Raw 16-byte piece -> bf16 elements (8 for bf16, 16 for fp8 = two uint4).
__device__ __forceinline__ uint32_t cvt_pair_e4m3(uint32_t b2) {
  return e4m3_to_bf16_bits(b2 & 0xffu) | (e4m3_to_bf16_bits((b2 >> 8) & 0xffu) << 16);
}
__device__ __forceinline__ uint32_t cvt_pair_e5m2(uint32_t b2) {
  return e5m2_to_bf16_bits(b2 & 0xffu) | (e5m2_to_bf16_bits((b2 >> 8) & 0xffu) << 16);
}

// Store one 16-byte load piece (raw KV bytes) as bf16 into an LDS row at
// element offset e0.
template <typename KV>
__device__ __forceinline__ void store_piece_bf16(unsigned char* row, int e0, uint4 raw) {
  if constexpr (sizeof(typename KV::storage) == 2) {
    *reinterpret_cast<uint4*>(row + 2 * e0) = raw;
  } else {
    constexpr bool e5 = KV::kIsE5M2;
    const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
    uint32_t o[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      o[2 * i] = e5 ? cvt_pair_e5m2(w[i] & 0xffffu) : cvt_pair_e4m3(w[i] & 0xffffu);
      o[2 * i + 1] = e5 ? cvt_pair_e5m2(w[i] >> 16) : cvt_pair_e4m3(w[i] >> 16);
    }
    *reinterpret_cast<uint4*>(row + 2 * e0) = make_uint4(o[0], o[1], o[2], o[3]);
    *reinterpret_cast<uint4*>(row + 2 * e0 + 16) = make_uint4(o[4], o[5], o[6], o[7]);
  }
}

typedef short v4i16 __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------
// Partials that cross wavefronts.  Each XCD of the chip has its own L2, and a
// device-scope fence is implemented as a writeback plus an invalidation of the
// whole L2 -- far too costly once per work item.  The partials are instead
// written and read with relaxed agent-scope atomic accesses, which are
// coherent across XCDs by themselves (they are issued with the sc1 policy);
// the writer waits for its stores to complete (vmcnt(0)) before its arrival
// increment, and the merger's loads are issued only after the increment that
// made it the last arriver has returned.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void st_coherent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_coherent(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void wait_stores_complete() {
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

// Rows of a partial slot: min(q_heads_per_kv_head, 16) rounded up to a power
// of two (padding rows are never written and never output).
__host__ __device__ constexpr int decode_slot_rows(int qpk) {
  int r = qpk < 16 ? qpk : 16;
  int rp = 1;
  while (rp < r) rp *= 2;
  return rp;
}

// Online combination of a (row max, row sum) pair into (M, L); every
// quantity is in log2 units.  A NaN sum propagates.
__device__ __forceinline__ void ml_combine(float& M, float& L, float m, float l) {
  const float mn = fmaxf(M, m);
  const float a = (M == -INFINITY) ? 0.0f : exp2f(M - mn);
  const float b = (m == -INFINITY) ? 0.0f : exp2f(m - mn);
  L = L * a + l * b;
  M = mn;
}

// Merge the `nunits` partials of one (sequence, kv head) and write its
// output rows [0, rows).  The partial of unit k sits in slot first + k * Hkv:
// RP rows x DP floats of un-normalised O, and RP (m, l) pairs.  One
// wavefront; lane e of load j covers element e + 64 j of a slot, so every
// load is a wave-wide contiguous 256-byte read and row (j * 64 / DP) is the
// same for the whole wavefront.  Loads are batched over UB units so that a
// merge costs a few memory round trips.
template <int DP, int RP, typename OutS>
__device__ __forceinline__ void merge_partials(const Params& p, const float* __restrict__ part_o,
                                            const float* __restrict__ part_ml, int32_t first,
                                            int32_t nunits, int32_t rows, OutS* __restrict__ out,
                                            int64_t orow0) {
  constexpr int NDW = RP * DP / 64;             // dwords per lane per slot
  constexpr int UB = NDW >= 64 ? 1 : 64 / NDW;  // slots per load batch
  const int lane = threadIdx.x & 63;
  const int64_t stride = static_cast<int64_t>(p.Hkv);

  // (M, L) per row over all units.
  float M[RP], L[RP];
#pragma unroll
  for (int r = 0; r < RP; ++r) {
    M[r] = -INFINITY;
    L[r] = 0.0f;
  }
  for (int32_t k = lane; k < nunits; k += 64) {
    const float* ml = part_ml + (first + k * stride) * (2 * RP);
    float mv[RP], lv[RP];
#pragma unroll
    for (int r = 0; r < RP; ++r) {
      mv[r] = ld_coherent(ml + 2 * r);
      lv[r] = ld_coherent(ml + 2 * r + 1);
    }
#pragma unroll
    for (int r = 0; r < RP; ++r) ml_combine(M[r], L[r], mv[r], lv[r]);
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
        const float m = ld_coherent(ml + 2 * r);
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
        for (int j = 0; j < NDW; ++j) v[u][j] = ld_coherent(po + 64 * j);
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

// ---------------------------------------------------------------------------
// The decode kernel (one wavefront per SIMD, two tile buffers in flight).
// ---------------------------------------------------------------------------
template <typename KV, int DP, typename OutS, bool FULL_D>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 1)))
decode_kernel(Params p, const uint16_t* __restrict__ q, const typename KV::storage* __restrict__ cache,
              const int32_t* __restrict__ kv_lens, const int32_t* __restrict__ page_indices,
              const int32_t* __restrict__ cu, const int32_t* __restrict__ dist,
              OutS* __restrict__ out, float* __restrict__ part_o, float* __restrict__ part_ml,
              int32_t* __restrict__ counters, int32_t max_units) {
  using C = DecodeCfg<KV, DP>;
  constexpr int TT = C::TT, NOCT = C::NOCT, NPART = C::NPART, NG = C::NG, NU = C::NU;
  constexpr int KP = NPART / 2;        // K parts (then V parts)
  constexpr int EPP = 128 / C::EB;     // elements per part
  constexpr int KK = DP / 32;          // MFMA k-steps over head_dim
  constexpr int NT = DP / 16;          // PV output tiles over head_dim

  __shared__ __align__(16) unsigned char smem[kWaves * C::WAVE_LDS];
  __shared__ int32_t s_nt[kMaxDecodeSeqs];
  __shared__ int32_t s_units[kMaxDecodeSeqs + 1];
  __shared__ int32_t s_kvlen[kMaxDecodeSeqs];
  __shared__ int32_t s_tq[kMaxDecodeSeqs];
  __shared__ int32_t s_red[2 * kWaves];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int g = lane >> 4;   // MFMA lane group
  const int n = lane & 15;   // MFMA column: q row within the kv head's group
  const int tl = lane >> 3;  // load shape: token within the octet
  const int ol = lane & 7;   // load shape: 16-byte column within a 128-byte part

  const Plan pl =
      build_plan(p, kv_lens, cu, dist, TT, max_units, s_nt, s_units, s_kvlen, s_tq, s_red);
  const int32_t total_items = pl.total_units * p.Hkv;
  const int32_t gw = static_cast<int32_t>(blockIdx.x) * kWaves + wave;
  const int32_t nw = static_cast<int32_t>(gridDim.x) * kWaves;
  if (gw >= total_items) return;  // no barrier follows the plan
  unsigned char* buf = smem + wave * C::WAVE_LDS;
  const int32_t rows = min(p.qpk, 16);
  const int32_t rp = decode_slot_rows(p.qpk);
  const int32_t max_tok = p.pps * p.ps - 1;

  // ---- item walk (wavefront-uniform) ---------------------------------------
  auto locate = [&](int32_t unit) __attribute__((always_inline)) {
    TileInfo ti;
    ti.unit = unit;
    if (unit >= total_items) return ti;
    const int32_t pu = unit / p.Hkv;
    ti.h = uni(unit - pu * p.Hkv);
    ti.s = uni(find_prefix(s_units, pl.num_seqs, pu));
    const int32_t u = uni(pu - s_units[ti.s]);
    const int32_t nt = uni(s_nt[ti.s]);
    ti.lt = u * pl.tpu;
    ti.lt_end = min(nt, ti.lt + pl.tpu);
    int32_t lo, hi;
    decode_range(p, s_kvlen[ti.s], &lo, &hi);
    ti.lo = uni(lo);
    ti.hi = uni(hi);
    return ti;
  };
  auto advance = [&](const TileInfo& c) __attribute__((always_inline)) {
    if (c.lt + 1 < c.lt_end) {
      TileInfo ti = c;
      ti.lt = c.lt + 1;
      return ti;
    }
    return locate(c.unit + nw);
  };

  // ---- addressing ------------------------------------------------------------
  // Lane (tl, ol) loads token base + 8o + tl of octet o (clamped into the key
  // range, so masked slots hold a copy of a valid key and every address is
  // inside the cache).  Its page id is a per-lane vector load issued one
  // pipeline step ahead of the tile load that uses it.
  auto clamp_tok = [&](const TileInfo& ti, int32_t j) __attribute__((always_inline)) -> int32_t {
    return min(max(min(j, ti.hi - 1), 0), max_tok);
  };
  struct Pages {
    int32_t pg[NOCT];
  };
  auto pages_of = [&](const TileInfo& ti, Pages& pp) __attribute__((always_inline)) {
    const int32_t sq = min(max(ti.s, 0), p.S - 1);
    const int32_t* ptab = page_indices + static_cast<int64_t>(sq) * p.pps;
    const int32_t base = ti.lo + ti.lt * TT;
#pragma unroll
    for (int o = 0; o < NOCT; ++o) pp.pg[o] = ptab[clamp_tok(ti, base + 8 * o + tl) / p.ps];
  };
  // Tile loads: octet o, part pt -> bytes [128pt + 16ol, +16) of the head's
  // K|V chunk of that token.
  auto load_tile = [&](const TileInfo& ti, const Pages& pp, uint4 (*rb)[NPART]) __attribute__((always_inline)) {
    const int32_t base = ti.lo + ti.lt * TT;
#pragma unroll
    for (int o = 0; o < NOCT; ++o) {
      const int32_t c = clamp_tok(ti, base + 8 * o + tl);
      const int32_t pg = min(max(pp.pg[o], 0), p.P - 1);
      const unsigned char* rec = reinterpret_cast<const unsigned char*>(
          cache + (static_cast<int64_t>(pg) * p.ps + c % p.ps) * p.rec +
          static_cast<int64_t>(2 * ti.h) * DP);
#pragma unroll
      for (int pt = 0; pt < NPART; ++pt)
        rb[o][pt] = *reinterpret_cast<const uint4*>(rec + 128 * pt + 16 * ol);
    }
  };
  // Q^T operand of (s, h): row n -> q head h*qpk + (n % qpk); dims 8g + 32kk
  // (clamped into the row; dims >= head_dim are zeroed where they are used).
  auto load_q = [&](const TileInfo& ti, uint4* qv) __attribute__((always_inline)) {
    const int32_t qh = ti.h * p.qpk + (n % p.qpk);
    const int32_t tq = s_tq[min(max(ti.s, 0), p.S - 1)];
    const uint16_t* qrow = q + (static_cast<int64_t>(tq) * p.Hq + qh) * p.D;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      const int d0 = FULL_D ? 8 * g + 32 * kk : min(8 * g + 32 * kk, p.D - 8);
      qv[kk] = *reinterpret_cast<const uint4*>(qrow + d0);
    }
  };

  // ---- pipeline ----------------------------------------------------------------
  TileInfo cur = locate(gw);
  uint4 qbuf[2][KK];
  uint4 bufr[2][NOCT][NPART];
  Pages pbuf[2];
  pages_of(cur, pbuf[0]);
  load_tile(cur, pbuf[0], bufr[0]);
  load_q(cur, qbuf[0]);
  TileInfo nxt = advance(cur);
  pages_of(nxt.unit < total_items ? nxt : cur, pbuf[0]);

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
                  const Pages& CP, Pages& NP) __attribute__((always_inline)) -> bool {
    const bool has_nxt = nxt.unit < total_items;
    const bool nxt_new_unit = has_nxt && nxt.unit != cur.unit;
    const TileInfo nn = has_nxt ? advance(nxt) : nxt;
    const TileInfo ldt = has_nxt ? nxt : cur;
    pages_of(nn.unit < total_items ? nn : ldt, NP);
    load_tile(ldt, CP, NB);
    load_q(ldt, NQ);

    // ---- K: registers -> LDS rows (stride KS) -> MFMA A operand.
    const int32_t base = cur.lo + cur.lt * TT;
    wave_lds_sync();  // the previous tile's V reads are complete
#pragma unroll
    for (int o = 0; o < NOCT; ++o)
#pragma unroll
      for (int pt = 0; pt < KP; ++pt)
        store_piece_bf16<KV>(buf + (8 * o + tl) * C::KS, pt * EPP + ol * (EPP / 8), CB[o][pt]);
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
        sc[i] = soft_cap_fn(sc[i] * p.score_scale, p.cap, p.inv_cap) * kLog2e;
    } else {
#pragma unroll
      for (int i = 0; i < 4 * NG; ++i) sc[i] *= p.score_scale * kLog2e;
    }
    float tmax = -INFINITY;
#pragma unroll
    for (int i = 0; i < 4 * NG; ++i) {
      const int32_t j = base + 16 * (i >> 2) + 4 * g + (i & 3);
      sc[i] = (j < cur.hi) ? sc[i] : -INFINITY;
      tmax = fmaxf(tmax, sc[i]);
    }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
    const float m_new = fmaxf(m_run, tmax);
    const float alpha = (m_run == -INFINITY) ? 0.0f : exp2f(m_run - m_new);
    float psum = 0.0f;
#pragma unroll
    for (int i = 0; i < 4 * NG; ++i) {
      sc[i] = (sc[i] == -INFINITY) ? 0.0f : exp2f(sc[i] - m_new);
      psum += sc[i];
    }
    l_run = l_run * alpha + psum;
    m_run = m_new;
#pragma unroll
    for (int t = 0; t < NT; ++t) oacc[t] *= alpha;

    // ---- V: registers -> LDS rows (stride VS) -> V^T operand via
    // ds_read_b64_tr_b16.  In 16-lane group g, source lane j points at token
    // T(j / 4), dims 16t + 4(j % 4); lane n then holds V[T(k)][16t + n], k < 4.
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
    wave_lds_sync();
#pragma unroll
    for (int u = 0; u < NU; ++u) {
      // P^T operand: k-slot k -> token 32u + 4g + k (k < 4), 32u + 16 + 4g + k - 4.
      uint4 pw;
      pw.x = pack_bf16x2(sc[8 * u + 0], sc[8 * u + 1]);
      pw.y = pack_bf16x2(sc[8 * u + 2], sc[8 * u + 3]);
      pw.z = pack_bf16x2(sc[8 * u + 4], sc[8 * u + 5]);
      pw.w = pack_bf16x2(sc[8 * u + 6], sc[8 * u + 7]);
      const bf16x8_t pop = as_bf16x8(pw);
      const unsigned char* ra = buf + (32 * u + 4 * g + (n >> 2)) * C::VS + 8 * (n & 3);
      const unsigned char* rb = ra + 16 * C::VS;
      v4i16 lo4[NT], hi4[NT];
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        lo4[t] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) v4i16*)(ra + 32 * t));
        hi4[t] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) v4i16*)(rb + 32 * t));
      }
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const uint2 l2 = __builtin_bit_cast(uint2, lo4[t]), h2 = __builtin_bit_cast(uint2, hi4[t]);
        const uint4 vv = make_uint4(l2.x, l2.y, h2.x, h2.y);
        oacc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(vv), pop, oacc[t], 0, 0, 0);
      }
    }

    // ---- end of a unit: finish (single-unit pair) or hand off a partial.
    if (cur.lt + 1 >= cur.lt_end) {
      float lsum = l_run;
      lsum += __shfl_xor(lsum, 16, 64);
      lsum += __shfl_xor(lsum, 32, 64);
      const int32_t s = cur.s, h = cur.h;
      const int32_t nunits = s_units[s + 1] - s_units[s];
      const int64_t orow0 = static_cast<int64_t>(s_tq[s]) * p.Hq + h * p.qpk;
      if (nunits == 1) {
        if (n < rows) {
          const float inv = (lsum == 0.0f) ? 0.0f : p.v_scale / lsum;
          OutS* orow = out + (orow0 + n) * p.D;
#pragma unroll
          for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const int d = 16 * t + 4 * g + i;
              if (d < p.D) store_out(orow, d, oacc[t][i] * inv);
            }
        }
      } else {
        const int64_t slot = cur.unit;  // one slot per (unit, head) item
        if (n < rows) {
          float* po = part_o + (slot * rp + n) * DP;
#pragma unroll
          for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i) st_coherent(po + 16 * t + 4 * g + i, oacc[t][i]);
          if (g == 0) {
            float* pm = part_ml + (slot * rp + n) * 2;
            st_coherent(pm, m_run);
            st_coherent(pm + 1, lsum);
          }
        }
        wait_stores_complete();
        int32_t* ctr = counters + s * p.Hkv + h;
        int32_t old = 0;
        if (lane == 0) old = __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        old = __shfl(old, 0, 64);
        asm volatile("" ::: "memory");
        if (old == nunits - 1) {
          const int32_t first = s_units[s] * p.Hkv + h;
          switch (rp) {
            case 1: merge_partials<DP, 1>(p, part_o, part_ml, first, nunits, rows, out, orow0); break;
            case 2: merge_partials<DP, 2>(p, part_o, part_ml, first, nunits, rows, out, orow0); break;
            case 4: merge_partials<DP, 4>(p, part_o, part_ml, first, nunits, rows, out, orow0); break;
            case 8: merge_partials<DP, 8>(p, part_o, part_ml, first, nunits, rows, out, orow0); break;
            default: merge_partials<DP, 16>(p, part_o, part_ml, first, nunits, rows, out, orow0); break;
          }
          // Ready for the next call (every arrival of this call has happened).
          if (lane == 0) __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      }
      m_run = -INFINITY;
      l_run = 0.0f;
#pragma unroll
      for (int t = 0; t < NT; ++t) oacc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    }
    (void)nxt_new_unit;

    if (!has_nxt) return false;
    cur = nxt;
    nxt = nn;
    return true;
  };

  while (step(bufr[0], bufr[1], qbuf[0], qbuf[1], pbuf[0], pbuf[1]) &&
         step(bufr[1], bufr[0], qbuf[1], qbuf[0], pbuf[1], pbuf[0])) {
  }
}

template <typename KV, int DP, typename OutS>
hipError_t launch_typed(const Params& p, const DecodeWorkspace& ws, const void* q,
                        const void* cache, const int32_t* kv_lens, const int32_t* page_indices,
                        const int32_t* cu, const int32_t* dist, void* out, int grid,
                        hipStream_t stream) {
  if (p.D == DP) {
    hipLaunchKernelGGL((decode_kernel<KV, DP, OutS, true>), dim3(grid), dim3(kThreads), 0, stream,
                       p, static_cast<const uint16_t*>(q),
                       static_cast<const typename KV::storage*>(cache), kv_lens, page_indices, cu,
                       dist, static_cast<OutS*>(out), ws.part_o, ws.part_ml, ws.counters,
                       ws.max_units);
  } else {
    hipLaunchKernelGGL((decode_kernel<KV, DP, OutS, false>), dim3(grid), dim3(kThreads), 0, stream,
                       p, static_cast<const uint16_t*>(q),
                       static_cast<const typename KV::storage*>(cache), kv_lens, page_indices, cu,
                       dist, static_cast<OutS*>(out), ws.part_o, ws.part_ml, ws.counters,
                       ws.max_units);
  }
  return hipGetLastError();
}

template <typename KV, typename OutS>
hipError_t launch_dp(const Params& p, const DecodeWorkspace& ws, const void* q, const void* cache,
                     const int32_t* kv_lens, const int32_t* page_indices, const int32_t* cu,
                     const int32_t* dist, void* out, int grid, hipStream_t stream) {
  if (p.Dp == 128)
    return launch_typed<KV, 128, OutS>(p, ws, q, cache, kv_lens, page_indices, cu, dist, out, grid, stream);
  if (p.Dp == 256)
    return launch_typed<KV, 256, OutS>(p, ws, q, cache, kv_lens, page_indices, cu, dist, out, grid, stream);
  return hipErrorInvalidValue;
}

template <typename OutS>
hipError_t launch_kv(const Params& p, int kv_dtype, const DecodeWorkspace& ws, const void* q,
                     const void* cache, const int32_t* kv_lens, const int32_t* page_indices,
                     const int32_t* cu, const int32_t* dist, void* out, int grid,
                     hipStream_t stream) {
  switch (kv_dtype) {
    case RPA_DTYPE_BF16:
      return launch_dp<KvBF16, OutS>(p, ws, q, cache, kv_lens, page_indices, cu, dist, out, grid, stream);
    case RPA_DTYPE_FP8_E4M3FN:
      return launch_dp<KvFP8<false>, OutS>(p, ws, q, cache, kv_lens, page_indices, cu, dist, out, grid, stream);
    case RPA_DTYPE_FP8_E5M2:
      return launch_dp<KvFP8<true>, OutS>(p, ws, q, cache, kv_lens, page_indices, cu, dist, out, grid, stream);
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
  if (p.Dp != 128 && p.Dp != 256) return false;
  if (p.D % 8 != 0 || p.qpk > 16) return false;
  if (p.ps < 16) return false;  // a 16-token group must span at most two pages
  if (p.S > kMaxDecodeSeqs || p.Hkv > kMaxDecodeHeads) return false;
  return true;
}

int decode_grid(const Params& p, int num_cus) {
  // Persistent grid at the kernel's occupancy (one wavefront per SIMD, one
  // workgroup per CU); at least one wavefront per kv head.
  const int occ = num_cus;
  const int min_grid = (p.Hkv + kWaves - 1) / kWaves;
  return occ > min_grid ? occ : min_grid;
}

// Workspace layout: a fixed-size counter region first (so that no call, of
// any shape, ever stores anything else there: counters stay zero between
// calls), then the partial outputs, one slot per (sequence unit, kv head).
constexpr size_t kCounterBytes = static_cast<size_t>(kMaxDecodeSeqs) * kMaxDecodeHeads * sizeof(int32_t);
constexpr size_t kPartialBudget = size_t(256) << 20;

// Capacity in (sequence, unit) pairs.  The device plan grows units beyond two
// tiles whenever the batch would need more.
static int32_t decode_max_units(const Params& p, int kv_bytes) {
  const int64_t rows = decode_slot_rows(p.qpk);
  const int64_t per_unit = static_cast<int64_t>(p.Hkv) * rows * (p.Dp * 4 + 8);
  const int64_t unit_tokens = 2 * decode_tile_tokens(p.Dp, kv_bytes);
  const int64_t need = static_cast<int64_t>(p.S) * ((static_cast<int64_t>(p.pps) * p.ps + unit_tokens - 1) / unit_tokens);
  int64_t cap = static_cast<int64_t>(kPartialBudget) / per_unit;
  if (cap < p.S + 1024) cap = p.S + 1024;
  int64_t m = need < cap ? need : cap;
  if (m < p.S + 1) m = p.S + 1;
  return static_cast<int32_t>(m);
}

size_t decode_workspace_bytes(const Params& p, int kv_bytes) {
  const int64_t rows = decode_slot_rows(p.qpk);
  const int64_t slots = static_cast<int64_t>(decode_max_units(p, kv_bytes)) * p.Hkv;
  size_t bytes = 256 + kCounterBytes;
  bytes += static_cast<size_t>(slots) * rows * p.Dp * sizeof(float);  // part_o
  bytes += static_cast<size_t>(slots) * rows * 2 * sizeof(float);     // part_ml
  return bytes + 256;
}

DecodeWorkspace carve_decode_workspace(const Params& p, void* base, int kv_bytes) {
  DecodeWorkspace ws;
  const int64_t rows = decode_slot_rows(p.qpk);
  ws.max_units = decode_max_units(p, kv_bytes);
  const int64_t slots = static_cast<int64_t>(ws.max_units) * p.Hkv;
  uintptr_t ptr = (reinterpret_cast<uintptr_t>(base) + 255) & ~static_cast<uintptr_t>(255);
  ws.counters = reinterpret_cast<int32_t*>(ptr);
  ptr += kCounterBytes;
  ws.part_o = reinterpret_cast<float*>(ptr);
  ptr += static_cast<size_t>(slots) * rows * p.Dp * sizeof(float);
  ws.part_ml = reinterpret_cast<float*>(ptr);
  return ws;
}

hipError_t launch_decode(const Params& p, int q_dtype, int kv_dtype, int out_dtype,
                         const DecodeWorkspace& ws, const void* q, const void* cache,
                         const int32_t* kv_lens, const int32_t* page_indices, const int32_t* cu,
                         const int32_t* dist, void* out, int num_cus, hipStream_t stream) {
  (void)q_dtype;
  const int grid = decode_grid(p, num_cus);
  if (grid <= 0) return hipSuccess;
  if (out_dtype == RPA_DTYPE_F32)
    return launch_kv<float>(p, kv_dtype, ws, q, cache, kv_lens, page_indices, cu, dist, out, grid, stream);
  return launch_kv<uint16_t>(p, kv_dtype, ws, q, cache, kv_lens, page_indices, cu, dist, out, grid, stream);
}

}  // namespace rpa
