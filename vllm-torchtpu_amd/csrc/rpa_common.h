// Shared device-side definitions for the gfx950 RPA kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "rpa.h"

namespace rpa {

// ---------------------------------------------------------------------------
// Launch parameters.  Built once on the host from rpa_desc; passed by value.
// Element strides are in elements of the tensor's own dtype.
// ---------------------------------------------------------------------------
struct Params {
  int32_t T;       // max_num_tokens
  int32_t Hq;      // num_q_heads
  int32_t Hkv;     // num_kv_heads
  int32_t qpk;     // Hq / Hkv
  int32_t D;       // actual head_dim
  int32_t Dp;      // padded head_dim (cache last axis)
  int32_t P;       // total_num_pages
  int32_t ps;      // page_size
  int32_t Kx2;     // combined heads per record (padded)
  int32_t S;       // max_num_seqs
  int32_t pps;     // pages_per_seq
  int32_t causal;  // use_causal_mask
  int32_t window;  // sliding_window, <= 0 = none
  int32_t window_nc;  // the window also masks rows without the causal mask
  int32_t has_cap;
  float cap;
  float inv_cap;
  float score_scale;  // sm_scale * k_scale * q_scale
  float v_scale;
  int64_t rec;  // elements per token record = Kx2 * Dp
  int32_t ps_shift;        // log2(ps) when ps is a power of two, else -1
  int32_t skip_kv_update;  // new tokens are already in the cache (read them from there)
  int32_t decode_waves;    // wavefronts of the decode kernel's persistent grid (0: no decode kernel)
  int32_t prefill_on;      // the prefill kernel attends the non-decode rows
  int32_t dq;              // largest q_len of a decode row group (>= 1; dq * qpk <= 16)
  int32_t kv_bytes;        // bytes per cache element (2: bf16, 1: fp8)
  float* lse;              // [T, Hq] natural-log LSE of each output row, or null
  const float* sink;       // [Hq] attention-sink logits (natural log), or null
};

constexpr float kLn2 = 0.6931471805599453f;

// LSE of a row from its running max m (log2 units of the logits) and the sum
// l of 2^(s - m): (m + log2 l) ln 2, natural-log base; -inf for a row that
// attends no key (l == 0), as the reference's m + log(max(l, 1e-9)) with
// m = -inf gives (batched_rpa/kernel.py:116-124).
__device__ __forceinline__ float lse_from_log2(float m, float l) {
  return l > 0.0f ? (m + __log2f(l)) * kLn2 : -INFINITY;
}

// Row sum with q head g's attention sink (kernel_hd64.py:161-172, :450-456):
// the sink is one more logit in the softmax, with value 0, so it adds
// 2^(sink log2 e - m) to the sum l of 2^(s - m) (m: the row's reference max,
// log2 units).  A sink far above m sends the sum to +inf and the row to 0.
__device__ __forceinline__ float sum_with_sink(const Params& p, int32_t g, float m, float l) {
  if (p.sink == nullptr) return l;
  return l + exp2f(p.sink[g] * 1.4426950408889634f - m);
}

// Page and slot of logical position j (>= 0): shifts for power-of-two page
// sizes (a wavefront-uniform branch), division otherwise.
__device__ __forceinline__ int32_t page_of(const Params& p, int32_t j) {
  return p.ps_shift >= 0 ? (j >> p.ps_shift) : j / p.ps;
}
__device__ __forceinline__ int32_t slot_of(const Params& p, int32_t j) {
  return p.ps_shift >= 0 ? (j & (p.ps - 1)) : j % p.ps;
}

// ---------------------------------------------------------------------------
// Scalar conversions, written from the format definitions.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

// Round-to-nearest-even f32 -> bf16 bits; NaN stays a quiet NaN.
// Lazy rescaling of the online softmax: a row's reference max moves only when
// a tile's max exceeds it by more than 2^kRescaleLog2 (P values then stay
// below 2^8), so most tiles skip the rescale of the accumulators.
constexpr float kRescaleLog2 = 8.0f;

__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

// Four packed OCP fp8 values (byte i = element i) -> four bf16 values
// (element i in bits [16i, 16i + 16) of the pair).  gfx950's
// v_cvt_scalef32_pk_bf16_{fp8,bf8} with scale 1.0 converts two elements per
// instruction; every e4m3fn / e5m2 value, subnormals included, is exactly
// representable in bf16, so the result is exact (NaN stays NaN).
template <bool kE5M2>
__device__ __forceinline__ uint2 fp8x4_to_bf16x4(uint32_t w) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  bf16x2_t lo, hi;
  if constexpr (kE5M2) {
    lo = __builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(static_cast<int>(w), 1.0f, false);
    hi = __builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(static_cast<int>(w), 1.0f, true);
  } else {
    lo = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(static_cast<int>(w), 1.0f, false);
    hi = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(static_cast<int>(w), 1.0f, true);
  }
  return make_uint2(__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi));
}

// OCP fp8 e4m3fn: 1 sign, 4 exponent (bias 7), 3 mantissa; S.1111.111 = NaN,
// no infinities; subnormals are m * 2^-9.
__device__ __forceinline__ float fp8e4m3_to_f32(uint8_t x) {
  const uint32_t e = (x >> 3) & 0xfu;
  const uint32_t m = x & 7u;
  float v;
  if (e == 0xfu && m == 7u) {
    v = __uint_as_float(0x7fc00000u);
  } else if (e == 0u) {
    v = static_cast<float>(m) * 0x1p-9f;
  } else {
    v = __uint_as_float(((e + 120u) << 23) | (m << 20));
  }
  return (x & 0x80u) ? -v : v;
}

// OCP fp8 e5m2 is the upper byte of an IEEE binary16.
__device__ __forceinline__ float fp8e5m2_to_f32(uint8_t x) {
  const uint16_t h = static_cast<uint16_t>(x) << 8;
  return static_cast<float>(__builtin_bit_cast(_Float16, h));
}

__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) {
  return static_cast<float>(__builtin_bit_cast(_Float16, h));
}

// Element-type tags: storage type + conversion to f32.
struct TF32 {
  using storage = float;
  static __device__ __forceinline__ float load(const storage* p, int64_t i) { return p[i]; }
};
struct TBF16 {
  using storage = uint16_t;
  static __device__ __forceinline__ float load(const storage* p, int64_t i) {
    return bf16_bits_to_f32(p[i]);
  }
};
struct TF16 {
  using storage = uint16_t;
  static __device__ __forceinline__ float load(const storage* p, int64_t i) {
    return f16_bits_to_f32(p[i]);
  }
};
struct TE4M3 {
  using storage = uint8_t;
  static __device__ __forceinline__ float load(const storage* p, int64_t i) {
    return fp8e4m3_to_f32(p[i]);
  }
};
struct TE5M2 {
  using storage = uint8_t;
  static __device__ __forceinline__ float load(const storage* p, int64_t i) {
    return fp8e5m2_to_f32(p[i]);
  }
};

// Output stores (f32; bf16 as uint16_t bits; f16 as _Float16, round to
// nearest even).
__device__ __forceinline__ void store_out(float* p, int64_t i, float v) { p[i] = v; }
__device__ __forceinline__ void store_out(_Float16* p, int64_t i, float v) {
  p[i] = static_cast<_Float16>(v);
}
__device__ __forceinline__ void store_out(uint16_t* p, int64_t i, float v) {
  p[i] = f32_to_bf16_bits(v);
}

// ---------------------------------------------------------------------------
// Metadata helpers (all reads are clamped so bad metadata cannot address
// memory outside the tensors).
// ---------------------------------------------------------------------------
__device__ __forceinline__ int32_t num_seqs_of(const int32_t* distribution, int32_t S) {
  int32_t n = distribution[2];
  return n < 0 ? 0 : (n > S ? S : n);
}

// Largest s in [0, n) with cu[s] <= t (cu non-decreasing); -1 if none.
__device__ __forceinline__ int32_t find_seq(const int32_t* cu, int32_t n, int32_t t) {
  int32_t lo = 0, hi = n;  // answer in [lo, hi)
  if (n <= 0 || cu[0] > t) return -1;
  while (hi - lo > 1) {
    int32_t mid = (lo + hi) >> 1;
    if (cu[mid] <= t) lo = mid; else hi = mid;
  }
  return lo;
}

__device__ __forceinline__ float warp_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ float warp_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Orders a wavefront's own LDS writes before its later LDS reads (and
// reads before later writes) without a workgroup barrier.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// logit transform shared by every attention kernel: scale then soft cap
// (kernel.py:185-194): s = cap * tanh(s / cap).  tanh is built from exp:
// tanh(x) = 1 - 2 / (exp(2x) + 1), exact at the limits (+-1) and odd.  The
// exponential is v_exp_f32 (2^y with y = 2 x log2 e) and the reciprocal
// v_rcp_f32 (1 ulp each), not an IEEE division: the result is within a few
// ulp of cap (absolute), far inside every tolerance the logits feed.
__device__ __forceinline__ float soft_cap_fn(float s, float cap, float inv_cap) {
  const float e = __builtin_amdgcn_exp2f(s * (inv_cap * 2.8853900817779268f));  // e^(2 s / cap)
  const float r = __builtin_amdgcn_rcpf(e + 1.0f);
  return cap * fmaf(-2.0f, r, 1.0f);
}

// The same transform of a raw dot product x, in log2 units, with the
// constants folded: a = sm-scale * 2 log2(e) / cap, b = cap * log2(e);
// returns b * tanh(x * sm-scale / cap) = b - 2 b / (2^(a x) + 1).
__device__ __forceinline__ float soft_cap_log2(float x, float a, float b) {
  const float r = __builtin_amdgcn_rcpf(__builtin_amdgcn_exp2f(x * a) + 1.0f);
  return fmaf(-2.0f * b, r, b);
}
struct SoftCapLog2 {
  float a, b;
};
__device__ __forceinline__ SoftCapLog2 soft_cap_log2_consts(const Params& p) {
  return SoftCapLog2{p.score_scale * p.inv_cap * 2.8853900817779268f,
                     p.cap * 1.4426950408889634f};
}

}  // namespace rpa
