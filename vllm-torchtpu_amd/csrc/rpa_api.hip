// C ABI of librpa_hip.so (declared in include/rpa.h).
//
// Host-side only: validates the descriptor, derives the launch parameters and
// enqueues the kernels on the caller's stream.  No allocation, no host sync.
#include <math.h>
#include <string.h>

#include <mutex>

#include "rpa.h"
#include "rpa_common.h"
#include "rpa_internal.h"

namespace {

int dtype_bytes(int dt) {
  switch (dt) {
    case RPA_DTYPE_F32: return 4;
    case RPA_DTYPE_BF16:
    case RPA_DTYPE_F16: return 2;
    case RPA_DTYPE_FP8_E4M3FN:
    case RPA_DTYPE_FP8_E5M2: return 1;
    default: return 0;
  }
}

int64_t cdiv64(int64_t a, int64_t b) { return (a + b - 1) / b; }
int64_t align64(int64_t x, int64_t a) { return cdiv64(x, a) * a; }

rpa::Params make_params(const rpa_desc* d) {
  rpa::Params p;
  memset(&p, 0, sizeof(p));
  p.T = d->max_num_tokens;
  p.Hq = d->num_q_heads;
  p.Hkv = d->num_kv_heads;
  p.qpk = d->num_q_heads / d->num_kv_heads;
  p.D = d->head_dim;
  p.Dp = d->head_dim_padded;
  p.P = d->total_num_pages;
  p.ps = d->page_size;
  p.Kx2 = d->kv_heads_x2;
  p.S = d->max_num_seqs;
  p.pps = d->pages_per_seq;
  p.causal = d->use_causal_mask ? 1 : 0;
  p.window = d->sliding_window > 0 ? d->sliding_window : 0;
  p.window_nc = (d->window_all_rows && !d->use_causal_mask && p.window > 0) ? 1 : 0;
  p.has_cap = d->has_soft_cap ? 1 : 0;
  p.cap = d->soft_cap;
  p.inv_cap = d->has_soft_cap ? 1.0f / d->soft_cap : 0.0f;
  p.score_scale = d->sm_scale * d->k_scale * d->q_scale;
  p.v_scale = d->v_scale;
  p.rec = static_cast<int64_t>(d->kv_heads_x2) * d->head_dim_padded;
  p.kv_bytes = dtype_bytes(d->kv_dtype);
  p.skip_kv_update = d->skip_kv_update ? 1 : 0;
  p.ps_shift = -1;
  for (int sh = 0; sh < 31; ++sh)
    if ((1 << sh) == d->page_size) p.ps_shift = sh;
  p.decode_waves = 0;
  // Decode row groups: q_len tokens x qpk heads fill at most the 16 MFMA
  // columns of the decode kernel.
  const int32_t dq_max = p.qpk > 0 && p.qpk <= 16 ? 16 / p.qpk : 1;
  p.dq = d->decode_query_size < 1 ? 1 : (d->decode_query_size > dq_max ? dq_max : d->decode_query_size);
  return p;
}

// Launch structure of a call.  The fused path is the decode kernel (when
// the shape allows it) followed by the finish kernel; the generic path is the
// KV-page write followed by the shape-generic attention kernel.
bool use_fused_path(const rpa_desc* d, const rpa::Params& p) {
  // A window on rows without the causal mask is the generic kernels' only.
  return d->path != RPA_PATH_GENERIC && !p.window_nc &&
         rpa::finish_supported(p, d->q_dtype, d->kv_dtype, d->out_dtype);
}
bool use_decode_kernel(const rpa_desc* d, const rpa::Params& p) {
  return use_fused_path(d, p) && rpa::decode_supported(p, d->q_dtype, d->kv_dtype, d->out_dtype);
}

// Compute units of the current device (cached per device id).
int current_num_cus() {
  static int cache[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cache[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    cache[dev] = n;
  }
  return cache[dev];
}

}  // namespace

// Scratch of rpa_forward_noalloc: the decode partials and the published plan
// that rpa_forward keeps in the caller's workspace.  Each GPU the library runs
// on holds its own copy of this array until the process ends.  In host code
// the name is a host-side stand-in, never a device address: host code uses
// only the per-device address hipGetSymbolAddress returns (g_scratch_dev).
static __device__ __align__(256) unsigned char scratch[RPA_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_dev[kMaxDevices] = {};

// Device address of the current device's copy of `scratch`, looked up once per
// device (with that device current) on its first rpa_forward_noalloc call.
int scratch_of_current_device(void** ptr) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess) return RPA_ERR_LAUNCH;
  if (dev < 0 || dev >= kMaxDevices) return RPA_ERR_UNSUPPORTED;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_dev[dev] == nullptr) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || p == nullptr)
      return RPA_ERR_LAUNCH;
    g_scratch_dev[dev] = p;
  }
  *ptr = g_scratch_dev[dev];
  return RPA_OK;
}

}  // namespace

extern "C" {

int rpa_abi_version(void) { return RPA_ABI_VERSION; }

const char* rpa_status_str(int status) {
  switch (status) {
    case RPA_OK: return "ok";
    case RPA_ERR_INVALID_ARG: return "invalid argument: descriptor violates the RPA input contract";
    case RPA_ERR_UNSUPPORTED: return "unsupported: valid RPA input not implemented by this library";
    case RPA_ERR_WORKSPACE: return "workspace missing or smaller than rpa_workspace_size()";
    case RPA_ERR_LAUNCH: return "HIP kernel launch failed";
    case RPA_ERR_NULL_PTR: return "a required device pointer is NULL";
    case RPA_ERR_ABI: return "rpa_desc.abi_version does not match the library";
    case RPA_ERR_SCRATCH:
      return "the call needs more scratch than rpa_forward_noalloc's fixed buffer "
             "(RPA_NOALLOC_SCRATCH_BYTES); call rpa_forward with a workspace instead";
    default: return "unknown status";
  }
}

int rpa_get_kv_cache_shape(int32_t total_num_pages, int32_t page_size, int32_t num_kv_heads,
                           int32_t head_dim, int32_t kv_dtype, int64_t shape_out[5]) {
  const int b = dtype_bytes(kv_dtype);
  if (b == 0 || shape_out == nullptr) return RPA_ERR_INVALID_ARG;
  const int pack = 4 / b;
  shape_out[0] = total_num_pages;
  shape_out[1] = page_size;
  shape_out[2] = align64(2LL * num_kv_heads, pack) / pack;
  shape_out[3] = pack;
  shape_out[4] = align64(head_dim, 128);
  return RPA_OK;
}

int rpa_validate_desc(const rpa_desc* d) {
  if (d == nullptr) return RPA_ERR_NULL_PTR;
  if (d->abi_version != RPA_ABI_VERSION) return RPA_ERR_ABI;
  const int kvb = dtype_bytes(d->kv_dtype);
  if (kvb == 0 || dtype_bytes(d->q_dtype) == 0) return RPA_ERR_INVALID_ARG;
  if (d->num_q_heads <= 0 || d->num_kv_heads <= 0 || d->head_dim <= 0) return RPA_ERR_INVALID_ARG;
  if (d->num_q_heads % d->num_kv_heads != 0) return RPA_ERR_INVALID_ARG;
  const int pack = 4 / kvb;
  if (d->kv_packing != pack) return RPA_ERR_INVALID_ARG;
  // Two cache layouts (kernel.py:278-292 and kernel_hd64.py:246-261): heads
  // packed with head_dim padded to 128, or, for head_dim 64 only, K|V of a
  // head side by side in one 128-wide row -- the same bytes as head_dim_padded
  // 64 with kv heads padded to the packing before doubling.
  const bool hd64_packed = d->head_dim == 64 && d->head_dim_padded == 64;
  if (!hd64_packed && d->head_dim_padded != align64(d->head_dim, 128)) return RPA_ERR_INVALID_ARG;
  const int64_t kx2 = hd64_packed ? 2 * align64(d->num_kv_heads, pack)
                                  : align64(2LL * d->num_kv_heads, pack);
  if (d->kv_heads_x2 != kx2) return RPA_ERR_INVALID_ARG;
  if (d->page_size <= 0 || d->page_size % pack != 0) return RPA_ERR_INVALID_ARG;
  if (d->total_num_pages <= 0 || d->max_num_tokens < 0) return RPA_ERR_INVALID_ARG;
  if (d->max_num_seqs <= 0 || d->pages_per_seq < 0) return RPA_ERR_INVALID_ARG;
  if (d->has_soft_cap && d->soft_cap == 0.0f) return RPA_ERR_INVALID_ARG;
  if (d->sliding_window < 0) return RPA_ERR_INVALID_ARG;
  if (d->decode_query_size < 0) return RPA_ERR_INVALID_ARG;
  if (d->path < RPA_PATH_AUTO || d->path > RPA_PATH_DECODE_ONLY) return RPA_ERR_INVALID_ARG;
  // Implemented combinations.
  if (d->out_dtype != RPA_DTYPE_F32 && d->out_dtype != RPA_DTYPE_BF16 &&
      d->out_dtype != RPA_DTYPE_F16)
    return RPA_ERR_UNSUPPORTED;
  const bool q_is_fp8 = d->q_dtype == RPA_DTYPE_FP8_E4M3FN || d->q_dtype == RPA_DTYPE_FP8_E5M2;
  if (q_is_fp8 && d->q_dtype != d->kv_dtype) return RPA_ERR_UNSUPPORTED;
  if (d->head_dim_padded > 512) return RPA_ERR_UNSUPPORTED;
  return RPA_OK;
}

size_t rpa_workspace_size(const rpa_desc* d) {
  if (rpa_validate_desc(d) != RPA_OK) return 0;
  rpa::Params p = make_params(d);
  size_t bytes = 256;
  if (use_decode_kernel(d, p)) {
    p.decode_waves = rpa::decode_waves(p, current_num_cus());
    bytes += rpa::decode_workspace_bytes(p);
  }
  return bytes;
}

int rpa_kv_cache_update(const rpa_desc* d, const void* keys, const void* values, void* kv_cache,
                        const int32_t* kv_lens, const int32_t* page_indices,
                        const int32_t* cu_q_lens, const int32_t* distribution, void* stream) {
  const int st = rpa_validate_desc(d);
  if (st != RPA_OK) return st;
  if (d->max_num_tokens == 0) return RPA_OK;
  if (!keys || !values || !kv_cache || !kv_lens || !page_indices || !cu_q_lens || !distribution)
    return RPA_ERR_NULL_PTR;
  const rpa::Params p = make_params(d);
  hipError_t e = rpa::launch_kv_update(p, dtype_bytes(d->kv_dtype), keys, values, kv_cache,
                                       kv_lens, page_indices, cu_q_lens, distribution,
                                       static_cast<hipStream_t>(stream));
  return e == hipSuccess ? RPA_OK : RPA_ERR_LAUNCH;
}

int rpa_forward(const rpa_desc* d, const void* queries, const void* keys, const void* values,
                void* kv_cache, const int32_t* kv_lens, const int32_t* page_indices,
                const int32_t* cu_q_lens, const int32_t* distribution, void* out,
                void* workspace, size_t workspace_bytes, void* stream) {
  return rpa_forward_ex(d, queries, keys, values, kv_cache, kv_lens, page_indices, cu_q_lens,
                        distribution, out, nullptr, nullptr, workspace, workspace_bytes, stream);
}

int rpa_forward_lse(const rpa_desc* d, const void* queries, const void* keys, const void* values,
                    void* kv_cache, const int32_t* kv_lens, const int32_t* page_indices,
                    const int32_t* cu_q_lens, const int32_t* distribution, void* out, float* lse,
                    void* workspace, size_t workspace_bytes, void* stream) {
  return rpa_forward_ex(d, queries, keys, values, kv_cache, kv_lens, page_indices, cu_q_lens,
                        distribution, out, nullptr, lse, workspace, workspace_bytes, stream);
}

int rpa_forward_ex(const rpa_desc* d, const void* queries, const void* keys, const void* values,
                   void* kv_cache, const int32_t* kv_lens, const int32_t* page_indices,
                   const int32_t* cu_q_lens, const int32_t* distribution, void* out,
                   const float* attention_sink, float* lse, void* workspace,
                   size_t workspace_bytes, void* stream) {
  const int st = rpa_validate_desc(d);
  if (st != RPA_OK) return st;
  if (d->max_num_tokens == 0) return RPA_OK;
  if (!queries || !kv_cache || !kv_lens || !page_indices || !cu_q_lens || !distribution || !out)
    return RPA_ERR_NULL_PTR;
  if (workspace_bytes < rpa_workspace_size(d) || workspace == nullptr) return RPA_ERR_WORKSPACE;
  if (!d->skip_kv_update && (!keys || !values)) return RPA_ERR_NULL_PTR;
  // Every kernel reads and writes 8- or 16-byte pieces.
  const uintptr_t align = reinterpret_cast<uintptr_t>(queries) | reinterpret_cast<uintptr_t>(kv_cache) |
                          reinterpret_cast<uintptr_t>(out) | reinterpret_cast<uintptr_t>(keys) |
                          reinterpret_cast<uintptr_t>(values);
  if (align & 15u) return RPA_ERR_INVALID_ARG;
  // An LSE over keys with a sink folded in would count the sink once per
  // merged partial; the reference has no such output either.
  if (lse != nullptr && attention_sink != nullptr) return RPA_ERR_UNSUPPORTED;
  hipStream_t s = static_cast<hipStream_t>(stream);
  rpa::Params p = make_params(d);
  p.lse = lse;
  p.sink = attention_sink;
  const bool decode_only = d->path == RPA_PATH_DECODE_ONLY;
  if (decode_only && !use_decode_kernel(d, p)) return RPA_ERR_UNSUPPORTED;
  if (!use_fused_path(d, p)) {
    if (!d->skip_kv_update) {
      hipError_t e = rpa::launch_kv_update(p, dtype_bytes(d->kv_dtype), keys, values, kv_cache,
                                           kv_lens, page_indices, cu_q_lens, distribution, s);
      if (e != hipSuccess) return RPA_ERR_LAUNCH;
    }
    hipError_t e = rpa::launch_attn_generic(p, d->q_dtype, d->kv_dtype, d->out_dtype, queries,
                                            kv_cache, kv_lens, page_indices, cu_q_lens,
                                            distribution, out, s);
    return e == hipSuccess ? RPA_OK : RPA_ERR_LAUNCH;
  }
  const int cus = current_num_cus();
  rpa::DecodeWorkspace ws{nullptr, nullptr, nullptr, 0};
  if (use_decode_kernel(d, p)) {
    p.decode_waves = rpa::decode_waves(p, cus);
    ws = rpa::carve_decode_workspace(p, workspace);
    hipError_t e = rpa::launch_decode(p, d->kv_dtype, d->out_dtype, ws, queries, keys, values,
                                      kv_cache, kv_lens, page_indices, cu_q_lens, distribution,
                                      out, s);
    if (e != hipSuccess) return RPA_ERR_LAUNCH;
    if (decode_only) return RPA_OK;
  }
  // The prefill launch also carries the merge and write items; the finish
  // kernel runs only for shapes the prefill kernel does not take.
  if (rpa::prefill_supported(p, d->q_dtype, d->kv_dtype, d->out_dtype)) {
    p.prefill_on = 1;
    hipError_t e = rpa::launch_prefill(p, d->kv_dtype, d->out_dtype, queries, keys, values,
                                       kv_cache, kv_lens, page_indices, cu_q_lens, distribution,
                                       out, ws, cus, s);
    if (e != hipSuccess) return RPA_ERR_LAUNCH;
    if (rpa::prefill_has_finish_roles(p) || (p.decode_waves <= 0 && d->skip_kv_update))
      return RPA_OK;
    // Merges and cache writes in a finish launch after the prefill kernel
    // (which reads new tokens from k/v, never from the pages being written).
    e = rpa::launch_finish(p, d->kv_dtype, d->out_dtype, ws, queries, keys, values, kv_cache,
                           kv_lens, page_indices, cu_q_lens, distribution, out, cus, s);
    return e == hipSuccess ? RPA_OK : RPA_ERR_LAUNCH;
  }
  hipError_t e = rpa::launch_finish(p, d->kv_dtype, d->out_dtype, ws, queries, keys, values,
                                    kv_cache, kv_lens, page_indices, cu_q_lens, distribution, out,
                                    cus, s);
  return e == hipSuccess ? RPA_OK : RPA_ERR_LAUNCH;
}

int rpa_forward_noalloc(const rpa_desc* d, const void* queries, const void* keys,
                        const void* values, void* kv_cache, const int32_t* kv_lens,
                        const int32_t* page_indices, const int32_t* cu_q_lens,
                        const int32_t* distribution, void* out, void* stream) {
  const int st = rpa_validate_desc(d);
  if (st != RPA_OK) return st;
  const size_t need = rpa_workspace_size(d);
  if (need > RPA_NOALLOC_SCRATCH_BYTES) return RPA_ERR_SCRATCH;
  if (d->max_num_tokens == 0) return RPA_OK;
  void* ws = nullptr;
  const int sst = scratch_of_current_device(&ws);
  if (sst != RPA_OK) return sst;
  // The same kernels as rpa_forward, on this device's scratch (nothing in it
  // needs clearing: the kernels write every slot before reading it).
  return rpa_forward_ex(d, queries, keys, values, kv_cache, kv_lens, page_indices, cu_q_lens,
                        distribution, out, nullptr, nullptr, ws, RPA_NOALLOC_SCRATCH_BYTES,
                        stream);
}

}  // extern "C"
