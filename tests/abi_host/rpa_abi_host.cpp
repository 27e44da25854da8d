// A non-Python host of the C ABI (include/rpa.h), as a C or C++ serving
// runtime would drive it: it allocates its own device buffers and workspace
// with hipMalloc, creates its own stream, and calls rpa_forward and
// rpa_forward_lse -- the entry points the reference's
// ragged_paged_attention (kernels/ragged_paged_attention/v3/kernel.py:1609-1671)
// and the batched wrapper's return_lse (batched_rpa/wrapper.py:553) map to.
//
//   rpa_abi_host DIR
//
// DIR holds desc.txt ("field value" per line: the rpa_desc fields) and the
// raw little-endian inputs q.bin k.bin v.bin kv_cache.bin kv_lens.bin
// page_indices.bin cu_q_lens.bin distribution.bin.  It writes
//   out.bin, cache.bin          after rpa_forward on a copy of the cache,
//   out_lse.bin, lse.bin,
//   cache_lse.bin               after rpa_forward_lse on a second copy,
// and exits 0, or prints the failing call and its status and exits 1.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <map>
#include <sstream>
#include <string>
#include <vector>

#include "rpa.h"

namespace {

std::vector<char> read_file(const std::string& path) {
  std::ifstream f(path, std::ios::binary);
  if (!f) {
    std::fprintf(stderr, "cannot read %s\n", path.c_str());
    std::exit(1);
  }
  return std::vector<char>((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
}

void write_file(const std::string& path, const std::vector<char>& data) {
  std::ofstream f(path, std::ios::binary);
  f.write(data.data(), static_cast<std::streamsize>(data.size()));
}

#define HIP_OK(x)                                                                   \
  do {                                                                              \
    hipError_t e_ = (x);                                                            \
    if (e_ != hipSuccess) {                                                         \
      std::fprintf(stderr, "%s failed: %s\n", #x, hipGetErrorString(e_));           \
      std::exit(1);                                                                 \
    }                                                                               \
  } while (0)

struct DevBuf {
  void* p = nullptr;
  size_t n = 0;
};

DevBuf upload(const std::vector<char>& h, hipStream_t s) {
  DevBuf b;
  b.n = h.size();
  HIP_OK(hipMalloc(&b.p, b.n > 0 ? b.n : 16));
  if (b.n) HIP_OK(hipMemcpyAsync(b.p, h.data(), b.n, hipMemcpyHostToDevice, s));
  return b;
}

std::vector<char> download(const DevBuf& b, hipStream_t s) {
  std::vector<char> h(b.n);
  if (b.n) HIP_OK(hipMemcpyAsync(h.data(), b.p, b.n, hipMemcpyDeviceToHost, s));
  HIP_OK(hipStreamSynchronize(s));
  return h;
}

}  // namespace

int main(int argc, char** argv) {
  if (argc != 2) {
    std::fprintf(stderr, "usage: %s DIR\n", argv[0]);
    return 2;
  }
  const std::string dir = argv[1];
  std::map<std::string, double> f;
  {
    std::ifstream in(dir + "/desc.txt");
    std::string line;
    while (std::getline(in, line)) {
      std::istringstream ls(line);
      std::string k;
      double v;
      if (ls >> k >> v) f[k] = v;
    }
  }
  rpa_desc d;
  std::memset(&d, 0, sizeof(d));
  d.abi_version = RPA_ABI_VERSION;
  auto i32 = [&](const char* k) { return static_cast<int32_t>(f.at(k)); };
  d.q_dtype = i32("q_dtype");
  d.kv_dtype = i32("kv_dtype");
  d.out_dtype = i32("out_dtype");
  d.max_num_tokens = i32("max_num_tokens");
  d.num_q_heads = i32("num_q_heads");
  d.num_kv_heads = i32("num_kv_heads");
  d.head_dim = i32("head_dim");
  d.head_dim_padded = i32("head_dim_padded");
  d.total_num_pages = i32("total_num_pages");
  d.page_size = i32("page_size");
  d.kv_packing = i32("kv_packing");
  d.kv_heads_x2 = i32("kv_heads_x2");
  d.max_num_seqs = i32("max_num_seqs");
  d.pages_per_seq = i32("pages_per_seq");
  d.use_causal_mask = i32("use_causal_mask");
  d.skip_kv_update = i32("skip_kv_update");
  d.sliding_window = i32("sliding_window");
  d.has_soft_cap = i32("has_soft_cap");
  d.soft_cap = static_cast<float>(f.at("soft_cap"));
  d.sm_scale = static_cast<float>(f.at("sm_scale"));
  d.q_scale = static_cast<float>(f.at("q_scale"));
  d.k_scale = static_cast<float>(f.at("k_scale"));
  d.v_scale = static_cast<float>(f.at("v_scale"));
  d.path = RPA_PATH_AUTO;
  d.decode_query_size = 1;

  int st = rpa_validate_desc(&d);
  if (st != RPA_OK) {
    std::fprintf(stderr, "rpa_validate_desc: %s (%d)\n", rpa_status_str(st), st);
    return 1;
  }
  hipStream_t s;
  HIP_OK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
  const std::vector<char> hq = read_file(dir + "/q.bin"), hk = read_file(dir + "/k.bin"),
                          hv = read_file(dir + "/v.bin"), hc = read_file(dir + "/kv_cache.bin"),
                          hkl = read_file(dir + "/kv_lens.bin"),
                          hpi = read_file(dir + "/page_indices.bin"),
                          hcu = read_file(dir + "/cu_q_lens.bin"),
                          hdi = read_file(dir + "/distribution.bin");
  DevBuf q = upload(hq, s), k = upload(hk, s), v = upload(hv, s);
  DevBuf cache = upload(hc, s), cache2 = upload(hc, s);
  DevBuf kl = upload(hkl, s), pi = upload(hpi, s), cu = upload(hcu, s), di = upload(hdi, s);
  const int out_bytes = d.out_dtype == RPA_DTYPE_F32 ? 4 : 2;
  DevBuf out, out2, lse;
  out.n = out2.n = static_cast<size_t>(d.max_num_tokens) * d.num_q_heads * d.head_dim * out_bytes;
  lse.n = static_cast<size_t>(d.max_num_tokens) * d.num_q_heads * sizeof(float);
  HIP_OK(hipMalloc(&out.p, out.n));
  HIP_OK(hipMalloc(&out2.p, out2.n));
  HIP_OK(hipMalloc(&lse.p, lse.n));
  HIP_OK(hipMemsetAsync(out.p, 0, out.n, s));
  HIP_OK(hipMemsetAsync(out2.p, 0, out2.n, s));
  HIP_OK(hipMemsetAsync(lse.p, 0, lse.n, s));
  // The caller owns the workspace: rpa_workspace_size bytes, no initialisation.
  const size_t ws_bytes = rpa_workspace_size(&d);
  void* ws = nullptr;
  HIP_OK(hipMalloc(&ws, ws_bytes > 0 ? ws_bytes : 16));

  st = rpa_forward(&d, q.p, k.p, v.p, cache.p, static_cast<const int32_t*>(kl.p),
                   static_cast<const int32_t*>(pi.p), static_cast<const int32_t*>(cu.p),
                   static_cast<const int32_t*>(di.p), out.p, ws, ws_bytes, s);
  if (st != RPA_OK) {
    std::fprintf(stderr, "rpa_forward: %s (%d)\n", rpa_status_str(st), st);
    return 1;
  }
  st = rpa_forward_lse(&d, q.p, k.p, v.p, cache2.p, static_cast<const int32_t*>(kl.p),
                       static_cast<const int32_t*>(pi.p), static_cast<const int32_t*>(cu.p),
                       static_cast<const int32_t*>(di.p), out2.p, static_cast<float*>(lse.p),
                       ws, ws_bytes, s);
  if (st != RPA_OK) {
    std::fprintf(stderr, "rpa_forward_lse: %s (%d)\n", rpa_status_str(st), st);
    return 1;
  }
  // A short workspace is refused, not written through.
  if (ws_bytes > 0) {
    st = rpa_forward(&d, q.p, k.p, v.p, cache.p, static_cast<const int32_t*>(kl.p),
                     static_cast<const int32_t*>(pi.p), static_cast<const int32_t*>(cu.p),
                     static_cast<const int32_t*>(di.p), out.p, ws, ws_bytes - 1, s);
    if (st != RPA_ERR_WORKSPACE) {
      std::fprintf(stderr, "short workspace: expected RPA_ERR_WORKSPACE, got %d\n", st);
      return 1;
    }
  }
  write_file(dir + "/out.bin", download(out, s));
  write_file(dir + "/cache.bin", download(cache, s));
  write_file(dir + "/out_lse.bin", download(out2, s));
  write_file(dir + "/lse.bin", download(lse, s));
  write_file(dir + "/cache_lse.bin", download(cache2, s));
  for (void* p : {q.p, k.p, v.p, cache.p, cache2.p, kl.p, pi.p, cu.p, di.p, out.p, out2.p, lse.p, ws})
    HIP_OK(hipFree(p));
  HIP_OK(hipStreamDestroy(s));
  std::printf("rpa_abi_host ok: workspace %zu bytes\n", ws_bytes);
  return 0;
}
