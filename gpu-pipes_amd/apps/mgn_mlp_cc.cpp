// Stand-alone C++ driver of the MGN MLP, the counterpart of the reference's
// apps/mgn_fullmlp/pipelined/mgn_fullmlp_pl_cc.cu:12-78 and
// apps/mgn_linears/pipelined/mgn_linears_pl_cc.cu: allocate device buffers,
// run the operator NI times on one stream and print the time per call.
//
//   mgn_mlp_cc [NI=1000] [edge|node|linears] [fused|pipelined|pipelined_split_ln] [M]
//
// Inputs are deterministic (not random) fp16 values; the driver measures
// speed only.
//
//   mgn_mlp_cc check DIR
//
// runs one call through the C++ wrappers of include/gpipes.hpp on inputs read
// from DIR (raw fp16 files x, w1, b1, w2, b2, w3, b3 [, gamma, beta] and a
// text file `shape` holding "M K ln impl") and writes the result to DIR/out:
// mgn_fullmlp_out / mgn_linears_out for K = 384 with the fused impl (the
// reference's operator names), mgn_mlp_out otherwise.  It then checks that a
// misaligned x makes the wrapper throw gpipes::Error with GP_ERR_ALIGN.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/gpipes.hpp"

#define HIP_OK(call)                                                                        \
  do {                                                                                      \
    hipError_t e_ = (call);                                                                 \
    if (e_ != hipSuccess) {                                                                 \
      std::fprintf(stderr, "%s:%d: %s: %s\n", __FILE__, __LINE__, #call, hipGetErrorString(e_)); \
      std::exit(1);                                                                         \
    }                                                                                       \
  } while (0)

static uint16_t to_half(float f) {
  _Float16 h = (_Float16)f;
  uint16_t u;
  std::memcpy(&u, &h, 2);
  return u;
}

static void* upload(const std::vector<uint16_t>& v) {
  void* p = nullptr;
  HIP_OK(hipMalloc(&p, v.size() * 2));
  HIP_OK(hipMemcpy(p, v.data(), v.size() * 2, hipMemcpyHostToDevice));
  return p;
}

// A fixed pseudo-random fill (LCG) scaled to +-scale.
static std::vector<uint16_t> fill(size_t n, float scale, uint32_t seed) {
  std::vector<uint16_t> v(n);
  uint32_t s = seed * 2654435761u + 1;
  for (size_t i = 0; i < n; ++i) {
    s = s * 1664525u + 1013904223u;
    v[i] = to_half(scale * ((float)(s >> 8) * (2.f / 16777216.f) - 1.f));
  }
  return v;
}

static std::vector<uint16_t> read_file(const std::string& path, size_t n) {
  std::vector<uint16_t> v(n);
  FILE* f = std::fopen(path.c_str(), "rb");
  if (!f || std::fread(v.data(), 2, n, f) != n) {
    std::fprintf(stderr, "cannot read %zu halves from %s\n", n, path.c_str());
    std::exit(1);
  }
  std::fclose(f);
  return v;
}

static int check_mode(const std::string& dir) {
  long long M = 0, K = 0;
  int ln = 0, impl = GP_IMPL_FUSED;
  FILE* f = std::fopen((dir + "/shape").c_str(), "r");
  if (!f || std::fscanf(f, "%lld %lld %d %d", &M, &K, &ln, &impl) != 4) {
    std::fprintf(stderr, "cannot read %s/shape\n", dir.c_str());
    return 1;
  }
  std::fclose(f);
  void* x = upload(read_file(dir + "/x", (size_t)M * K));
  void* w1 = upload(read_file(dir + "/w1", (size_t)K * 128));
  void* b1 = upload(read_file(dir + "/b1", 128));
  void* w2 = upload(read_file(dir + "/w2", 128 * 128));
  void* b2 = upload(read_file(dir + "/b2", 128));
  void* w3 = upload(read_file(dir + "/w3", 128 * 128));
  void* b3 = upload(read_file(dir + "/b3", 128));
  void* gamma = ln ? upload(read_file(dir + "/gamma", 128)) : nullptr;
  void* beta = ln ? upload(read_file(dir + "/beta", 128)) : nullptr;
  void* out = nullptr;
  HIP_OK(hipMalloc(&out, (size_t)M * 128 * 2 + 16));
  hipStream_t s;
  HIP_OK(hipStreamCreate(&s));
  try {
    if (K == 384 && impl == GP_IMPL_FUSED && ln) {
      gpipes::mgn_fullmlp_out(M, x, w1, b1, w2, b2, w3, b3, gamma, beta, out, s);
      std::printf("called mgn_fullmlp_out\n");
    } else if (K == 384 && impl == GP_IMPL_FUSED) {
      gpipes::mgn_linears_out(M, x, w1, b1, w2, b2, w3, b3, out, s);
      std::printf("called mgn_linears_out\n");
    } else {
      gpipes::mgn_mlp_out(M, K, x, w1, b1, w2, b2, w3, b3, gamma, beta, out, 1e-5f, impl, s);
      std::printf("called mgn_mlp_out impl %d\n", impl);
    }
    gpipes::pipeline_check(s);
  } catch (const gpipes::Error& e) {
    std::fprintf(stderr, "unexpected: %s\n", e.what());
    return 1;
  }
  std::vector<uint16_t> y((size_t)M * 128);
  HIP_OK(hipMemcpy(y.data(), out, y.size() * 2, hipMemcpyDeviceToHost));
  FILE* o = std::fopen((dir + "/out").c_str(), "wb");
  if (!o || std::fwrite(y.data(), 2, y.size(), o) != y.size()) return 1;
  std::fclose(o);
  // A misaligned input must throw, not abort or launch.
  int code = 0;
  try {
    gpipes::mgn_mlp_out(M, K, (char*)x + 2, w1, b1, w2, b2, w3, b3, gamma, beta, out, 1e-5f, impl, s);
  } catch (const gpipes::Error& e) {
    code = e.code();
  }
  std::printf("misaligned x: error code %d\n", code);
  HIP_OK(hipStreamSynchronize(s));
  return code == GP_ERR_ALIGN ? 0 : 1;
}

int main(int argc, char** argv) {
  if (argc > 2 && !std::strcmp(argv[1], "check")) return check_mode(argv[2]);
  const int ni = argc > 1 ? std::atoi(argv[1]) : 1000;
  const char* which = argc > 2 ? argv[2] : "edge";
  const char* impl_s = argc > 3 ? argv[3] : "fused";
  const bool node = !std::strcmp(which, "node");
  const bool ln = std::strcmp(which, "linears") != 0;
  const int64_t K = node ? 256 : 384;
  const int64_t M = argc > 4 ? std::atoll(argv[4]) : (node ? 262144 : 1048576);
  int impl = GP_IMPL_FUSED;
  if (!std::strcmp(impl_s, "pipelined")) impl = GP_IMPL_PIPELINED;
  if (!std::strcmp(impl_s, "pipelined_split_ln")) impl = GP_IMPL_PIPELINED_SPLIT_LN;
  std::printf("NI: %d  workload: %s  impl: %s  M: %lld  K: %lld\n", ni, which, impl_s, (long long)M, (long long)K);

  void* x = upload(fill((size_t)M * K, 1.f, 1));
  void* w1 = upload(fill((size_t)K * 128, 1.f / 20.f, 2));
  void* w2 = upload(fill(128 * 128, 1.f / 11.f, 3));
  void* w3 = upload(fill(128 * 128, 1.f / 11.f, 4));
  void* b1 = upload(fill(128, 0.05f, 5));
  void* b2 = upload(fill(128, 0.05f, 6));
  void* b3 = upload(fill(128, 0.05f, 7));
  void* gamma = upload(std::vector<uint16_t>(128, to_half(1.f)));
  void* beta = upload(std::vector<uint16_t>(128, to_half(0.f)));
  void* out = nullptr;
  HIP_OK(hipMalloc(&out, (size_t)M * 128 * 2));

  hipStream_t s;
  HIP_OK(hipStreamCreate(&s));
  auto call = [&] {
    gpipes::mgn_mlp_out(M, K, x, w1, b1, w2, b2, w3, b3, ln ? gamma : nullptr, ln ? beta : nullptr, out, 1e-5f, impl,
                        s);
  };
  try {
    for (int i = 0; i < 10; ++i) call();
    if (impl != GP_IMPL_FUSED) gpipes::pipeline_check(s);
    HIP_OK(hipStreamSynchronize(s));
    hipEvent_t e0, e1;
    HIP_OK(hipEventCreate(&e0));
    HIP_OK(hipEventCreate(&e1));
    HIP_OK(hipEventRecord(e0, s));
    for (int i = 0; i < ni; ++i) call();
    HIP_OK(hipEventRecord(e1, s));
    HIP_OK(hipEventSynchronize(e1));
    if (impl != GP_IMPL_FUSED) gpipes::pipeline_check(s);
    float ms = 0.f;
    HIP_OK(hipEventElapsedTime(&ms, e0, e1));
    const double per = ms / ni;
    const double flops = 2.0 * M * (K * 128 + 2 * 128 * 128);
    const double bytes = (double)M * (K + 128) * 2;
    std::printf("Avg latency: %.4f ms, %.3f G rows/s, %.1f TFLOP/s, %.0f GB/s\n", per, M / per / 1e6,
                flops / per / 1e9, bytes / per / 1e6);
  } catch (const gpipes::Error& e) {
    std::fprintf(stderr, "%s\n", e.what());
    return 1;
  }
  return 0;
}
