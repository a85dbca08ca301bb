// Stand-alone C++ driver of the MGN MLP, the counterpart of the reference's
// apps/mgn_fullmlp/pipelined/mgn_fullmlp_pl_cc.cu:12-78 and
// apps/mgn_linears/pipelined/mgn_linears_pl_cc.cu: allocate device buffers,
// run the operator NI times on one stream and print the time per call.
//
//   mgn_mlp_cc [NI=1000] [edge|node|linears] [fused|pipelined|pipelined_split_ln] [M]
//
// Inputs are deterministic (not random) fp16 values; the driver measures
// speed only -- parity is the job of the test suite.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
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

int main(int argc, char** argv) {
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
