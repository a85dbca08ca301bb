// C ABI entry points (include/gpipes.h): argument validation, error
// reporting and dispatch to the gfx950 kernels.
//
// Error behaviour differs from the reference on purpose: the reference
// checks device/contiguity with TORCH_CHECK and shapes with assert()
// (apps/mgn_fullmlp/pipelined/mgn_fullmlp_pl_ext.cu:36-50), which either
// throws or aborts; here every failure is a negative return code plus a
// message from gp_last_error(), and the process is never aborted.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <mutex>
#include <string>

#include "../../include/gpipes.h"
#include "gp_host.hpp"
#include "gp_kernels.hpp"

namespace gp {

static thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int fail_hip(hipError_t e, const char* what) {
  return fail(GP_ERR_HIP, "%s: %s (%d)", what, hipGetErrorString(e), (int)e);
}

void clear_error() { g_last_error.clear(); }

// Per-device properties, queried once per device.
struct DevInfo {
  bool valid = false;
  int num_cus = 0;
  bool gfx950 = false;
};
static std::mutex g_dev_mu;
static DevInfo g_dev[64];

int current_device_info(int* dev_out, int* num_cus) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail_hip(e, "hipGetDevice");
  if (dev < 0 || dev >= 64) return fail(GP_ERR_NO_DEVICE, "device index %d out of range", dev);
  std::lock_guard<std::mutex> lk(g_dev_mu);
  DevInfo& d = g_dev[dev];
  if (!d.valid) {
    hipDeviceProp_t prop;
    e = hipGetDeviceProperties(&prop, dev);
    if (e != hipSuccess) return fail_hip(e, "hipGetDeviceProperties");
    d.num_cus = prop.multiProcessorCount;
    // GPIPES_NUM_CUS=n sizes every launch for n CUs instead of all of them
    // (a caller sharing the GPU, or a measurement on part of the chip).
    if (const char* v = getenv("GPIPES_NUM_CUS")) {
      const int n = atoi(v);
      if (n >= 1 && n < d.num_cus) d.num_cus = n;
    }
    d.gfx950 = std::string(prop.gcnArchName).rfind("gfx950", 0) == 0;
    d.valid = true;
  }
  if (!d.gfx950) return fail(GP_ERR_NO_DEVICE, "device %d is not gfx950", dev);
  *dev_out = dev;
  *num_cus = d.num_cus;
  return GP_OK;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

int check_mgn_args(const MgnArgs& a) {
  if (a.M < 0) return fail(GP_ERR_INVALID_ARG, "M must be >= 0 (got %lld)", (long long)a.M);
  if (a.K != 128 && a.K != 256 && a.K != 384)
    return fail(GP_ERR_SHAPE, "K must be 128, 256 or 384 (got %lld)", (long long)a.K);
  if (a.M > (int64_t(1) << 40)) return fail(GP_ERR_SHAPE, "M too large (%lld)", (long long)a.M);
  const void* req[] = {a.w1, a.b1, a.w2, a.b2, a.w3, a.b3};
  const char* names[] = {"w1", "b1", "w2", "b2", "w3", "b3"};
  for (int i = 0; i < 6; ++i)
    if (!req[i]) return fail(GP_ERR_INVALID_ARG, "%s is NULL", names[i]);
  if ((a.gamma == nullptr) != (a.beta == nullptr))
    return fail(GP_ERR_INVALID_ARG, "gamma and beta must both be set or both be NULL");
  if (a.M > 0 && (!a.x || !a.out)) return fail(GP_ERR_INVALID_ARG, "x and out must be non-NULL when M > 0");
  if (a.M > 0 && (!aligned16(a.x) || !aligned16(a.out)))
    return fail(GP_ERR_ALIGN, "x and out must be 16-byte aligned");
  if (!aligned16(a.w1) || !aligned16(a.w2) || !aligned16(a.w3))
    return fail(GP_ERR_ALIGN, "w1, w2 and w3 must be 16-byte aligned");
  if (!(a.eps >= 0.f)) return fail(GP_ERR_INVALID_ARG, "eps must be >= 0");
  return GP_OK;
}

int run_mgn(const MgnArgs& a, int impl, hipStream_t stream) {
  clear_error();
  int rc = check_mgn_args(a);
  if (rc != GP_OK) return rc;
  if (impl != GP_IMPL_FUSED && impl != GP_IMPL_PIPELINED && impl != GP_IMPL_PIPELINED_SPLIT_LN)
    return fail(GP_ERR_INVALID_ARG, "unknown impl %d", impl);
  if (a.dtype != GP_DTYPE_F16 && a.dtype != GP_DTYPE_BF16) return fail(GP_ERR_INVALID_ARG, "unknown dtype %d", a.dtype);
  if (a.dtype == GP_DTYPE_BF16 && impl != GP_IMPL_FUSED)
    return fail(GP_ERR_INVALID_ARG, "bf16 runs on the fused kernel (impl %d) only", GP_IMPL_FUSED);
  if (a.M == 0) return GP_OK;
  int dev = 0, ncu = 0;
  rc = current_device_info(&dev, &ncu);
  if (rc != GP_OK) return rc;
  if (impl == GP_IMPL_FUSED) {
    MgnArgs f = a;
    rc = status_acquire(dev, stream, &f.status, &f.epoch);
    if (rc != GP_OK) return rc;
    f.spin_limit = (int)wait_limit(0);
    hipError_t e = mgn_fused_launch(f, ncu, stream);
    if (e != hipSuccess) return fail_hip(e, "mgn_fused launch");
    return GP_OK;
  }
  return mgn_pipelined_run(a, impl == GP_IMPL_PIPELINED_SPLIT_LN, dev, ncu, stream);
}

// Common prologue of the stage-level entry points.
static int stage_prologue(int64_t M, int* dev, int* ncu) {
  clear_error();
  if (M < 0) return fail(GP_ERR_INVALID_ARG, "M must be >= 0 (got %lld)", (long long)M);
  if (M > (int64_t(1) << 40)) return fail(GP_ERR_SHAPE, "M too large (%lld)", (long long)M);
  if (M == 0) return 1;  // nothing to do
  int rc = current_device_info(dev, ncu);
  return rc;
}

static int need(const void* p, const char* name, bool align = true) {
  if (!p) return fail(GP_ERR_INVALID_ARG, "%s is NULL", name);
  if (align && !aligned16(p)) return fail(GP_ERR_ALIGN, "%s must be 16-byte aligned", name);
  return GP_OK;
}

}  // namespace gp

using namespace gp;

extern "C" {

int gp_version(void) { return 0x000100; }

const char* gp_last_error(void) { return g_last_error.c_str(); }

int gp_mgn_mlp_out(int64_t M, int64_t K, const void* x, const void* w1, const void* b1, const void* w2,
                   const void* b2, const void* w3, const void* b3, const void* gamma, const void* beta,
                   float eps, void* out, int impl, void* stream) {
  MgnArgs a{M, K, x, w1, b1, w2, b2, w3, b3, gamma, beta, eps, out};
  return run_mgn(a, impl, (hipStream_t)stream);
}

int gp_mgn_mlp_dtype_out(int64_t M, int64_t K, const void* x, const void* w1, const void* b1, const void* w2,
                         const void* b2, const void* w3, const void* b3, const void* gamma, const void* beta,
                         float eps, void* out, int impl, int dtype, void* stream) {
  MgnArgs a{M, K, x, w1, b1, w2, b2, w3, b3, gamma, beta, eps, out};
  a.dtype = dtype;
  return run_mgn(a, impl, (hipStream_t)stream);
}

int gp_linear_out(int64_t M, int64_t K, const void* x, const void* w, const void* b, const void* acc, int act,
                  void* out, void* stream) {
  int dev = 0, ncu = 0;
  if (K != 128 && K != 256 && K != 384) return fail(GP_ERR_SHAPE, "K must be 128, 256 or 384 (got %lld)", (long long)K);
  if (act < GP_ACT_NONE || act > GP_ACT_SIGMOID) return fail(GP_ERR_INVALID_ARG, "unknown act %d", act);
  int rc = need(w, "w");
  if (rc) return rc;
  rc = stage_prologue(M, &dev, &ncu);
  if (rc) return rc < 0 ? rc : GP_OK;
  if ((rc = need(x, "x")) || (rc = need(out, "out"))) return rc;
  if (acc && !aligned16(acc)) return fail(GP_ERR_ALIGN, "acc must be 16-byte aligned");
  LinearArgs a{M, K, x, w, b, acc, nullptr, nullptr, 0.f, act, out};
  hipError_t e = linear_launch(a, ncu, (hipStream_t)stream);
  return e == hipSuccess ? GP_OK : fail_hip(e, "linear launch");
}

int gp_linear_layer_norm_out(int64_t M, int64_t K, const void* x, const void* w, const void* b, const void* gamma,
                             const void* beta, float eps, void* out, void* stream) {
  int dev = 0, ncu = 0;
  if (K != 128 && K != 256 && K != 384) return fail(GP_ERR_SHAPE, "K must be 128, 256 or 384 (got %lld)", (long long)K);
  int rc = need(w, "w");
  if (rc) return rc;
  if ((rc = need(gamma, "gamma", false)) || (rc = need(beta, "beta", false))) return rc;
  if (!(eps >= 0.f)) return fail(GP_ERR_INVALID_ARG, "eps must be >= 0");
  rc = stage_prologue(M, &dev, &ncu);
  if (rc) return rc < 0 ? rc : GP_OK;
  if ((rc = need(x, "x")) || (rc = need(out, "out"))) return rc;
  LinearArgs a{M, K, x, w, b, nullptr, gamma, beta, eps, GP_ACT_NONE, out};
  hipError_t e = linear_launch(a, ncu, (hipStream_t)stream);
  return e == hipSuccess ? GP_OK : fail_hip(e, "linear+LayerNorm launch");
}

int gp_layer_norm_out(int64_t M, int64_t D, const void* x, const void* gamma, const void* beta, float eps, void* out,
                      void* stream) {
  int dev = 0, ncu = 0;
  if (D != 128 && D != 256 && D != 512 && D != 1024)
    return fail(GP_ERR_SHAPE, "D must be 128, 256, 512 or 1024 (got %lld)", (long long)D);
  if (!(eps >= 0.f)) return fail(GP_ERR_INVALID_ARG, "eps must be >= 0");
  int rc = stage_prologue(M, &dev, &ncu);
  if (rc) return rc < 0 ? rc : GP_OK;
  if ((rc = need(x, "x")) || (rc = need(out, "out"))) return rc;
  hipError_t e = layer_norm_launch(M, D, x, gamma, beta, eps, out, ncu, (hipStream_t)stream);
  return e == hipSuccess ? GP_OK : fail_hip(e, "layer_norm launch");
}

int gp_add_out(int64_t M, int64_t N, const void* a, const void* b, void* c, void* stream) {
  int dev = 0, ncu = 0;
  if (N <= 0 || N % 8 || N > (1 << 20)) return fail(GP_ERR_SHAPE, "N must be a positive multiple of 8");
  int rc = stage_prologue(M, &dev, &ncu);
  if (rc) return rc < 0 ? rc : GP_OK;
  if ((rc = need(a, "a")) || (rc = need(b, "b")) || (rc = need(c, "c"))) return rc;
  hipError_t e = add_launch(M, N, a, b, c, ncu, (hipStream_t)stream);
  return e == hipSuccess ? GP_OK : fail_hip(e, "add launch");
}

int gp_concat_out(int64_t M, int64_t N0, int64_t N1, const void* a, const void* b, void* c, void* stream) {
  int dev = 0, ncu = 0;
  if (N0 <= 0 || N1 <= 0 || N0 % 8 || N1 % 8 || N0 + N1 > (1 << 20))
    return fail(GP_ERR_SHAPE, "N0 and N1 must be positive multiples of 8");
  int rc = stage_prologue(M, &dev, &ncu);
  if (rc) return rc < 0 ? rc : GP_OK;
  if ((rc = need(a, "a")) || (rc = need(b, "b")) || (rc = need(c, "c"))) return rc;
  hipError_t e = concat_launch(M, N0, N1, a, b, c, ncu, (hipStream_t)stream);
  return e == hipSuccess ? GP_OK : fail_hip(e, "concat launch");
}

int gp_pipe_ident(int64_t M, const void* x, void* out, int max_pipes, void* stream) {
  int dev = 0, ncu = 0;
  int rc = stage_prologue(M, &dev, &ncu);
  if (rc) return rc < 0 ? rc : GP_OK;
  if ((rc = need(x, "x")) || (rc = need(out, "out"))) return rc;
  return pipe_route_run(M, x, out, nullptr, GP_ROUTE_IDENT, max_pipes, dev, ncu, (hipStream_t)stream);
}

int gp_pipe_route(int64_t M, const void* x, void* out, void* out2, int route, int max_pipes, void* stream) {
  int dev = 0, ncu = 0;
  if (route != GP_ROUTE_IDENT && route != GP_ROUTE_BROADCAST && route != GP_ROUTE_SPLIT && route != GP_ROUTE_DRAIN &&
      route != GP_ROUTE_HANDOFF && route != GP_ROUTE_RELOAD)
    return fail(GP_ERR_INVALID_ARG, "unknown route %d", route);
  if (route == GP_ROUTE_HANDOFF) {
    clear_error();
    if (x != nullptr) return fail(GP_ERR_INVALID_ARG, "the hand-off route takes no input (x must be NULL)");
    if (M > 0 && out == nullptr) return fail(GP_ERR_INVALID_ARG, "out is NULL");
    if ((uintptr_t)out % 4 != 0) return fail(GP_ERR_ALIGN, "out (uint32 checksums) must be 4-byte aligned");
  }
  int rc = stage_prologue(M, &dev, &ncu);
  if (rc) return rc < 0 ? rc : GP_OK;
  if (route == GP_ROUTE_HANDOFF)
    return pipe_route_run(M, nullptr, out, nullptr, route, max_pipes, dev, ncu, (hipStream_t)stream);
  if ((rc = need(x, "x")) || (rc = need(out, "out"))) return rc;
  if (route == GP_ROUTE_BROADCAST && (rc = need(out2, "out2"))) return rc;
  return pipe_route_run(M, x, out, out2, route, max_pipes, dev, ncu, (hipStream_t)stream);
}

int gp_phase_timers_read(void* dst, int64_t bytes) {
  clear_error();
  switch (mgn_phase_timers_read(dst, bytes)) {
    case 0: return GP_OK;
    case -1: return fail(GP_ERR_INVALID_ARG, "dst must hold %d bytes", 256 * 8 * 12 * 8);
    case -2: return fail(GP_ERR_HIP, "copy of the phase timers failed");
    default: return fail(GP_ERR_INVALID_ARG, "this library was built without phase timers (libgpipes_phase.so has them)");
  }
}

int gp_pipeline_check(void* stream) {
  clear_error();
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail_hip(e, "hipGetDevice");
  unsigned long long* word = nullptr;
  uint32_t epoch = 0;
  int rc = status_last(dev, (hipStream_t)stream, &word, &epoch);
  if (rc != GP_OK) return rc;
  e = hipStreamSynchronize((hipStream_t)stream);
  if (e != hipSuccess) return fail_hip(e, "hipStreamSynchronize");
  unsigned long long err = 0;
  e = hipMemcpy(&err, word, sizeof(err), hipMemcpyDeviceToHost);
  if (e != hipSuccess) return fail_hip(e, "hipMemcpy (launch status)");
  if ((uint32_t)(err >> 32) == epoch && (uint32_t)err != 0)
    return fail(GP_ERR_TIMEOUT, "the last launch on this stream failed on the device: %s (error bits 0x%x)",
                (err & 1) ? "a wait timed out; its outputs are not valid" : "no complete pipeline fitted on one XCD",
                (unsigned)err);
  return GP_OK;
}

int gp_set_wait_limit(int64_t polls) {
  clear_error();
  if (polls < 0 || polls > (int64_t(1) << 30)) return fail(GP_ERR_INVALID_ARG, "polls must be in [0, 2^30]");
  set_wait_limit((long long)polls);
  return GP_OK;
}

int gp_mgn_fullmlp_out(int64_t M, const void* x, const void* w1, const void* b1, const void* w2,
                       const void* b2, const void* w3, const void* b3, const void* gamma, const void* beta,
                       void* out, void* stream) {
  if (!gamma || !beta) return fail(GP_ERR_INVALID_ARG, "gamma and beta are required");
  MgnArgs a{M, 384, x, w1, b1, w2, b2, w3, b3, gamma, beta, 1e-5f, out};
  return run_mgn(a, GP_IMPL_FUSED, (hipStream_t)stream);
}

int gp_mgn_linears_out(int64_t M, const void* x, const void* w1, const void* b1, const void* w2,
                       const void* b2, const void* w3, const void* b3, void* out, void* stream) {
  MgnArgs a{M, 384, x, w1, b1, w2, b2, w3, b3, nullptr, nullptr, 0.f, out};
  return run_mgn(a, GP_IMPL_FUSED, (hipStream_t)stream);
}

int gp_mgn_edge_gather_out(int64_t E, int64_t N, const void* nf, const void* ef, const void* src, const void* dst,
                           int idx_bytes, const void* w1, const void* b1, const void* w2, const void* b2,
                           const void* w3, const void* b3, const void* gamma, const void* beta, float eps, void* out,
                           void* stream) {
  clear_error();
  if (idx_bytes != 4 && idx_bytes != 8) return fail(GP_ERR_INVALID_ARG, "idx_bytes must be 4 or 8 (got %d)", idx_bytes);
  if (E < 0 || N < 0) return fail(GP_ERR_INVALID_ARG, "E and N must be >= 0");
  if (E > 0 && N < 1) return fail(GP_ERR_SHAPE, "a non-empty edge set needs N >= 1 nodes");
  if (N * 256 > (int64_t(1) << 31) - 16) return fail(GP_ERR_SHAPE, "N too large (%lld nodes; at most 8388607)", (long long)N);
  MgnArgs a{E, 384, ef, w1, b1, w2, b2, w3, b3, gamma, beta, eps, out};
  a.nf = nf;
  a.N = N;
  a.src = src;
  a.dst = dst;
  a.idx_bytes = idx_bytes;
  int rc = check_mgn_args(a);
  if (rc != GP_OK) return rc;
  if (E == 0) return GP_OK;
  if (!nf || !src || !dst) return fail(GP_ERR_INVALID_ARG, "nf, src and dst must be non-NULL when E > 0");
  if (!aligned16(nf) || !aligned16(src) || !aligned16(dst))
    return fail(GP_ERR_ALIGN, "nf, src and dst must be 16-byte aligned");
  int dev = 0, ncu = 0;
  rc = current_device_info(&dev, &ncu);
  if (rc != GP_OK) return rc;
  rc = status_acquire(dev, (hipStream_t)stream, &a.status, &a.epoch);
  if (rc != GP_OK) return rc;
  a.spin_limit = (int)wait_limit(0);
  hipError_t e = mgn_fused_launch(a, ncu, (hipStream_t)stream);
  return e == hipSuccess ? GP_OK : fail_hip(e, "mgn_edge_gather launch");
}

}  // extern "C"
