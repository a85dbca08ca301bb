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
    d.gfx950 = std::string(prop.gcnArchName).rfind("gfx950", 0) == 0;
    d.valid = true;
  }
  if (!d.gfx950) return fail(GP_ERR_NO_DEVICE, "device %d is not gfx950", dev);
  *dev_out = dev;
  *num_cus = d.num_cus;
  return GP_OK;
}

static bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

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
  if (impl != GP_IMPL_FUSED && impl != GP_IMPL_PIPELINED)
    return fail(GP_ERR_INVALID_ARG, "unknown impl %d", impl);
  if (a.M == 0) return GP_OK;
  int dev = 0, ncu = 0;
  rc = current_device_info(&dev, &ncu);
  if (rc != GP_OK) return rc;
  hipError_t e;
  if (impl == GP_IMPL_FUSED) {
    e = mgn_fused_launch(a, ncu, stream);
    if (e != hipSuccess) return fail_hip(e, "mgn_fused launch");
    return GP_OK;
  }
  return mgn_pipelined_run(a, dev, ncu, stream);
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

}  // extern "C"
