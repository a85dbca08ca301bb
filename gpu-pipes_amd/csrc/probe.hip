// Diagnostics: the dense MFMA rate the device sustains with no memory traffic.
//
// The MFMA-bound kernels of this library run at the board's power cap, where
// the engine clock sits well below the 2.4 GHz the 2.5 PFLOP/s fp16 figure is
// quoted at.  This probe measures the ceiling under the same conditions: every
// SIMD runs two waves that issue back-to-back MFMAs from register operands --
// v_mfma_f32_32x32x16 on eight independent accumulators, or
// v_mfma_f32_16x16x32 on sixteen (the same FLOPs per round) -- for `iters`
// rounds, and stores one value per lane so that nothing is optimised away.
// It has no counterpart in the reference.
#include <hip/hip_runtime.h>

#include "../../include/gpipes.h"
#include "gp_device.hpp"
#include "gp_host.hpp"

namespace gp {
namespace probe {

constexpr int NT = 256;    // four waves per workgroup
constexpr int NACC = 8;    // independent 32x32 accumulators per wave (16x16: twice as many)
constexpr int kBlocksPerCu = 2;  // two workgroups per CU: two waves per SIMD

typedef float f4v __attribute__((ext_vector_type(4)));
__device__ __forceinline__ f4v mma16(F16, h8 a, h8 b, f4v c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f4v mma16(BF16, h8 a, h8 b, f4v c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf8, a), __builtin_bit_cast(bf8, b), c, 0, 0, 0);
}

template <typename E, int SHAPE>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(2, 2))) void mfma_peak_kernel(int64_t iters,
                                                                                                  float* out) {
  // Operands of ordinary data in [-1, 1) (a hash of lane and element), not
  // constants: the matrix core's power depends on the bits it multiplies.
  const int lane = threadIdx.x & 63;
  h8 a, b;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const unsigned ha = (unsigned)(lane * 8 + e + 1) * 2654435761u, hb = (unsigned)(lane * 8 + e + 97) * 2246822519u;
    a[e] = E::cvt1((float)(int)(ha >> 16 & 0xffff) * (1.f / 32768) - 1.f);
    b[e] = E::cvt1((float)(int)(hb >> 16 & 0xffff) * (1.f / 32768) - 1.f);
  }
  // operand values the compiler cannot see through
  asm volatile("" : "+v"(a), "+v"(b));
  float s = 0.f;
  if constexpr (SHAPE == 32) {
    f16x acc[NACC];
#pragma unroll
    for (int j = 0; j < NACC; ++j) acc[j] = f16x{};
    for (int64_t i = 0; i < iters; ++i) {
#pragma unroll
      for (int j = 0; j < NACC; ++j) acc[j] = E::mma(a, b, acc[j]);
    }
#pragma unroll
    for (int j = 0; j < NACC; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) s += acc[j][e];
  } else {
    f4v acc[2 * NACC];
#pragma unroll
    for (int j = 0; j < 2 * NACC; ++j) acc[j] = f4v{};
    for (int64_t i = 0; i < iters; ++i) {
#pragma unroll
      for (int j = 0; j < 2 * NACC; ++j) acc[j] = mma16(E{}, a, b, acc[j]);
    }
#pragma unroll
    for (int j = 0; j < 2 * NACC; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) s += acc[j][e];
  }
  out[(int64_t)blockIdx.x * NT + threadIdx.x] = s;
}

}  // namespace probe
}  // namespace gp

using namespace gp;

extern "C" int gp_probe_mfma(int64_t iters, int dtype, int shape, void* out, int64_t out_floats, int64_t* flops,
                             void* stream) {
  clear_error();
  if (iters < 1 || iters > (int64_t(1) << 40)) return fail(GP_ERR_INVALID_ARG, "iters must be in [1, 2^40]");
  if (dtype != GP_DTYPE_F16 && dtype != GP_DTYPE_BF16) return fail(GP_ERR_INVALID_ARG, "unknown dtype %d", dtype);
  if (shape != 32 && shape != 16) return fail(GP_ERR_INVALID_ARG, "shape must be 32 (32x32x16) or 16 (16x16x32)");
  if (!out || !flops) return fail(GP_ERR_INVALID_ARG, "out and flops must be non-NULL");
  int dev = 0, ncu = 0;
  if (int rc = current_device_info(&dev, &ncu)) return rc;
  const int64_t grid = (int64_t)probe::kBlocksPerCu * ncu;
  if (out_floats < grid * probe::NT)
    return fail(GP_ERR_INVALID_ARG, "out must hold %lld floats", (long long)(grid * probe::NT));
  hipStream_t s = (hipStream_t)stream;
  auto kern = dtype == GP_DTYPE_BF16 ? (shape == 32 ? probe::mfma_peak_kernel<BF16, 32> : probe::mfma_peak_kernel<BF16, 16>)
                                     : (shape == 32 ? probe::mfma_peak_kernel<F16, 32> : probe::mfma_peak_kernel<F16, 16>);
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(probe::NT), 0, s, iters, (float*)out);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail_hip(e, "MFMA probe launch");
  *flops = grid * (probe::NT / kWave) * iters * probe::NACC * (2LL * 32 * 32 * 16);  // either shape
  return GP_OK;
}
