// Synthetic workload inputs generated on the device: X ~ N(0, 1) from a
// counter-based generator, so that a given (seed, element index) yields the
// same value on the host (oracle/synth.c restates the same steps in C) and on
// any device, independent of launch shape.  No counterpart in the reference,
// whose inputs come from torch's host generator (apps/*/pipelined/val.py).
//
// Element e of the stream is normal (e % 4) of group g = e / 4:
//  * Philox-4x32-10 (Salmon, Moraes, Dror, Shaw, "Parallel random numbers: as
//    easy as 1, 2, 3", SC 2011) of counter {g lo, g hi, 0, 0} under key
//    {seed lo, seed hi} gives four 32-bit words x0..x3;
//  * Box-Muller on (x0, x1) and on (x2, x3): u1 = ((x >> 8) + 1) / 2^24 in
//    (0, 1], u2 = (x >> 8) / 2^24 in [0, 1), r = sqrt(-2 ln u1), and the pair
//    (r cos 2 pi u2, r sin 2 pi u2) is elements 4g + {0, 1} (or {2, 3}).
// The logarithm, sine, cosine, reciprocal and square root are computed from
// fp32 multiplies, adds and fused multiply-adds only (series and Newton
// steps), never contracted by the compiler, so the host and the device
// round every step the same way; the result is then rounded to the element
// type (round to nearest even).
#include <hip/hip_runtime.h>

#include <stdint.h>

#include "../../include/gpipes.h"
#include "gp_host.hpp"

#pragma clang fp contract(off)

namespace gp {
namespace synth {

constexpr uint32_t kM0 = 0xD2511F53u, kM1 = 0xCD9E8D57u;  // Philox-4x32 multipliers
constexpr uint32_t kW0 = 0x9E3779B9u, kW1 = 0xBB67AE85u;  // Weyl key increments

__device__ __forceinline__ void philox4x32_10(uint32_t c[4], uint32_t k0, uint32_t k1) {
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    if (r > 0) {
      k0 += kW0;
      k1 += kW1;
    }
    const uint32_t lo0 = kM0 * c[0], hi0 = __umulhi(kM0, c[0]);
    const uint32_t lo1 = kM1 * c[2], hi1 = __umulhi(kM1, c[2]);
    const uint32_t n0 = hi1 ^ c[1] ^ k0, n2 = hi0 ^ c[3] ^ k1;
    c[0] = n0;
    c[1] = lo1;
    c[2] = n2;
    c[3] = lo0;
  }
}

// 1 / d for d in [1.7, 2.5]: four Newton steps from 1/2.
__device__ __forceinline__ float recip_near2(float d) {
  float y = 0.5f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float e = __builtin_fmaf(-d, y, 1.0f);
    y = __builtin_fmaf(y, e, y);
  }
  return y;
}

// ln u for u in (0, 1]: u = m 2^e with m in [sqrt(1/2), sqrt(2)), ln m =
// 2 atanh(s), s = (m - 1) / (m + 1), by its series to s^11.
__device__ __forceinline__ float log_unit(float u) {
  const uint32_t b = __builtin_bit_cast(uint32_t, u);
  int e = (int)(b >> 23) - 127;
  float m = __builtin_bit_cast(float, (b & 0x7FFFFFu) | 0x3F800000u);
  if (m > 1.41421356f) {
    m = m * 0.5f;
    e += 1;
  }
  const float f = m - 1.0f;
  const float s = f * recip_near2(2.0f + f);
  const float z = s * s;
  float p = __builtin_fmaf(z, 0.0909090936f, 0.111111112f);
  p = __builtin_fmaf(z, p, 0.142857149f);
  p = __builtin_fmaf(z, p, 0.200000003f);
  p = __builtin_fmaf(z, p, 0.333333343f);
  const float two_s = 2.0f * s;
  const float lm = __builtin_fmaf(two_s * z, p, two_s);
  return __builtin_fmaf((float)e, 0.693147182f, lm);
}

// sqrt v for v in [0, 34]: three Newton steps of 1 / sqrt v from the
// exponent-halving first guess, then v / sqrt v.
__device__ __forceinline__ float sqrt_small(float v) {
  if (v == 0.0f) return 0.0f;
  float y = __builtin_bit_cast(float, 0x5F3759DFu - (__builtin_bit_cast(uint32_t, v) >> 1));
  const float h = 0.5f * v;
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    const float t = y * y;
    y = y * __builtin_fmaf(-h, t, 1.5f);
  }
  return v * y;
}

// sin a and cos a for a in [0, pi/2): Taylor series to a^15 and a^14.
__device__ __forceinline__ void sincos_quarter(float a, float* s, float* c) {
  const float a2 = a * a;
  float p = __builtin_fmaf(a2, -7.64716373e-13f, 1.60590438e-10f);
  p = __builtin_fmaf(a2, p, -2.50521084e-08f);
  p = __builtin_fmaf(a2, p, 2.75573192e-06f);
  p = __builtin_fmaf(a2, p, -1.98412698e-04f);
  p = __builtin_fmaf(a2, p, 8.33333333e-03f);
  p = __builtin_fmaf(a2, p, -1.66666667e-01f);
  *s = __builtin_fmaf(a * a2, p, a);
  float q = __builtin_fmaf(a2, -1.14707456e-11f, 2.08767570e-09f);
  q = __builtin_fmaf(a2, q, -2.75573192e-07f);
  q = __builtin_fmaf(a2, q, 2.48015873e-05f);
  q = __builtin_fmaf(a2, q, -1.38888889e-03f);
  q = __builtin_fmaf(a2, q, 4.16666667e-02f);
  q = __builtin_fmaf(a2, q, -0.5f);
  *c = __builtin_fmaf(a2, q, 1.0f);
}

__device__ __forceinline__ void box_muller(uint32_t x1, uint32_t x2, float* z0, float* z1) {
  const float u1 = (float)((x1 >> 8) + 1u) * 5.96046448e-08f;  // 2^-24
  const float u2 = (float)(x2 >> 8) * 5.96046448e-08f;
  const float r = sqrt_small(-2.0f * log_unit(u1));
  const float t = u2 * 4.0f;
  const int q = (int)t;
  const float a = (t - (float)q) * 1.57079637f;
  float s, c;
  sincos_quarter(a, &s, &c);
  float sn, cs;  // sin, cos of 2 pi u2 = (q + a / (pi/2)) pi/2
  if (q == 0) {
    sn = s;
    cs = c;
  } else if (q == 1) {
    sn = c;
    cs = -s;
  } else if (q == 2) {
    sn = -s;
    cs = -c;
  } else {
    sn = -c;
    cs = s;
  }
  *z0 = r * cs;
  *z1 = r * sn;
}

__device__ __forceinline__ uint16_t to_bits(float v, bool bf16) {
  if (bf16) return __builtin_bit_cast(uint16_t, (__bf16)v);
  return __builtin_bit_cast(uint16_t, (_Float16)v);
}

// Thread t of the grid stride takes groups g0 + t, g0 + t + stride, ... and
// writes the elements of each group that fall in [offset, offset + n).
__global__ void fill_normal_kernel(uint16_t* dst, int64_t n, uint64_t seed, uint64_t offset, int bf16) {
  const uint64_t g0 = offset / 4, g1 = (offset + (uint64_t)n + 3) / 4;
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t g = g0 + (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; g < g1; g += stride) {
    uint32_t c[4] = {(uint32_t)g, (uint32_t)(g >> 32), 0u, 0u};
    philox4x32_10(c, (uint32_t)seed, (uint32_t)(seed >> 32));
    float z[4];
    box_muller(c[0], c[1], &z[0], &z[1]);
    box_muller(c[2], c[3], &z[2], &z[3]);
    const uint64_t e0 = 4 * g;
    if (e0 >= offset && e0 + 4 <= offset + (uint64_t)n && ((e0 - offset) & 3) == 0 &&
        (((uintptr_t)(dst + (e0 - offset))) & 7) == 0) {
      const uint32_t lo = (uint32_t)to_bits(z[0], bf16) | ((uint32_t)to_bits(z[1], bf16) << 16);
      const uint32_t hi = (uint32_t)to_bits(z[2], bf16) | ((uint32_t)to_bits(z[3], bf16) << 16);
      *(uint2*)(dst + (e0 - offset)) = make_uint2(lo, hi);
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint64_t e = e0 + j;
        if (e >= offset && e < offset + (uint64_t)n) dst[e - offset] = to_bits(z[j], bf16);
      }
    }
  }
}

}  // namespace synth
}  // namespace gp

extern "C" int gp_fill_normal(void* dst, int64_t n, uint64_t seed, uint64_t offset, int dtype, void* stream) {
  using namespace gp;
  clear_error();
  if (n < 0) return fail(GP_ERR_INVALID_ARG, "n must be >= 0 (got %lld)", (long long)n);
  if (dtype != GP_DTYPE_F16 && dtype != GP_DTYPE_BF16) return fail(GP_ERR_INVALID_ARG, "unknown dtype %d", dtype);
  if (n == 0) return GP_OK;
  if (dst == nullptr) return fail(GP_ERR_INVALID_ARG, "dst is NULL");
  if (((uintptr_t)dst & 1) != 0) return fail(GP_ERR_ALIGN, "dst must be 2-byte aligned");
  if (offset > UINT64_MAX - (uint64_t)n - 4) return fail(GP_ERR_INVALID_ARG, "offset + n overflows");
  int dev = 0, ncu = 0;
  if (const int rc = current_device_info(&dev, &ncu)) return rc;
  const uint64_t groups = (offset + (uint64_t)n + 3) / 4 - offset / 4;
  const uint64_t blocks_needed = (groups + 255) / 256;
  const unsigned blocks = (unsigned)(blocks_needed < 8192 ? blocks_needed : 8192);
  hipLaunchKernelGGL(synth::fill_normal_kernel, dim3(blocks), dim3(256), 0, (hipStream_t)stream, (uint16_t*)dst, n,
                     seed, offset, dtype == GP_DTYPE_BF16 ? 1 : 0);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail_hip(e, "fill_normal_kernel launch");
  return GP_OK;
}
