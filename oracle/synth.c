/* Synthetic workload inputs on the host -- TEST INFRASTRUCTURE ONLY.
 *
 * The C restatement of the device generator behind gp_fill_normal: element e
 * is normal (e % 4) of group g = e / 4, from Philox-4x32-10 (Salmon, Moraes,
 * Dror, Shaw, SC 2011) of counter {g lo, g hi, 0, 0} under key {seed lo,
 * seed hi}, and Box-Muller on the word pairs (x0, x1) and (x2, x3):
 * u1 = ((x >> 8) + 1) / 2^24, u2 = (x >> 8) / 2^24, r = sqrt(-2 ln u1),
 * (r cos 2 pi u2, r sin 2 pi u2).  The logarithm, sine, cosine, reciprocal
 * and square root use fp32 multiplies, adds and fused multiply-adds only
 * (series and Newton steps), built with -ffp-contract=off, so every step
 * rounds as on the device.  Philox is pinned by its published known-answer
 * vectors, the transforms by the closed forms (tests/test_synth.py).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#include "oracle.h"

static const uint32_t kM0 = 0xD2511F53u, kM1 = 0xCD9E8D57u;
static const uint32_t kW0 = 0x9E3779B9u, kW1 = 0xBB67AE85u;

void oracle_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]) {
  uint32_t c0 = ctr[0], c1 = ctr[1], c2 = ctr[2], c3 = ctr[3], k0 = key[0], k1 = key[1];
  for (int r = 0; r < 10; ++r) {
    if (r > 0) {
      k0 += kW0;
      k1 += kW1;
    }
    const uint64_t p0 = (uint64_t)kM0 * c0, p1 = (uint64_t)kM1 * c2;
    const uint32_t n0 = (uint32_t)(p1 >> 32) ^ c1 ^ k0, n1 = (uint32_t)p1;
    const uint32_t n2 = (uint32_t)(p0 >> 32) ^ c3 ^ k1, n3 = (uint32_t)p0;
    c0 = n0;
    c1 = n1;
    c2 = n2;
    c3 = n3;
  }
  out[0] = c0;
  out[1] = c1;
  out[2] = c2;
  out[3] = c3;
}

static float bits_f(uint32_t b) {
  float f;
  memcpy(&f, &b, 4);
  return f;
}

static uint32_t f_bits(float f) {
  uint32_t b;
  memcpy(&b, &f, 4);
  return b;
}

/* 1 / d for d in [1.7, 2.5]: four Newton steps from 1/2. */
static float recip_near2(float d) {
  float y = 0.5f;
  for (int i = 0; i < 4; ++i) {
    const float e = fmaf(-d, y, 1.0f);
    y = fmaf(y, e, y);
  }
  return y;
}

/* ln u for u in (0, 1]: ln m = 2 atanh((m - 1) / (m + 1)) to s^11. */
float oracle_log_unit(float u) {
  const uint32_t b = f_bits(u);
  int e = (int)(b >> 23) - 127;
  float m = bits_f((b & 0x7FFFFFu) | 0x3F800000u);
  if (m > 1.41421356f) {
    m = m * 0.5f;
    e += 1;
  }
  const float f = m - 1.0f;
  const float s = f * recip_near2(2.0f + f);
  const float z = s * s;
  float p = fmaf(z, 0.0909090936f, 0.111111112f);
  p = fmaf(z, p, 0.142857149f);
  p = fmaf(z, p, 0.200000003f);
  p = fmaf(z, p, 0.333333343f);
  const float two_s = 2.0f * s;
  const float lm = fmaf(two_s * z, p, two_s);
  return fmaf((float)e, 0.693147182f, lm);
}

/* sqrt v for v in [0, 34]: three Newton steps of 1 / sqrt v, then v / sqrt v. */
float oracle_sqrt_small(float v) {
  if (v == 0.0f) return 0.0f;
  float y = bits_f(0x5F3759DFu - (f_bits(v) >> 1));
  const float h = 0.5f * v;
  for (int i = 0; i < 3; ++i) {
    const float t = y * y;
    y = y * fmaf(-h, t, 1.5f);
  }
  return v * y;
}

/* sin a and cos a for a in [0, pi/2): Taylor series to a^15 and a^14. */
void oracle_sincos_quarter(float a, float* s, float* c) {
  const float a2 = a * a;
  float p = fmaf(a2, -7.64716373e-13f, 1.60590438e-10f);
  p = fmaf(a2, p, -2.50521084e-08f);
  p = fmaf(a2, p, 2.75573192e-06f);
  p = fmaf(a2, p, -1.98412698e-04f);
  p = fmaf(a2, p, 8.33333333e-03f);
  p = fmaf(a2, p, -1.66666667e-01f);
  *s = fmaf(a * a2, p, a);
  float q = fmaf(a2, -1.14707456e-11f, 2.08767570e-09f);
  q = fmaf(a2, q, -2.75573192e-07f);
  q = fmaf(a2, q, 2.48015873e-05f);
  q = fmaf(a2, q, -1.38888889e-03f);
  q = fmaf(a2, q, 4.16666667e-02f);
  q = fmaf(a2, q, -0.5f);
  *c = fmaf(a2, q, 1.0f);
}

static void box_muller(uint32_t x1, uint32_t x2, float* z0, float* z1) {
  const float u1 = (float)((x1 >> 8) + 1u) * 5.96046448e-08f;
  const float u2 = (float)(x2 >> 8) * 5.96046448e-08f;
  const float r = oracle_sqrt_small(-2.0f * oracle_log_unit(u1));
  const float t = u2 * 4.0f;
  const int q = (int)t;
  const float a = (t - (float)q) * 1.57079637f;
  float s, c, sn, cs;
  oracle_sincos_quarter(a, &s, &c);
  switch (q) {
    case 0: sn = s; cs = c; break;
    case 1: sn = c; cs = -s; break;
    case 2: sn = -s; cs = -c; break;
    default: sn = -c; cs = s; break;
  }
  *z0 = r * cs;
  *z1 = r * sn;
}

static void normals4(uint64_t g, uint64_t seed, float z[4]) {
  const uint32_t ctr[4] = {(uint32_t)g, (uint32_t)(g >> 32), 0u, 0u};
  const uint32_t key[2] = {(uint32_t)seed, (uint32_t)(seed >> 32)};
  uint32_t x[4];
  oracle_philox4x32_10(ctr, key, x);
  box_muller(x[0], x[1], &z[0], &z[1]);
  box_muller(x[2], x[3], &z[2], &z[3]);
}

void oracle_normal_f32(int64_t n, uint64_t seed, uint64_t offset, float* dst) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) {
    const uint64_t e = offset + (uint64_t)i;
    float z[4];
    normals4(e / 4, seed, z);
    dst[i] = z[e % 4];
  }
}

/* float -> bfloat16, round to nearest even (finite inputs). */
static uint16_t f2bf(float f) {
  const uint32_t b = f_bits(f);
  return (uint16_t)((b + 0x7FFFu + ((b >> 16) & 1u)) >> 16);
}

void oracle_normal_16(int64_t n, uint64_t seed, uint64_t offset, int bf16, uint16_t* dst) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) {
    const uint64_t e = offset + (uint64_t)i;
    float z[4];
    normals4(e / 4, seed, z);
    dst[i] = bf16 ? f2bf(z[e % 4]) : oracle_f2h(z[e % 4]);
  }
}
