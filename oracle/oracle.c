/*
 * CPU oracle for the gpu-pipes fused-MLP path -- TEST INFRASTRUCTURE ONLY.
 *
 * This file restates, in plain C with fp32 arithmetic, what the reference's
 * pipelined MLP path computes.  It is the checker for the HIP kernels and the
 * CPU baseline timed by bench.py; nothing in the product library links,
 * loads or calls it.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may use it.
 *
 * Every function names the reference lines it follows.  Each one is pinned by
 * tests/test_oracle.py against checks that do not retype its formula: numpy's
 * binary16 conversion over all 65536 patterns, torch.nn library modules in
 * float64, closed forms, the reference's literal LayerNorm row, and planted
 * mistakes that must fail.
 */
#include "oracle.h"

#include <math.h>
#include <stdint.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* ---------------------------------------------------------------- fp16 --- */

float oracle_h2f(uint16_t h) {
  const uint32_t s = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1fu;
  const uint32_t m = h & 0x3ffu;
  uint32_t bits;
  if (e == 0) {
    if (m == 0) {
      bits = s;
    } else { /* subnormal: renormalise */
      uint32_t mm = m;
      int ee = -1;
      do {
        ++ee;
        mm <<= 1;
      } while ((mm & 0x400u) == 0);
      bits = s | ((uint32_t)(127 - 15 - ee) << 23) | ((mm & 0x3ffu) << 13);
    }
  } else if (e == 31) {
    bits = s | 0x7f800000u | (m << 13);
  } else {
    bits = s | ((e + 127 - 15) << 23) | (m << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

/* Round-to-nearest-even float -> binary16 (IEEE 754-2008). */
uint16_t oracle_f2h(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const uint32_t absx = x & 0x7fffffffu;
  if (absx >= 0x7f800000u) /* inf / nan */
    return (uint16_t)(sign | 0x7c00u | (absx > 0x7f800000u ? 0x200u : 0u));
  if (absx >= 0x477ff000u) /* rounds to >= 65520 -> inf */
    return (uint16_t)(sign | 0x7c00u);
  if (absx < 0x38800000u) { /* below the smallest normal half: subnormal or 0 */
    if (absx < 0x33000000u) return (uint16_t)sign; /* < 2^-25: rounds to 0 */
    const uint32_t e = absx >> 23;
    const uint32_t mant = (absx & 0x7fffffu) | 0x800000u;
    const uint32_t shift = 126 - e; /* 14 .. 24 */
    uint32_t r = mant >> shift;
    const uint32_t rem = mant & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (r & 1u))) ++r;
    return (uint16_t)(sign | r);
  }
  uint32_t r = (absx - 0x38000000u) >> 13; /* rebias exponent, drop 13 bits */
  const uint32_t rem = absx & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) ++r;
  return (uint16_t)(sign | r);
}

void oracle_h2f_array(int64_t n, const uint16_t* src, float* dst) {
  for (int64_t i = 0; i < n; ++i) dst[i] = oracle_h2f(src[i]);
}

void oracle_f2h_array(int64_t n, const float* src, uint16_t* dst) {
  for (int64_t i = 0; i < n; ++i) dst[i] = oracle_f2h(src[i]);
}

/* --------------------------------------------------------------- layers --- */

static float act_apply(float v, int act) {
  switch (act) {
    case ORACLE_ACT_RELU: /* torch.nn.ReLU, common/mlps.py:9-11 */
      return v > 0.f ? v : 0.f;
    case ORACLE_ACT_GELU_TANH: { /* GELU(approximate='tanh'), the BERT FFN activation */
      const float c = 0.7978845608028654f; /* sqrt(2/pi) */
      return 0.5f * v * (1.f + tanhf(c * (v + 0.044715f * v * v * v)));
    }
    case ORACLE_ACT_SIGMOID: /* torch.nn.Sigmoid, common/mlps.py:30 */
      return 1.f / (1.f + expf(-v));
    default:
      return v;
  }
}

/*
 * y[m, :] = act(x[m, :] . W + b), W stored [K, N] row-major.
 * The reference feeds nn.Linear.weight.t().contiguous() as W
 * (apps/mgn_fullmlp/pipelined/val.py:17-19) and applies the epilogue
 * relu(acc + b) (common/pipe_gemm_bias_relu.cuh:173-188) or acc + b
 * (common/pipe_gemm_bias.cuh:32-37).  Accumulation is fp32 here, as the parity bar
 * assumes (the reference GPU path accumulates in fp16,
 * common/pipe_gemm_bias_relu.cuh:43).
 */
void oracle_linear(int64_t M, int64_t K, int64_t N, const float* x, const float* w, const float* b,
                   int act, float* y) {
#pragma omp parallel for schedule(static)
  for (int64_t m = 0; m < M; ++m) {
    float* yr = y + m * N;
    const float* xr = x + m * K;
    for (int64_t n = 0; n < N; ++n) yr[n] = 0.f;
    for (int64_t k = 0; k < K; ++k) {
      const float xv = xr[k];
      const float* wr = w + k * N;
      for (int64_t n = 0; n < N; ++n) yr[n] += xv * wr[n];
    }
    for (int64_t n = 0; n < N; ++n) yr[n] = act_apply(yr[n] + (b ? b[n] : 0.f), act);
  }
}

/*
 * LayerNorm over the last dimension D with biased variance, two-pass:
 * mean = sum(x)/D; var = sum((x-mean)^2)/D; y = (x-mean)/sqrt(var+eps)*g+b.
 * Follows common/layer_norm_v2.cuh:42-70 (eps a parameter here; the reference
 * hard-codes 1e-5 at :62) and torch.nn.LayerNorm (common/mlps.py:16).
 */
void oracle_layer_norm(int64_t M, int64_t D, const float* x, const float* gamma, const float* beta,
                       float eps, float* y) {
#pragma omp parallel for schedule(static)
  for (int64_t m = 0; m < M; ++m) {
    const float* xr = x + m * D;
    float* yr = y + m * D;
    float mean = 0.f;
    for (int64_t d = 0; d < D; ++d) mean += xr[d];
    mean /= (float)D;
    float var = 0.f;
    for (int64_t d = 0; d < D; ++d) {
      const float t = xr[d] - mean;
      var += t * t;
    }
    var /= (float)D;
    const float sd = sqrtf(var + eps);
    for (int64_t d = 0; d < D; ++d) {
      const float g = gamma ? gamma[d] : 1.f;
      const float bb = beta ? beta[d] : 0.f;
      yr[d] = (xr[d] - mean) / sd * g + bb;
    }
  }
}

/*
 * MgnMlp(K, [128, 128, 128], layernorm) forward, common/mlps.py:3-20:
 * Linear+ReLU, Linear+ReLU, Linear (no ReLU on the last layer, :12-14),
 * then LayerNorm(128) when gamma != NULL (:16).  `work` must hold 2*M*128
 * floats.  Rows are processed in blocks so the whole batch need not be
 * materialised between layers.
 */
void oracle_mgn_mlp(int64_t M, int64_t K, const float* x, const float* w1, const float* b1,
                    const float* w2, const float* b2, const float* w3, const float* b3,
                    const float* gamma, const float* beta, float eps, float* out, float* work) {
  const int64_t N = 128;
  float* h1 = work;
  float* h2 = work + M * N;
  oracle_linear(M, K, N, x, w1, b1, ORACLE_ACT_RELU, h1);
  oracle_linear(M, N, N, h1, w2, b2, ORACLE_ACT_RELU, h2);
  if (gamma) {
    oracle_linear(M, N, N, h2, w3, b3, ORACLE_ACT_NONE, h1);
    oracle_layer_norm(M, N, h1, gamma, beta, eps, out);
  } else {
    oracle_linear(M, N, N, h2, w3, b3, ORACLE_ACT_NONE, out);
  }
}

/*
 * BertFfn forward, apps/bert_ffn/torch/model.py:3-14: ln(ffn(x) + x) with
 * ffn = Linear(H, FF) -> activation -> Linear(FF, H).  The reference app uses
 * ReLU and LayerNorm eps 1e-5 (model.py:8,11; common/layer_norm_v2.cuh:62);
 * the BERT-large workload uses GELU(tanh) and eps 1e-12, so both are
 * parameters.  In the reference's pipelined kernel the residual enters as the
 * accumulator of the second GEMM (apps/bert_ffn/pipelined/bert_ffn_pl.cuh:
 * 90-99), which is the same sum.  `work` must hold M*FF + M*H floats.
 */
void oracle_bert_ffn(int64_t M, int64_t H, int64_t FF, const float* x, const float* w1, const float* b1,
                     const float* w2, const float* b2, const float* gamma, const float* beta, int act,
                     float eps, float* out, float* work) {
  float* h = work;
  float* y = work + M * FF;
  oracle_linear(M, H, FF, x, w1, b1, act, h);
  oracle_linear(M, FF, H, h, w2, b2, ORACLE_ACT_NONE, y);
  for (int64_t i = 0; i < M * H; ++i) y[i] += x[i];
  oracle_layer_norm(M, H, y, gamma, beta, eps, out);
}

/* c = a + b elementwise, common/elemwise_add.cuh:5-21 (fp32 here). */
void oracle_add(int64_t n, const float* a, const float* b, float* c) {
  for (int64_t i = 0; i < n; ++i) c[i] = a[i] + b[i];
}

/* c[m] = [a[m] || b[m]] row-wise, common/pipe_concat.cuh:6-39. */
void oracle_concat(int64_t M, int64_t N0, int64_t N1, const float* a, const float* b, float* c) {
  for (int64_t m = 0; m < M; ++m) {
    memcpy(c + m * (N0 + N1), a + m * N0, (size_t)N0 * sizeof(float));
    memcpy(c + m * (N0 + N1) + N0, b + m * N1, (size_t)N1 * sizeof(float));
  }
}

int oracle_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

void oracle_set_num_threads(int n) {
#ifdef _OPENMP
  if (n > 0) omp_set_num_threads(n);
#else
  (void)n;
#endif
}
