/* CPU oracle for the gpu-pipes fused-MLP path -- TEST INFRASTRUCTURE ONLY. */
#ifndef GP_ORACLE_H
#define GP_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORACLE_ACT_NONE 0
#define ORACLE_ACT_RELU 1
#define ORACLE_ACT_GELU_TANH 2
#define ORACLE_ACT_SIGMOID 3

float oracle_h2f(uint16_t h);
uint16_t oracle_f2h(float f);
void oracle_h2f_array(int64_t n, const uint16_t* src, float* dst);
void oracle_f2h_array(int64_t n, const float* src, uint16_t* dst);

void oracle_linear(int64_t M, int64_t K, int64_t N, const float* x, const float* w, const float* b,
                   int act, float* y);
void oracle_layer_norm(int64_t M, int64_t D, const float* x, const float* gamma, const float* beta,
                       float eps, float* y);
void oracle_mgn_mlp(int64_t M, int64_t K, const float* x, const float* w1, const float* b1,
                    const float* w2, const float* b2, const float* w3, const float* b3,
                    const float* gamma, const float* beta, float eps, float* out, float* work);
void oracle_bert_ffn(int64_t M, int64_t H, int64_t FF, const float* x, const float* w1, const float* b1,
                     const float* w2, const float* b2, const float* gamma, const float* beta, int act,
                     float eps, float* out, float* work);
void oracle_add(int64_t n, const float* a, const float* b, float* c);
void oracle_concat(int64_t M, int64_t N0, int64_t N1, const float* a, const float* b, float* c);

/* Synthetic inputs (synth.c): the host restatement of gp_fill_normal. */
void oracle_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]);
float oracle_log_unit(float u);
float oracle_sqrt_small(float v);
void oracle_sincos_quarter(float a, float* s, float* c);
void oracle_normal_f32(int64_t n, uint64_t seed, uint64_t offset, float* dst);
void oracle_normal_16(int64_t n, uint64_t seed, uint64_t offset, int bf16, uint16_t* dst);

int oracle_num_threads(void);
void oracle_set_num_threads(int n);

#ifdef __cplusplus
}
#endif

#endif
