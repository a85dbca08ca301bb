/*
 * gpipes.hpp -- C++ wrappers over the C ABI of gpipes.h with the reference's
 * operator names and argument order.
 *
 * The reference's host entry points are functions such as
 *   void mgn_fullmlp_out(x, w1, b1, w2, b2, w3, b3, gamma, beta, out)
 * (apps/mgn_fullmlp/pipelined/mgn_fullmlp_pl_ext.cu:24-71) that report errors
 * by throwing (TORCH_CHECK).  These wrappers keep that shape for C++ callers
 * that hold raw device pointers: the row count comes first, the stream last
 * (default: the null stream), and a failing call throws gpipes::Error with
 * the library's message.  Header-only; link against libgpipes.so.
 */
#ifndef GPIPES_HPP
#define GPIPES_HPP

#include <cstdint>
#include <stdexcept>
#include <string>

#include "gpipes.h"

namespace gpipes {

class Error : public std::runtime_error {
 public:
  Error(int code, const std::string& what) : std::runtime_error(what), code_(code) {}
  int code() const { return code_; }

 private:
  int code_;
};

inline void check(int rc) {
  if (rc != GP_OK) throw Error(rc, "gpipes error " + std::to_string(rc) + ": " + gp_last_error());
}

// mgn_fullmlp_pl_ext.cu:24-71
inline void mgn_fullmlp_out(int64_t M, const void* x, const void* w1, const void* b1, const void* w2, const void* b2,
                            const void* w3, const void* b3, const void* gamma, const void* beta, void* out,
                            void* stream = nullptr) {
  check(gp_mgn_fullmlp_out(M, x, w1, b1, w2, b2, w3, b3, gamma, beta, out, stream));
}

// mgn_linears_pl_ext.cu:24-66
inline void mgn_linears_out(int64_t M, const void* x, const void* w1, const void* b1, const void* w2, const void* b2,
                            const void* w3, const void* b3, void* out, void* stream = nullptr) {
  check(gp_mgn_linears_out(M, x, w1, b1, w2, b2, w3, b3, out, stream));
}

// common/mlps.py:3-20, MgnMlp(K, [128, 128, 128], layernorm = gamma != nullptr)
inline void mgn_mlp_out(int64_t M, int64_t K, const void* x, const void* w1, const void* b1, const void* w2,
                        const void* b2, const void* w3, const void* b3, const void* gamma, const void* beta, void* out,
                        float eps = 1e-5f, int impl = GP_IMPL_FUSED, void* stream = nullptr) {
  check(gp_mgn_mlp_out(M, K, x, w1, b1, w2, b2, w3, b3, gamma, beta, eps, out, impl, stream));
}

// gp_mgn_mlp_dtype_out: the same MLP with every tensor in `dtype`
// (GP_DTYPE_F16 or GP_DTYPE_BF16; bf16 on the fused kernel only).
inline void mgn_mlp_dtype_out(int64_t M, int64_t K, const void* x, const void* w1, const void* b1, const void* w2,
                              const void* b2, const void* w3, const void* b3, const void* gamma, const void* beta,
                              void* out, int dtype, float eps = 1e-5f, int impl = GP_IMPL_FUSED,
                              void* stream = nullptr) {
  check(gp_mgn_mlp_dtype_out(M, K, x, w1, b1, w2, b2, w3, b3, gamma, beta, eps, out, impl, dtype, stream));
}

// common/pipe_gemm_bias_relu.cuh:85-192, pipe_gemm_bias.cuh:85-191, pipe_gemm.cuh:78-183
inline void linear_out(int64_t M, int64_t K, const void* x, const void* w, const void* b, const void* acc, int act,
                       void* out, void* stream = nullptr) {
  check(gp_linear_out(M, K, x, w, b, acc, act, out, stream));
}

// common/pipe_gemm_bias_layer_norm.cuh:100-249
inline void linear_layer_norm_out(int64_t M, int64_t K, const void* x, const void* w, const void* b, const void* gamma,
                                  const void* beta, float eps, void* out, void* stream = nullptr) {
  check(gp_linear_layer_norm_out(M, K, x, w, b, gamma, beta, eps, out, stream));
}

// common/layer_norm_v2.cuh:129-147 (host_layer_norm)
inline void layer_norm_out(int64_t M, int64_t D, const void* x, const void* gamma, const void* beta, float eps,
                           void* out, void* stream = nullptr) {
  check(gp_layer_norm_out(M, D, x, gamma, beta, eps, out, stream));
}

// common/elemwise_add.cuh:42-54 (host_add2)
inline void add_out(int64_t M, int64_t N, const void* a, const void* b, void* c, void* stream = nullptr) {
  check(gp_add_out(M, N, a, b, c, stream));
}

// common/concat.cuh:50-69 (host_concat2)
inline void concat_out(int64_t M, int64_t N0, int64_t N1, const void* a, const void* b, void* c,
                       void* stream = nullptr) {
  check(gp_concat_out(M, N0, N1, a, b, c, stream));
}

// Waits for `stream` and throws if its last launch that reports device-side
// failures (gp_pipeline_check) timed out.
inline void pipeline_check(void* stream = nullptr) { check(gp_pipeline_check(stream)); }

// bert_ffn_pl_ext.cu:24-56 (H 128, FF 512, ReLU, eps 1e-5 there, the defaults here)
inline void bert_ffn_out(int64_t M, int64_t H, int64_t FF, const void* x, const void* w1, const void* b1,
                         const void* w2, const void* b2, const void* ga, const void* be, void* out,
                         float eps = 1e-5f, int act = GP_ACT_RELU, void* stream = nullptr) {
  check(gp_bert_ffn_out(M, H, FF, x, w1, b1, w2, b2, ga, be, eps, act, out, stream));
}

// the same with a choice of layout: GP_IMPL_PIPELINED is the app's
// queue-chained layout (bert_ffn_pl.cuh:79-162; H 128, FF 512)
inline void bert_ffn_out(int64_t M, int64_t H, int64_t FF, const void* x, const void* w1, const void* b1,
                         const void* w2, const void* b2, const void* ga, const void* be, void* out, float eps,
                         int act, int impl, void* stream) {
  check(gp_bert_ffn_impl_out(M, H, FF, x, w1, b1, w2, b2, ga, be, eps, act, out, impl, stream));
}

// the wide GEMM stage (bert_ffn_pl.cuh:79-99, bulksync_gemm)
inline void gemm_out(int64_t M, int64_t N, int64_t K, const void* x, const void* w, const void* b, const void* r,
                     int act, void* out, void* stream = nullptr) {
  check(gp_gemm_out(M, N, K, x, w, b, r, act, out, stream));
}

// DlrmMlp chain (common/mlps.py:23-34): widths[0..nlayers], w/b/acts per layer.
inline void mlp_out(int64_t M, int nlayers, const int64_t* widths, const void* const* w, const void* const* b,
                    const int* acts, const void* x, void* out, void* stream = nullptr) {
  check(gp_mlp_out(M, nlayers, widths, w, b, acts, x, out, stream));
}

// dlrm_botmlp_out / dlrm_topmlp_out (apps/dlrm_botmlp/pipelined/dlrm_botmlp_pl_ext.cu:24-66,
// apps/dlrm_topmlp/pipelined/dlrm_topmlp_pl_ext.cu:24-71).
inline void dlrm_botmlp_out(int64_t M, int64_t K0, const void* x, const void* w1, const void* b1, const void* w2,
                            const void* b2, const void* w3, const void* b3, void* out, void* stream = nullptr) {
  check(gp_dlrm_botmlp_out(M, K0, x, w1, b1, w2, b2, w3, b3, out, stream));
}
inline void dlrm_topmlp_out(int64_t M, int64_t K0, int64_t N5, const void* x, const void* w1, const void* b1,
                            const void* w2, const void* b2, const void* w3, const void* b3, const void* w4,
                            const void* b4, const void* w5, const void* b5, void* out, int act5 = GP_ACT_RELU,
                            void* stream = nullptr) {
  check(gp_dlrm_topmlp_out(M, K0, N5, x, w1, b1, w2, b2, w3, b3, w4, b4, w5, b5, act5, out, stream));
}

// nerf_full_out (apps/nerf_full/pipelined/nerf_full_pl_ext.cu:24-97); w[0..11], b[0..11] = w1..w12, b1..b12.
inline void nerf_full_out(int64_t M, int64_t Kx, int64_t Kd, int64_t Na, int64_t Nrgb, const void* x, const void* d,
                          const void* const* w, const void* const* b, void* out_r, void* out_rgb,
                          int rgb_act = GP_ACT_NONE, void* stream = nullptr) {
  check(gp_nerf_full_out(M, Kx, Kd, Na, Nrgb, x, d, w, b, rgb_act, out_r, out_rgb, stream));
}

// bert_addln_ffn_out (apps/bert_addln_ffn/pipelined/bert_addln_ffn_pl_ext.cu:17-58; H 128, FF 512,
// ReLU, eps 1e-5 there, the defaults here).
inline void bert_addln_ffn_out(int64_t M, int64_t H, int64_t FF, const void* attn_out, const void* x, const void* w0,
                               const void* b0, const void* w1, const void* b1, const void* w2, const void* b2,
                               const void* ga0, const void* be0, const void* ga2, const void* be2, void* out,
                               float eps = 1e-5f, int act = GP_ACT_RELU, int impl = GP_IMPL_FUSED,
                               void* stream = nullptr) {
  check(gp_bert_addln_ffn_out(M, H, FF, attn_out, x, w0, b0, w1, b1, w2, b2, ga0, be0, ga2, be2, eps, act, out, impl,
                              stream));
}

// nerf_a_out (apps/nerf_a/pipelined/nerf_a_pl_ext.cu:24-76); w[0..7], b[0..7] = w1..w8, b1..b8.
inline void nerf_a_out(int64_t M, int64_t Kx, const void* x, const void* const* w, const void* const* b, void* out,
                       int impl = GP_IMPL_FUSED, void* stream = nullptr) {
  check(gp_nerf_a_out(M, Kx, x, w, b, out, impl, stream));
}

}  // namespace gpipes

#endif  // GPIPES_HPP
