// Host-side launch interface between the C ABI (capi.cpp) and the kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>

#include "../../include/gpipes.h"

namespace gp {

// One MGN-shaped MLP call: x[M,K] -> Linear(K,128)+ReLU -> Linear(128,128)+ReLU
// -> Linear(128,128) [-> LayerNorm(128) when gamma != nullptr] -> out[M,128].
// All tensors fp16, row-major, weights stored [K, N] (nn.Linear.weight.t()).
struct MgnArgs {
  int64_t M;
  int64_t K;
  const void* x;
  const void* w1;
  const void* b1;
  const void* w2;
  const void* b2;
  const void* w3;
  const void* b3;
  const void* gamma;  // nullptr: no LayerNorm (mgn_linears)
  const void* beta;
  float eps;
  void* out;
  // Gather front end (nf != nullptr): x is the edge features [M][128] and
  // row e of the MLP input is [nf[src[e]] | x[e] | nf[dst[e]]].
  const void* nf = nullptr;
  int64_t N = 0;
  const void* src = nullptr;
  const void* dst = nullptr;
  int idx_bytes = 0;  // 4 (int32) or 8 (int64)
  // Launch status word and epoch (status_acquire) and the poll bound of the
  // kernel's waits (0: the default).
  unsigned long long* status = nullptr;
  uint32_t epoch = 0;
  int spin_limit = 0;
  int dtype = GP_DTYPE_F16;  // element type of x, the weights and out (GP_DTYPE_BF16: fused kernel only)
};

// Persistent fused kernel (all layers in one workgroup per CU).
hipError_t mgn_fused_launch(const MgnArgs& a, int num_cus, hipStream_t stream);
// Copies the fused MGN kernels' phase timers of the last launch (diagnostic
// build only): 0, -1 (dst NULL or too small), -2 (copy failed), -3 (built
// without GP_PHASE_TIMERS).
int mgn_phase_timers_read(void* dst, int64_t bytes);

// The add + LayerNorm + FFN block of apps/bert_addln_ffn (attn, x [M,H] ->
// out [M,H]): h0 = LN0(attn w0 + b0 + x), out = LN2(act(h0 w1 + b1) w2 + b2 + h0).
// w0 [H,H], w1 [H,FF], w2 [FF,H] (weight.t()); biases and affines may be null.
struct BertAddlnArgs {
  int64_t M, H, FF;
  const void* attn;
  const void* x;
  const void *w0, *b0, *w1, *b1, *w2, *b2;
  const void *ga0, *be0, *ga2, *be2;
  float eps;
  int act;  // GP_ACT_*
  void* out;
};

// The BERT FFN block of apps/bert_ffn (x [M,H] -> out [M,H]):
// out = LayerNorm(act(x w1 + b1) w2 + b2 + x) * gamma + beta, w1 [H,FF], w2
// [FF,H] (weight.t()); biases and affines may be null (gamma null: 1).
struct BertFfnArgs {
  int64_t M, H, FF;
  const void* x;
  const void *w1, *b1, *w2, *b2;
  const void *gamma, *beta;
  float eps;
  int act;  // GP_ACT_*
  void* out;
};

// NerfA of apps/nerf_a (x [M,Kx] -> out [M,256]): five Linear + ReLU layers,
// the skip concatenation [h | x], three more Linear + ReLU layers.  w[0] is
// [Kx,256], w[5] [256+Kx,256], the rest [256,256]; biases may be null.
struct NerfAArgs {
  int64_t M, Kx;
  const void* x;
  const void* w[8];
  const void* b[8];
  void* out;
};

// One GEMM stage over M rows: out = act(x W + b [+ acc]) or LayerNorm(x W + b).
struct LinearArgs {
  int64_t M;
  int64_t K;          // 128, 256 or 384 (N is 128)
  const void* x;      // [M, K]
  const void* w;      // [K, 128]
  const void* b;      // [128] or nullptr
  const void* acc;    // [M, 128] accumulator input or nullptr
  const void* gamma;  // LayerNorm epilogue when non-null
  const void* beta;
  float eps;
  int act;            // GP_ACT_* (ignored with LayerNorm)
  void* out;          // [M, 128]
};
hipError_t linear_launch(const LinearArgs& a, int num_cus, hipStream_t stream);
hipError_t layer_norm_launch(int64_t M, int64_t D, const void* x, const void* gamma, const void* beta, float eps,
                             void* out, int num_cus, hipStream_t stream);
hipError_t add_launch(int64_t M, int64_t N, const void* a, const void* b, void* c, int num_cus, hipStream_t stream);

// Wide GEMM stage: out = act(x W + b) or x W + b + r, N a multiple of 128,
// K a multiple of 64, with W passed transposed (wt = W^T, [N, K]).  Row
// strides (elements, multiples of 8) default to K / N / N when 0; out may be a
// column block of a wider matrix.
struct GemmArgs {
  int64_t M;
  int64_t N;
  int64_t K;
  const void* x;   // [M, lda]
  const void* wt;  // [N, K]
  const void* b;   // [N] or nullptr
  const void* r;   // [M, ldr] residual or nullptr (then act must be ACT_NONE)
  int act;
  void* out;       // [M, ldc]
  int64_t lda = 0, ldc = 0, ldr = 0;
  int64_t ka = 0;  // columns of x read (a multiple of 8; 0 = K); columns [ka, K) count as zero
  // Instead of wt: W in its own layout, w [kw, ldw] (k by feature, 16-byte
  // aligned, ldw a multiple of 8, ldw >= N; kw defaults to K and ldw to N);
  // rows [kw, K) count as zero.  No transposed copy is needed.
  const void* w = nullptr;
  int64_t ldw = 0, kw = 0;
  // LayerNorm epilogue (ln != 0, act must be ACT_NONE): out = LayerNorm(x W +
  // b + r) over each row's N features, gamma / beta (null: 1 / 0), eps.  For
  // N > 128 a row spans several waves and workgroups, which exchange partial
  // statistics through ln_ws (gemm_ln_ws_bytes(M, N) bytes of a queue arena,
  // zeroed when allocated; the status word is its first 8 bytes) under an
  // epoch; every workgroup must then be resident at once: at most
  // gemm_ln_max_rows(N, num_cus) rows (four passes of num_cus tiles when
  // num_cus is a multiple of N / 256, else one) and at most 1024 row blocks.  Launches of one epoch on
  // one ln_ws are numbered by ln_round (0, 1, ...) and must cover a prefix of
  // the same row blocks in every earlier round.
  int ln = 0;
  int64_t ln_round = 0;
  int dtype = GP_DTYPE_F16;  // element type of x, the weights, b, r, gamma, beta and out
  const void* gamma = nullptr;
  const void* beta = nullptr;
  float eps = 0.f;
  void* ln_ws = nullptr;
  unsigned long long* status = nullptr;
  uint32_t epoch = 0;
  int spin_limit = 0;
};
hipError_t gemm_launch(const GemmArgs& a, int num_cus, hipStream_t stream);
// Rows one LayerNorm-epilogue launch may cover (all tiles resident), and the
// size of its exchange area.
int64_t gemm_ln_max_rows(int64_t N, int num_cus);
size_t gemm_ln_ws_bytes(int64_t M, int64_t N);
// Whether a layer chain reads its weights in place instead of from
// transposed copies.  In place, each weight fragment of the GEMM's k-loop
// takes two transposing LDS reads instead of one 16-byte read, which slows
// the loop by about 15% (BERT-large FFN 1.21 -> 1.38 ms); the copies cost one
// transpose launch per call (5-9 us).  Below kInPlaceMaxFlop of GEMM work
// (about 80 us) in place comes out ahead: the bert_addln_ffn chain at its
// app's batch 0.1165 -> 0.1148 ms, nerf_a 0.1788 -> 0.1737 ms.
constexpr double kInPlaceMaxFlop = 8e10;
inline bool weights_in_place(double flop) { return flop < kInPlaceMaxFlop; }

// GEMM arguments for W [K, N] read in place (row stride N).
inline GemmArgs gemm_w(int64_t M, int64_t N, int64_t K, const void* x, const void* w, const void* b, const void* r,
                       int act, void* out) {
  GemmArgs g{M, N, K, x, nullptr, b, r, act, out};
  g.w = w;
  return g;
}
// out[Np, Kp] = in[K, N]^T, zero-padded (Kp, Np default to K, N); Kp and Np
// multiples of 64.
hipError_t transpose_launch(const void* in, void* out, int64_t K, int64_t N, hipStream_t stream, int64_t Kp = 0,
                            int64_t Np = 0);
// out[m] = act(a[m, 0:K] . w[0:K] + b[0]) for m < M (a one-output layer); K
// and lda multiples of 8, a and w 16-byte aligned, b may be null.
hipError_t gemv1_launch(int64_t M, int64_t K, const void* a, int64_t lda, const void* w, const void* b, int act,
                        void* out, int num_cus, hipStream_t stream, int dtype = GP_DTYPE_F16);
// One launch for the weights of a layer chain: wt[Np, Kp] = w[K, N]^T and
// bp[Np] = b (zeros for a null b), both zero-padded; Kp and Np multiples of 64.
// A null bp skips the bias.
struct PrepSpec {
  const void* w;
  void* wt;
  const void* b;
  void* bp;
  int64_t K, N, Kp, Np;
};
hipError_t prep_launch(const PrepSpec* layers, int n, hipStream_t stream);
hipError_t concat_launch(int64_t M, int64_t N0, int64_t N1, const void* a, const void* b, void* c, int num_cus,
                         hipStream_t stream);
// dst[m][j] = act(src[m][j]) for j < w and 0 for w <= j < wpad (strides in elements).
hipError_t place_launch(int64_t M, const void* src, int64_t lds, int64_t w, void* dst, int64_t ldd, int64_t wpad,
                        int act, int num_cus, hipStream_t stream);

// The NeRF MLP (apps/nerf_full/torch/model.py:5-66, hidden 256) as one fused
// kernel: supported for Kx, Kd, Na, Nrgb <= 64; x and d 16-byte aligned.
// w[i], b[i]: layer i+1's [K, N] weight and [N] bias (b may be null).  The
// workspace (nerf_fused_workspace() bytes, 16-byte aligned) receives the
// packed weight stream.  dtype: GP_DTYPE_F16 or GP_DTYPE_BF16, the element
// type of every tensor.
bool nerf_fused_supported(int64_t Kx, int64_t Kd, int64_t Na, int64_t Nrgb);
size_t nerf_fused_workspace();
hipError_t nerf_fused_launch(int64_t M, int Kx, int Kd, int Na, int Nrgb, const void* x, const void* d,
                             const void* const* w, const void* const* b, int rgb_act, void* out_r, void* out_rgb,
                             void* ws, int num_cus, hipStream_t stream, int dtype = GP_DTYPE_F16);
// NerfA (apps/nerf_a/torch/model.py:5-38): the same kernel stopped after
// layer 8, out [M, 256] = the trunk's ReLU output; Kx <= 64, x 16-byte
// aligned, w[0..7] / b[0..7], workspace as above.
inline bool nerf_trunk_supported(int64_t Kx) { return Kx >= 1 && Kx <= 64; }
hipError_t nerf_trunk_launch(int64_t M, int Kx, const void* x, const void* const* w, const void* const* b, void* out,
                             void* ws, int num_cus, hipStream_t stream, int dtype = GP_DTYPE_F16);
// The NeRF kernel's static scratch on device `dev` (the current device), for
// the allocation-free entry point: its device address and size, the event
// that chains the calls on that device (each eager call's stream waits for it
// and records it after its own kernels) and the lock that keeps the wait,
// the launches and the record of one call together.
struct NerfScratch {
  void* ptr;
  size_t bytes;
  hipEvent_t last;
  std::mutex* lock;
};
int nerf_static_scratch(int dev, NerfScratch* out);

// The DLRM bottom MLP (K0 -> 512 -> 256 -> 128, apps/dlrm_botmlp) as one fused
// kernel: supported for K0 <= 32, identity or ReLU after the first two layers
// and any activation after the third (acts[0..2]); x and out 16-byte aligned.
// w[i], b[i]: layer i+1's [K, N] weight and [N] bias (b may be null).  The
// workspace (dlrm_bot_workspace() bytes, 16-byte aligned) receives the packed
// weights.  dtype: GP_DTYPE_F16 or GP_DTYPE_BF16, the element type of every
// tensor.
inline bool dlrm_bot_supported(int64_t K0, const int* acts) {
  auto hidden = [](int a) { return a == GP_ACT_NONE || a == GP_ACT_RELU; };
  return K0 >= 1 && K0 <= 32 && hidden(acts[0]) && hidden(acts[1]) && acts[2] >= GP_ACT_NONE &&
         acts[2] <= GP_ACT_SIGMOID;
}
size_t dlrm_bot_workspace();
// The last two layers of the DLRM top MLP (K -> 256 -> 1, the click head,
// apps/dlrm_topmlp) as one fused kernel: K 256, 512 or 1024 with x [M][K]
// 16-byte aligned, identity or ReLU after the K -> 256 layer, any activation
// after the click head; out [M] (2-byte aligned).  w4 [K][256], b4 [256], w5
// [256] (the [256, 1] weight), b5 [1] (biases may be null).  The workspace
// (dlrm_tail_workspace(K) bytes, 16-byte aligned) receives the packed weights
// when `pack` is set (calls over row chunks of one set of weights pack once).
inline bool dlrm_tail_supported(int64_t K, int act4, int act5) {
  return (K == 256 || K == 512 || K == 1024) && (act4 == GP_ACT_NONE || act4 == GP_ACT_RELU) &&
         act5 >= GP_ACT_NONE && act5 <= GP_ACT_SIGMOID;
}
size_t dlrm_tail_workspace(int64_t K);
hipError_t dlrm_tail_launch(int64_t M, int64_t K, const void* x, const void* w4, const void* b4, int act4,
                            const void* w5, const void* b5, int act5, void* out, void* ws, int num_cus,
                            hipStream_t stream, int dtype = GP_DTYPE_F16, bool pack = true);
hipError_t dlrm_bot_launch(int64_t M, int K0, const void* x, const void* const* w, const void* const* b,
                           const int* acts, void* out, void* ws, int num_cus, hipStream_t stream,
                           int dtype = GP_DTYPE_F16);

}  // namespace gp
