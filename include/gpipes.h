/*
 * gpipes.h -- C ABI of the MI355X (gfx950) gpu-pipes fused-MLP library.
 *
 * Every entry point takes plain device pointers and sizes, launches on the
 * HIP stream it is given (NULL = the default stream), never aborts, never
 * synchronises, and returns GP_OK or a negative GP_ERR_* code.  The message
 * of the last failure on the calling thread is available from gp_last_error().
 *
 * Layouts are the reference's (apps/mgn_fullmlp/pipelined/val.py:15-21):
 *   x     [M, K]  fp16, row-major, contiguous
 *   w_i   [K, N]  fp16, row-major (= torch nn.Linear.weight.t().contiguous())
 *   b_i   [N]     fp16
 *   gamma, beta [N] fp16 (LayerNorm affine)
 *   out   [M, N]  fp16, row-major
 * x, out and every w_i must be 16-byte aligned.
 */
#ifndef GPIPES_H
#define GPIPES_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GP_OK 0
#define GP_ERR_INVALID_ARG (-1) /* null pointer, negative size, bad flag       */
#define GP_ERR_SHAPE (-2)       /* a dimension the kernels do not support      */
#define GP_ERR_ALIGN (-3)       /* pointer not 16-byte aligned                 */
#define GP_ERR_HIP (-4)         /* HIP runtime / launch failure                */
#define GP_ERR_TIMEOUT (-5)     /* a launch failed on the device: a wait       */
                                /* exceeded its poll bound (its outputs are not */
                                /* valid), or no pipeline fitted on one XCD;    */
                                /* reported by gp_pipeline_check                */
#define GP_ERR_NO_DEVICE (-6)   /* no usable gfx950 device                     */

/* Implementation selector for gp_mgn_mlp_out. */
#define GP_IMPL_FUSED 0              /* persistent fused kernel (default, fastest)        */
#define GP_IMPL_PIPELINED 1          /* stage workgroups linked by L2 ring queues;         */
                                     /* layer 3 and LayerNorm fused in one stage            */
#define GP_IMPL_PIPELINED_SPLIT_LN 2 /* the reference's layout: layer 3 feeds five         */
                                     /* LayerNorm workers through a round-robin split queue */

/* Element types of the *_dtype_out entry points (16-bit storage, fp32 accumulation). */
#define GP_DTYPE_F16 0  /* IEEE binary16 */
#define GP_DTYPE_BF16 1 /* bfloat16      */

/* Activations of gp_linear_out. */
#define GP_ACT_NONE 0
#define GP_ACT_RELU 1
#define GP_ACT_GELU_TANH 2
#define GP_ACT_SIGMOID 3

/* Library version as 0xMMmmpp. */
int gp_version(void);

/* Message describing the most recent failure on this thread ("" if none). */
const char* gp_last_error(void);

/*
 * MeshGraphNet edge MLP with LayerNorm: x[M,384] -> 384->128 ReLU -> 128->128
 * ReLU -> 128->128 -> LayerNorm(128, eps=1e-5) -> out[M,128].
 * Replaces mgn_fullmlp_out(x, w1, b1, w2, b2, w3, b3, gamma, beta, out),
 * apps/mgn_fullmlp/pipelined/mgn_fullmlp_pl_ext.cu:24-71 (eps as hard-coded
 * in common/layer_norm_v2.cuh:62).  Any M >= 0 is accepted (the reference
 * requires M % 20 == 0 and drops tail rows).
 */
int gp_mgn_fullmlp_out(int64_t M, const void* x, const void* w1, const void* b1, const void* w2,
                       const void* b2, const void* w3, const void* b3, const void* gamma,
                       const void* beta, void* out, void* stream);

/*
 * The same chain without LayerNorm: x[M,384] -> out[M,128].
 * Replaces mgn_linears_out(x, w1, b1, w2, b2, w3, b3, out),
 * apps/mgn_linears/pipelined/mgn_linears_pl_ext.cu:24-66.
 */
int gp_mgn_linears_out(int64_t M, const void* x, const void* w1, const void* b1, const void* w2,
                       const void* b2, const void* w3, const void* b3, void* out, void* stream);

/*
 * Generic MGN-shaped MLP (common/mlps.py:3-20, MgnMlp(K, [128,128,128],
 * layernorm=gamma!=NULL)): K in {128, 256, 384}; gamma == NULL (and beta ==
 * NULL) skips the LayerNorm.  `impl` is one of GP_IMPL_*.  The pipelined
 * implementations report a queue-wait timeout through gp_pipeline_check().
 * The node MLP of MeshGraphNet is K = 256.  Both entry points above are this
 * call with K = 384.
 */
int gp_mgn_mlp_out(int64_t M, int64_t K, const void* x, const void* w1, const void* b1,
                   const void* w2, const void* b2, const void* w3, const void* b3,
                   const void* gamma, const void* beta, float eps, void* out, int impl,
                   void* stream);

/*
 * gp_mgn_mlp_out with the element type of x, every weight / bias / gamma /
 * beta and out given by `dtype`: GP_DTYPE_F16 (the same call as
 * gp_mgn_mlp_out) or GP_DTYPE_BF16, which runs bf16 MFMAs with fp32
 * accumulation and rounds the two hidden activations and the output to bf16
 * (round to nearest even).  bf16 runs on the fused kernel only (impl
 * GP_IMPL_FUSED; other impls return GP_ERR_INVALID_ARG).  No counterpart in
 * the reference, whose extensions take fp16 tensors only; it is the bf16
 * form of the same MgnMlp (common/mlps.py:3-20) for callers that keep their
 * activations in bf16.
 */
int gp_mgn_mlp_dtype_out(int64_t M, int64_t K, const void* x, const void* w1, const void* b1,
                         const void* w2, const void* b2, const void* w3, const void* b3,
                         const void* gamma, const void* beta, float eps, void* out, int impl,
                         int dtype, void* stream);

/*
 * MeshGraphNet edge update with the gather front end fused in:
 *   out[e] = MLP([nf[src[e]] | ef[e] | nf[dst[e]]]),  e < E,
 * the edge MLP of gp_mgn_fullmlp_out (K = 384; gamma == NULL skips the
 * LayerNorm) whose input rows are gathered from the node table nf[N,128] and
 * the edge features ef[E,128] while they are copied into the kernel, so the
 * concatenated [E,384] input never exists in memory.  src / dst are int32
 * (idx_bytes = 4) or int64 (idx_bytes = 8); an index outside [0, N) gathers
 * zeros.  N <= 8388607.  Replaces the index / index / concat / mlp sequence
 * of update_edges, graphmodel/mgn_dp.py:28-32.
 */
int gp_mgn_edge_gather_out(int64_t E, int64_t N, const void* nf, const void* ef, const void* src, const void* dst,
                           int idx_bytes, const void* w1, const void* b1, const void* w2, const void* b2,
                           const void* w3, const void* b3, const void* gamma, const void* beta, float eps, void* out,
                           void* stream);

/*
 * BERT feed-forward block with residual add and LayerNorm:
 *   out[M,H] = LayerNorm(act(x . w1 + b1) . w2 + b2 + x) * gamma + beta
 * with w1 [H,FF], b1 [FF], w2 [FF,H], b2 [H], gamma / beta [H] (NULL: 1 / 0),
 * act GP_ACT_RELU (the reference app) or GP_ACT_GELU_TANH (BERT-large), eps
 * as given.  H in {128, 256, 512, 1024}; FF a multiple of 128, at most 16384.
 * Replaces bert_ffn_out(x, w1, b1, w2, b2, ga, be, out),
 * apps/bert_ffn/pipelined/bert_ffn_pl_ext.cu:24-56 (H = 128, FF = 512, ReLU,
 * eps 1e-5 fixed), and the bulk-sync chain gemm / gemm / add / LayerNorm of
 * apps/bert_ffn/bulksync/bert_ffn_bs.cuh:12-27.  Per row chunk, two GEMM
 * launches; the second computes the residual add and the LayerNorm in its
 * epilogue.  Above H = 128 a row spans several workgroups, which exchange
 * partial row statistics through the stream's queue arena with bounded waits:
 * such calls report failures through gp_pipeline_check.  Every workgroup of
 * that launch (one per CU) must be resident at once, as for the queue-chained
 * layouts: kernels of other streams or processes holding CUs meanwhile can
 * make its waits run out (GP_ERR_TIMEOUT; never a hang).  The FF-wide
 * activations pass through a workspace kept per (device, stream), allocated
 * on first use and grown when needed (a grow synchronises the stream).  Any
 * M >= 0 (the reference needs M to be a multiple of its pipeline rows x 128).
 */
int gp_bert_ffn_out(int64_t M, int64_t H, int64_t FF, const void* x, const void* w1, const void* b1,
                    const void* w2, const void* b2, const void* gamma, const void* beta, float eps, int act,
                    void* out, void* stream);

/*
 * gp_bert_ffn_out with a choice of implementation.  impl GP_IMPL_FUSED (0):
 * the same call as gp_bert_ffn_out.  GP_IMPL_PIPELINED: the reference app's
 * queue-chained layout (apps/bert_ffn/pipelined/bert_ffn_pl.cuh:79-162, the
 * operator bert_ffn_out of bert_ffn_pl_ext.cu:24-56): stage workgroups linked
 * by ring queues -- four W1 column slices write the FF-wide activations into
 * one queue, two workers compute W2 + b2 + x and the LayerNorm -- for H = 128,
 * FF = 512, ReLU or GELU(tanh), any M; failures (a wait that runs out) are
 * reported by gp_pipeline_check, and the call is refused while the stream is
 * capturing a graph.  fp16 tensors.
 */
int gp_bert_ffn_impl_out(int64_t M, int64_t H, int64_t FF, const void* x, const void* w1, const void* b1,
                         const void* w2, const void* b2, const void* gamma, const void* beta, float eps, int act,
                         void* out, int impl, void* stream);

/*
 * gp_bert_ffn_out with the element type of x, the weights, biases, gamma,
 * beta and out given by `dtype`: GP_DTYPE_F16 (the same call) or
 * GP_DTYPE_BF16 (bf16 MFMAs, fp32 accumulation and epilogue arithmetic, the
 * activations between the GEMMs and the output rounded to bf16).  No
 * counterpart in the reference, whose extensions take fp16 tensors only; the
 * bf16 form of the same block for callers that keep their activations in bf16.
 */
int gp_bert_ffn_dtype_out(int64_t M, int64_t H, int64_t FF, const void* x, const void* w1, const void* b1,
                          const void* w2, const void* b2, const void* gamma, const void* beta, float eps, int act,
                          void* out, int dtype, void* stream);

/*
 * The add + LayerNorm + FFN block of the bert_addln_ffn app,
 * apps/bert_addln_ffn/torch/model.py:3-20:
 *   h0  = LayerNorm(attn . w0 + b0 + x) * ga0 + be0
 *   out = LayerNorm(act(h0 . w1 + b1) . w2 + b2 + h0) * ga2 + be2
 * attn, x [M,H]; w0 [H,H], w1 [H,FF], w2 [FF,H] (weight.t()); biases [N] and
 * the affines [H] may be NULL (0, or 1 / 0); act GP_ACT_RELU (the app) or
 * GP_ACT_GELU_TANH; eps as given (the app's is 1e-5).  H in {128, 256, 512,
 * 1024}, FF a multiple of 128, at most 16384; any M >= 0.
 * Replaces bert_addln_ffn_out(attn_out, x, w0, b0, w1, b1, w2, b2, ga0, be0,
 * ga2, be2, out), apps/bert_addln_ffn/pipelined/bert_addln_ffn_pl_ext.cu:17-58
 * (H 128, FF 512, ReLU, M a multiple of 128).  impl GP_IMPL_FUSED (0, the
 * default) runs one GEMM launch per linear layer with bias, activation,
 * residual and LayerNorm fused into its epilogue, over row chunks in the
 * per-stream workspace (above H = 128 with failures reported by
 * gp_pipeline_check, as gp_bert_ffn_out); GP_IMPL_PIPELINED runs the reference's
 * queue-chained layout (bert_addln_ffn_pl.cuh:92-176: stage workgroups linked
 * by ring queues, both adds fed from queues) for H = 128, FF = 512 and ReLU or
 * GELU(tanh), with failures reported by gp_pipeline_check.  The reference's
 * defects are not reproduced: its ln0 never runs and its extension passes be0
 * for be2 (bert_addln_ffn_pl.cuh:227, _ext.cu:71).
 */
int gp_bert_addln_ffn_out(int64_t M, int64_t H, int64_t FF, const void* attn, const void* x, const void* w0,
                          const void* b0, const void* w1, const void* b1, const void* w2, const void* b2,
                          const void* ga0, const void* be0, const void* ga2, const void* be2, float eps, int act,
                          void* out, int impl, void* stream);

/*
 * gp_bert_addln_ffn_out with every tensor's element type given by `dtype`
 * (GP_DTYPE_F16 or GP_DTYPE_BF16, as gp_bert_ffn_dtype_out); bf16 runs the
 * fused implementation only (GP_IMPL_PIPELINED with bf16 returns
 * GP_ERR_INVALID_ARG).  No counterpart in the reference (fp16 only).
 */
int gp_bert_addln_ffn_dtype_out(int64_t M, int64_t H, int64_t FF, const void* attn, const void* x,
                                const void* w0, const void* b0, const void* w1, const void* b1, const void* w2,
                                const void* b2, const void* ga0, const void* be0, const void* ga2, const void* be2,
                                float eps, int act, void* out, int impl, int dtype, void* stream);

/*
 * NerfA, apps/nerf_a/torch/model.py:5-38 (hidden 256, skip after the fifth
 * layer): with w[0..7] / b[0..7] the reference's w1..w8 / b1..b8
 * (apps/nerf_a/pipelined/nerf_a_pl_ext.cu:24-76),
 *   h = ReLU chain of w1 [Kx,256], w2..w5 [256,256];  h = [h | x];
 *   out [M,256] = ReLU chain of w6 [256+Kx,256], w7, w8 [256,256].
 * x [M,Kx], Kx in [1, 1024] (the app's is 64); biases may be NULL.  impl
 * GP_IMPL_FUSED (0, the default) runs, for Kx <= 64, the NeRF MLP's fused
 * kernel stopped after layer 8 (x rows not 16-byte aligned are first copied
 * into the workspace), and for wider inputs one wide-GEMM launch per layer
 * over row chunks; GP_IMPL_PIPELINED runs the reference's queue-chained layout
 * (nerf_a_pl.cuh:97-179: stage workgroups linked by ring queues, the skip
 * concatenation a pipe_concat stage fed from a queue) for Kx a multiple of 8
 * up to 128, with failures reported by gp_pipeline_check.
 */
int gp_nerf_a_out(int64_t M, int64_t Kx, const void* x, const void* const* w, const void* const* b, void* out,
                  int impl, void* stream);

/*
 * gp_nerf_a_out with the element type as an argument: no counterpart in the
 * reference (fp16 only).  GP_DTYPE_BF16 takes x, every weight and bias and
 * out as bf16 on the default implementation (both of its paths);
 * GP_IMPL_PIPELINED with bf16 returns GP_ERR_INVALID_ARG.
 */
int gp_nerf_a_dtype_out(int64_t M, int64_t Kx, const void* x, const void* const* w, const void* const* b, void* out,
                        int impl, int dtype, void* stream);

/*
 * Dense MLP chain: widths[0] -> widths[1] -> ... -> widths[nlayers], layer i
 * out = act_i(in . w[i] + b[i]) with w[i] [widths[i], widths[i+1]] (fp16,
 * weight.t()), b[i] [widths[i+1]] or NULL, acts[i] one of GP_ACT_*.  Any
 * widths in [1, 16384]; x [M, widths[0]], out [M, widths[nlayers]].  This is
 * DlrmMlp(widths, sigmoid_i) of common/mlps.py:23-34 (ReLU after every layer,
 * sigmoid after layer sigmoid_i) with the activation of each layer given.
 * Rows go through in chunks of 262,144 with the activations in the per-stream
 * workspace.
 */
int gp_mlp_out(int64_t M, int nlayers, const int64_t* widths, const void* const* w, const void* const* b,
               const int* acts, const void* x, void* out, void* stream);

/*
 * gp_mlp_out with every tensor's element type given by `dtype` (GP_DTYPE_F16:
 * the same call; GP_DTYPE_BF16: bf16 MFMAs, fp32 accumulation and
 * activations, each layer's output rounded to bf16).  No counterpart in the
 * reference (fp16 only); the bf16 form of the DLRM towers for callers that
 * keep their activations in bf16.
 */
int gp_mlp_dtype_out(int64_t M, int nlayers, const int64_t* widths, const void* const* w, const void* const* b,
                     const int* acts, const void* x, void* out, int dtype, void* stream);

/*
 * DLRM bottom MLP: x[M,K0] -> 512 -> 256 -> 128, ReLU after each layer.
 * Replaces dlrm_botmlp_out(x, w1, b1, w2, b2, w3, b3, out),
 * apps/dlrm_botmlp/pipelined/dlrm_botmlp_pl_ext.cu:24-66 (K0 = 32 there;
 * 13 dense features padded to 16 in the DLRM workload).
 */
int gp_dlrm_botmlp_out(int64_t M, int64_t K0, const void* x, const void* w1, const void* b1, const void* w2,
                       const void* b2, const void* w3, const void* b3, void* out, void* stream);

/*
 * DLRM top MLP: x[M,K0] -> 1024 -> 1024 -> 512 -> 256 (ReLU after each) -> N5
 * with act5 after the last layer.  Replaces dlrm_topmlp_out(x, w1, b1, ...,
 * w5, b5, out), apps/dlrm_topmlp/pipelined/dlrm_topmlp_pl_ext.cu:24-71 (K0 =
 * 512, N5 = 64, every layer ReLU per DlrmMlp, common/mlps.py:23-34; the
 * reference kernel drops the ReLU of layer 4, dlrm_topmlp_pl.cuh:157, which is
 * not reproduced).  The DLRM click head is N5 = 1 with act5 = GP_ACT_SIGMOID.
 */
int gp_dlrm_topmlp_out(int64_t M, int64_t K0, int64_t N5, const void* x, const void* w1, const void* b1,
                       const void* w2, const void* b2, const void* w3, const void* b3, const void* w4,
                       const void* b4, const void* w5, const void* b5, int act5, void* out, void* stream);

/*
 * NeRF MLP, apps/nerf_full/torch/model.py:5-66 (hidden 256, skip after the
 * fifth layer, view directions): with w[0..11] / b[0..11] the reference's
 * w1..w12 / b1..b12 (nerf_full_pl_ext.cu:24-97),
 *   h = ReLU chain of w1 [Kx,256], w2..w5 [256,256]; h = [h | x];
 *   h = ReLU chain of w6 [256+Kx,256], w7, w8 [256,256];
 *   out_r [M,Na]   = h . w9 [256,Na] + b9;
 *   f = h . w10 [256,256] + b10;  g = ReLU([f | d] . w11 [256+Kd,128] + b11);
 *   out_rgb [M,Nrgb] = rgb_act(g . w12 [128,Nrgb] + b12).
 * x [M,Kx], d [M,Kd]; Kx, Kd, Na, Nrgb in [1, 1024].  The reference app has
 * Kx 64, Kd 32, Na = Nrgb = 64 and no colour activation; the NeRF workload has
 * Kx 64 (63 + 1 zero), Kd 27, Na 1, Nrgb 3 and a sigmoid.
 * With Kx <= 64, Kd <= 32, Na <= 64 and Nrgb <= 64 (both of those shapes) the
 * call is one fused kernel over 256-row tiles (x or d rows not 16-byte
 * aligned are first copied into the workspace); other widths run as one wide
 * GEMM launch per layer over chunks of 262,144 rows.
 */
int gp_nerf_full_out(int64_t M, int64_t Kx, int64_t Kd, int64_t Na, int64_t Nrgb, const void* x, const void* d,
                     const void* const* w, const void* const* b, int rgb_act, void* out_r, void* out_rgb,
                     void* stream);

/*
 * gp_nerf_full_out with the element type as an argument: no counterpart in
 * the reference (its NeRF MLP is fp16 only).  dtype GP_DTYPE_F16 is
 * gp_nerf_full_out; GP_DTYPE_BF16 takes x, d, every weight and bias and both
 * outputs as bf16 (fp32 accumulation, activations rounded to bf16 between
 * layers), on the same two paths: the fused kernel for the shapes above, one
 * wide-GEMM launch per layer otherwise.
 */
int gp_nerf_full_dtype_out(int64_t M, int64_t Kx, int64_t Kd, int64_t Na, int64_t Nrgb, const void* x,
                           const void* d, const void* const* w, const void* const* b, int rgb_act, void* out_r,
                           void* out_rgb, int dtype, void* stream);

/*
 * gp_nerf_full_out without any allocation: no reference counterpart.  For
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  Same arguments and
 * results as gp_nerf_full_out (bit-identical: the same kernels), limited to
 * the fused kernel's shapes (Kx <= 64, Kd <= 32, Na <= 64, Nrgb <= 64) and to
 * 16-byte aligned x and d; other shapes are rejected with GP_ERR_SHAPE /
 * GP_ERR_ALIGN.  Its scratch (the packed weight stream, 1,255,168 bytes) is a
 * static device array that every GPU the library runs on holds until the
 * process ends, shared by every call on that GPU.  Eager calls are chained
 * through one event per GPU: each call's stream waits for the previous call's
 * kernels (on whatever stream) and records the event after its own, so calls
 * on different streams run in turn.  Calls under graph capture are not
 * chained: graph replays that overlap each other or an eager call race for
 * the scratch.  The first call on a GPU looks up the array's address and
 * creates the event; no call makes hipMalloc, hipFree or an allocating
 * library routine.
 */
int gp_nerf_full_out_noalloc(int64_t M, int64_t Kx, int64_t Kd, int64_t Na, int64_t Nrgb, const void* x,
                             const void* d, const void* const* w, const void* const* b, int rgb_act, void* out_r,
                             void* out_rgb, void* stream);

/* ------------------------------------------------------------------------
 * Stage-level entry points: one stage function of the library run over a
 * whole matrix (tiles of 128 rows, persistent workgroups).
 * ------------------------------------------------------------------------ */

/*
 * out[M,128] = act(x[M,K] . w[K,128] + b [+ acc[M,128]]), fp32 accumulation.
 * K in {128, 256, 384}; b and acc may be NULL; act is GP_ACT_*.
 * The stage of common/pipe_gemm_bias_relu.cuh:85-192 (act = RELU),
 * common/pipe_gemm_bias.cuh:85-191 (act = NONE) and common/pipe_gemm.cuh:78-183
 * (acc = the AccumReader tile, b = NULL); as a whole-matrix call it also
 * replaces bulksync_gemm<M,N,K,RELU>, common/bulksync_gemm.cuh:13-110.
 */
int gp_linear_out(int64_t M, int64_t K, const void* x, const void* w, const void* b, const void* acc, int act,
                  void* out, void* stream);

/*
 * out = LayerNorm(x . w + b) * gamma + beta over the 128 outputs: the stage
 * intended by common/pipe_gemm_bias_layer_norm.cuh:100-249.
 */
int gp_linear_layer_norm_out(int64_t M, int64_t K, const void* x, const void* w, const void* b,
                             const void* gamma, const void* beta, float eps, void* out, void* stream);

/*
 * The wide GEMM stage: out[M,N] = act(x[M,K] . w[K,N] + b), or, with r
 * non-NULL, x . w + b + r[M,N] (act must then be GP_ACT_NONE).  N a multiple
 * of 128, K a multiple of 64 (both at most 16384); b may be NULL.  The
 * PipeGemmBiasRelu / PipeGemmBias blocks composed along N and K with the
 * residual as accumulator (apps/bert_ffn/pipelined/bert_ffn_pl.cuh:79-99,
 * common/pipe_gemm.cuh:128-146), and bulksync_gemm<M,N,K,RELU>
 * (common/bulksync_gemm.cuh:13-110) beyond the 128-wide stage of
 * gp_linear_out.  w is transposed into the per-stream workspace on each call.
 */
int gp_gemm_out(int64_t M, int64_t N, int64_t K, const void* x, const void* w, const void* b, const void* r,
                int act, void* out, void* stream);

/*
 * gp_gemm_out with the element type of x, w, b, r and out given by `dtype`
 * (GP_DTYPE_F16: the same call; GP_DTYPE_BF16: bf16 MFMAs, fp32 accumulation,
 * bias / activation / residual in fp32, output rounded to bf16).  No
 * counterpart in the reference (fp16 only).
 */
int gp_gemm_dtype_out(int64_t M, int64_t N, int64_t K, const void* x, const void* w, const void* b, const void* r,
                      int act, void* out, int dtype, void* stream);

/*
 * out[M,D] = LayerNorm(x[M,D]) * gamma + beta, biased variance, eps as given;
 * D in {128, 256, 512, 1024}; gamma / beta NULL mean 1 / 0.
 * Replaces host_layer_norm<D>(M, x, gamma, beta, out),
 * common/layer_norm_v2.cuh:129-147 (the pipe_layer_norm stage,
 * common/pipe_layer_norm.cuh:13-60).
 */
int gp_layer_norm_out(int64_t M, int64_t D, const void* x, const void* gamma, const void* beta, float eps,
                      void* out, void* stream);

/*
 * c[M,N] = a + b elementwise; N a multiple of 8.  Replaces host_add2,
 * common/elemwise_add.cuh:42-54 (the pipe_add stage, common/pipe_add.cuh:13-40).
 */
int gp_add_out(int64_t M, int64_t N, const void* a, const void* b, void* c, void* stream);

/*
 * c[M,N0+N1] = [a[M,N0] | b[M,N1]] row-wise; N0, N1 multiples of 8.
 * Replaces host_concat2, common/concat.cuh:50-69 (the pipe_concat stage,
 * common/pipe_concat.cuh:48-74).
 */
int gp_concat_out(int64_t M, int64_t N0, int64_t N1, const void* a, const void* b, void* c, void* stream);

/*
 * Identity pipelines: sender workgroups copy 128-row tiles of x[M,128] into
 * ring queues, receiver workgroups copy them out to out[M,128].  At most
 * max_pipes pipelines (<= 0: as many as fit).  The queue round trip of
 * misc_tests/pipeval/pipe_val_ext.cu:65-149 (ident).  Same as
 * gp_pipe_route(M, x, out, NULL, GP_ROUTE_IDENT, max_pipes, stream).
 */
int gp_pipe_ident(int64_t M, const void* x, void* out, int max_pipes, void* stream);

/* Queue topologies of gp_pipe_route. */
#define GP_ROUTE_IDENT 0     /* x -> queue -> out                                            */
#define GP_ROUTE_BROADCAST 1 /* x -> queue with two consumers -> out and out2                */
                             /* (MpmcRingQueue<E, N, 1, 2>, bert_addln_ffn_pl.cuh:55)        */
#define GP_ROUTE_SPLIT 2     /* x -> queue -> 3 workers round robin (SplitQueueReader) ->    */
                             /* queue written round robin (SplitQueueWriter,                 */
                             /* bert_addln_ffn_pl.cuh:121) -> out in sequence order          */
#define GP_ROUTE_DRAIN 3     /* the broadcast with the second consumer discarding its tiles  */
                             /* (NullWriter; dummy_consumer, bert_addln_ffn_pl.cuh:178-187);  */
                             /* out2 is not written                                          */
#define GP_ROUTE_HANDOFF 4   /* queue hand-off benchmark (misc_tests/pipeperf/pipeperf.cu:     */
                             /* 125-163): a producer writes generated 128 x 128 fp16 tiles   */
                             /* (32 KiB) into a two-slot queue, the consumer reads each tile */
                             /* and folds it into a checksum; no HBM input.  x must be NULL, */
                             /* out is uint32[ceil(M / 128)]: out[t] = the sum mod 2^32 of   */
                             /* the words w = (t * 0x9E3779B1) ^ (i * 0x85EBCA77) of tile t, */
                             /* i < 64 * rows (word i of the tile in row-major order, rows = */
                             /* min(128, M - 128 t)); tiles t = g, g + P, ... go through     */
                             /* pipeline g of P                                              */
#define GP_ROUTE_RELOAD 5    /* x -> one-slot queue of 64-row entries -> out: the consumer   */
                             /* reads the same slot addresses every tile, so stale L1 lines  */
                             /* of its previous round would show (the check of the queue's   */
                             /* agent-scope payload loads); no counterpart in the reference  */

/*
 * Copy pipelines over the queue topologies the reference's apps use; out
 * (and out2 for GP_ROUTE_BROADCAST) must equal x bit for bit.  The exercise
 * of the queue library's multi-consumer and split reader / writer paths,
 * the striped input reader (GP_ROUTE_IDENT) and the null writer
 * (GP_ROUTE_DRAIN; out2 may then be NULL).  GP_ROUTE_HANDOFF times the
 * queue itself: x is NULL and out receives per-tile checksums (see above).
 */
int gp_pipe_route(int64_t M, const void* x, void* out, void* out2, int route, int max_pipes, void* stream);

/*
 * Diagnostics, no counterpart in the reference: one launch of a probe kernel
 * in which every SIMD runs two waves of back-to-back dense MFMAs -- `shape`
 * 32: v_mfma_f32_32x32x16, 16: v_mfma_f32_16x16x32, the same FLOPs per round
 * -- (GP_DTYPE_F16 or GP_DTYPE_BF16 operands, fp32 accumulation) on register
 * data for `iters` rounds, with no memory traffic but one 4-byte store per
 * lane into `out` (at least 2 x CUs x 256 floats, `out_floats` of them).
 * *flops receives the launch's FLOP count; timed on the stream, it gives the
 * dense MFMA rate the device sustains with that instruction (the engine clock
 * is set by the board's power and current limits), the ceiling for the
 * MFMA-bound kernels' measured rates.
 */
int gp_probe_mfma(int64_t iters, int dtype, int shape, void* out, int64_t out_floats, int64_t* flops, void* stream);

/*
 * Synthetic inputs, no counterpart in the reference (whose inputs come from
 * torch's host generator, apps/mgn_fullmlp/pipelined/val.py:15-21): fills
 * dst[0 .. n) (GP_DTYPE_F16 or GP_DTYPE_BF16, 2-byte aligned) with elements
 * offset .. offset + n - 1 of the N(0, 1) stream of `seed`: element e is
 * normal e % 4 of Philox-4x32-10 counter e / 4 under key `seed`, by
 * Box-Muller, rounded to nearest even.  A given (seed, e) gives the same value
 * for any n, offset, launch shape and device, and the same as the oracle's
 * host restatement.  Enqueued on `stream`; n = 0 is a no-op.
 */
int gp_fill_normal(void* dst, int64_t n, uint64_t seed, uint64_t offset, int dtype, void* stream);

/*
 * Waits for `stream`, then reports whether the last launch on it that
 * reports device-side failures failed (GP_ERR_TIMEOUT) or completed (GP_OK).
 * Those are the launches of gp_mgn_fullmlp_out, gp_mgn_linears_out,
 * gp_mgn_mlp_out (every impl), gp_mgn_edge_gather_out, gp_pipe_ident,
 * gp_pipe_route, gp_bert_ffn_impl_out / gp_bert_addln_ffn_out / gp_nerf_a_out
 * with GP_IMPL_PIPELINED, and gp_bert_ffn_out / gp_bert_addln_ffn_out (fused) with
 * H > 128: every wait between their workgroups or waves is bounded, and
 * one that runs out makes the launch end early and leave its outputs invalid
 * (the fused kernels store nothing after it).  The pipelined layouts also fail
 * when no pipeline's workgroups shared an XCD.  GP_ERR_INVALID_ARG if no such
 * launch was made on this stream.  The reference has no such check: a stuck
 * queue spins forever (common/mpmcq.cuh:83,104).
 */
int gp_pipeline_check(void* stream);

/*
 * Test hook: bounds every device-side wait of later launches (of the entry
 * points gp_pipeline_check covers) to `polls` polls; 0 restores the defaults
 * (2^20 polls of about 0.1 us for the waits inside a fused kernel's
 * workgroup, 2^22 polls of about 1 us for the queue waits between
 * workgroups).  A tiny bound makes those launches time out, so that a caller
 * can check its handling of GP_ERR_TIMEOUT with kernels that still end
 * normally.  Process-wide.  No counterpart in the reference.
 */
int gp_set_wait_limit(int64_t polls);

/*
 * Diagnostics: copies into dst (at least 256 * 8 * 12 * 8 bytes) the phase
 * timers of the last fused MGN launch (gp_mgn_fullmlp_out, gp_mgn_linears_out,
 * gp_mgn_mlp_out with the fused implementation, gp_mgn_edge_gather_out).
 * For wave w of workgroup b < 256 the 12 uint64 values at (b * 8 + w) * 12
 * are: the shader-clock ticks (s_memtime) spent in each of the wave's 8
 * phases summed over its tiles (waves 0-3, layer 1: X wait, stage-A barrier,
 * layer 1, hand-off wait, hand-off store; waves 4-7, layers 2-3: hand-off
 * wait, layer 2, exchange-free wait, exchange store, exchange-full wait,
 * layer-3 issue, LayerNorm and stores), the loop's total ticks, its
 * s_memrealtime ticks (100 MHz), its tiles and the launch's grid size.  Only
 * the diagnostic build libgpipes_phase.so records them; the product library
 * returns GP_ERR_INVALID_ARG.  No counterpart in the reference.
 */
int gp_phase_timers_read(void* dst, int64_t bytes);

#ifdef __cplusplus
}
#endif

#endif /* GPIPES_H */
