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
#define GP_ERR_TIMEOUT (-5)     /* a queue wait exceeded its spin bound        */
#define GP_ERR_NO_DEVICE (-6)   /* no usable gfx950 device                     */

/* Implementation selector for gp_mgn_mlp_out. */
#define GP_IMPL_FUSED 0     /* persistent fused kernel (default, fastest)   */
#define GP_IMPL_PIPELINED 1 /* stage-chained kernel with L2 ring queues      */

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
 * NULL) skips the LayerNorm.  `impl` is GP_IMPL_FUSED or GP_IMPL_PIPELINED.
 * The node MLP of MeshGraphNet is K = 256.  Both entry points above are this
 * call with K = 384.
 */
int gp_mgn_mlp_out(int64_t M, int64_t K, const void* x, const void* w1, const void* b1,
                   const void* w2, const void* b2, const void* w3, const void* b3,
                   const void* gamma, const void* beta, float eps, void* out, int impl,
                   void* stream);

#ifdef __cplusplus
}
#endif

#endif /* GPIPES_H */
