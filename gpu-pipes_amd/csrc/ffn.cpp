// C ABI of the wide operators: the GEMM stage with any N / K (gp_gemm_out),
// the BERT feed-forward block (gp_bert_ffn_out) and the add + LayerNorm + FFN
// block of the bert_addln_ffn app (gp_bert_addln_ffn_out).
//
// The reference's pipelined BERT FFN (apps/bert_ffn/pipelined/bert_ffn_pl.cuh:
// 79-162) chains GEMM + bias + ReLU -> GEMM + bias with the residual as
// accumulator -> LayerNorm workers through queues, sized for H = 128 and
// FF = 512.  At BERT-large width the two GEMMs are compute-bound and their
// weights cannot be held on chip, so here the block is three launches per row
// chunk: GEMM1 with a bias + activation epilogue, GEMM2 with a bias +
// residual epilogue, and the LayerNorm stage -- the shape of the reference's
// bulk-sync variant (apps/bert_ffn/bulksync/bert_ffn_bs.cuh:12-27) with the add
// fused.  Rows are processed in chunks so the FF-wide activations of one chunk
// (at most 128 MiB: 16384 x 4096 at BERT-large width) can stay in the 256 MB
// Infinity Cache between the two GEMMs rather than make a round trip through
// HBM.
#include <hip/hip_runtime.h>

#include "../../include/gpipes.h"
#include "gp_host.hpp"
#include "gp_kernels.hpp"

namespace gp {
namespace {

constexpr int64_t kMaxDim = 16384;
constexpr int64_t kMaxRows = (int64_t(1) << 31) - 1;  // GEMM tile indices are 32-bit
// Row chunks hold their per-row workspace (the FF-wide activations plus any
// H-wide intermediate rows, `row_elems` 16-bit values a row) within
// kFfnChunkBytes (128 MiB, half the Infinity Cache): 16384 rows at BERT-large
// width, where GEMM1 has 1024 tiles and GEMM2 256 tiles per chunk, whole
// multiples of the 256 CUs.  Narrower blocks take more rows per chunk, hence
// fewer, fuller launches (the bert_addln_ffn app's 32,768 rows at FF 512 are
// one chunk).
constexpr int64_t kFfnChunkBytes = int64_t(128) << 20;
int64_t ffn_chunk_rows(int64_t row_elems) {
  const int64_t r = kFfnChunkBytes / (row_elems * 2) / 256 * 256;
  return r < 256 ? 256 : r;
}

size_t round_up(size_t v) { return (v + 255) & ~size_t(255); }

int check_act(int act) {
  if (act != GP_ACT_NONE && act != GP_ACT_RELU && act != GP_ACT_GELU_TANH && act != GP_ACT_SIGMOID)
    return fail(GP_ERR_INVALID_ARG, "unknown activation %d", act);
  return GP_OK;
}

int check_dtype(int dtype) {
  if (dtype != GP_DTYPE_F16 && dtype != GP_DTYPE_BF16) return fail(GP_ERR_INVALID_ARG, "unknown dtype %d", dtype);
  return GP_OK;
}

int need16(const void* p, const char* name) {
  if (!p) return fail(GP_ERR_INVALID_ARG, "%s is NULL", name);
  if (!aligned16(p)) return fail(GP_ERR_ALIGN, "%s must be 16-byte aligned", name);
  return GP_OK;
}

int opt16(const void* p, const char* name) {
  if (p && !aligned16(p)) return fail(GP_ERR_ALIGN, "%s must be 16-byte aligned", name);
  return GP_OK;
}

const char* at_row(const void* base, int64_t row, int64_t width) { return (const char*)base + row * width * 2; }

// The LayerNorm epilogues of one call.  Below 128 features a row stays in one
// wave; wider rows exchange partial statistics through a queue arena, under
// one epoch for the whole call (its launches are rounds of that epoch, so a
// failed wait in any of them reads as a failure of the call), whose status
// word gp_pipeline_check reads.
struct LnEpilogue {
  void* ws = nullptr;
  uint32_t epoch = 0;
  int64_t round = 0;

  int init(int dev, hipStream_t s, int64_t rows, int64_t H) {
    if (H == 128) return GP_OK;
    const int rc = arena_acquire(dev, s, gemm_ln_ws_bytes(rows, H), kArenaLayoutGemmLn, &ws, &epoch);
    if (rc) return rc;
    status_note(dev, s, (unsigned long long*)ws, epoch);
    return GP_OK;
  }
  GemmArgs apply(GemmArgs g, const void* gamma, const void* beta, float eps) {
    g.ln = 1;
    g.gamma = gamma;
    g.beta = beta;
    g.eps = eps;
    if (ws) {
      g.ln_ws = ws;
      g.status = (unsigned long long*)ws;
      g.epoch = epoch;
      g.spin_limit = (int)wait_limit(0);
      g.ln_round = round++;
    }
    return g;
  }
};

// Rows per chunk of the FFN blocks with the LayerNorm in the GEMM epilogue:
// at most ffn_chunk_rows(row_elems) and at most the rows one LayerNorm-exchange
// launch can take (gemm_ln_max_rows).  0 when the epilogue cannot take the LayerNorm.
int64_t ln_chunk_rows(int64_t H, int64_t row_elems, int ncu) {
  const int64_t r = gemm_ln_max_rows(H, ncu), c = ffn_chunk_rows(row_elems);
  return r < 256 ? 0 : (r < c ? r : c);
}

}  // namespace
}  // namespace gp

using namespace gp;

extern "C" {

int gp_gemm_dtype_out(int64_t M, int64_t N, int64_t K, const void* x, const void* w, const void* b, const void* r,
                      int act, void* out, int dtype, void* stream) {
  clear_error();
  int rc;
  if ((rc = check_dtype(dtype))) return rc;
  if (M < 0) return fail(GP_ERR_INVALID_ARG, "M must be >= 0 (got %lld)", (long long)M);
  if (N < 128 || N > kMaxDim || N % 128)
    return fail(GP_ERR_SHAPE, "N must be a multiple of 128 in [128, %lld] (got %lld)", (long long)kMaxDim,
                (long long)N);
  if (K < 64 || K > kMaxDim || K % 64)
    return fail(GP_ERR_SHAPE, "K must be a multiple of 64 in [64, %lld] (got %lld)", (long long)kMaxDim,
                (long long)K);
  if (M > kMaxRows) return fail(GP_ERR_SHAPE, "M too large (%lld)", (long long)M);
  if ((rc = check_act(act))) return rc;
  if (r && act != GP_ACT_NONE) return fail(GP_ERR_INVALID_ARG, "a residual input requires act = GP_ACT_NONE");
  if ((rc = need16(w, "w")) || (rc = opt16(b, "b")) || (rc = opt16(r, "r"))) return rc;
  if (M == 0) return GP_OK;
  if ((rc = need16(x, "x")) || (rc = need16(out, "out"))) return rc;
  int dev = 0, ncu = 0;
  if ((rc = current_device_info(&dev, &ncu))) return rc;
  hipStream_t s = (hipStream_t)stream;
  if (weights_in_place(2.0 * M * N * K)) {
    GemmArgs g = gemm_w(M, N, K, x, w, b, r, act, out);
    g.dtype = dtype;
    const hipError_t e = gemm_launch(g, ncu, s);
    return e == hipSuccess ? GP_OK : fail_hip(e, "gemm launch");
  }
  void* ws = nullptr;
  if ((rc = workspace_acquire(dev, s, (size_t)N * K * 2, &ws))) return rc;
  hipError_t e = transpose_launch(w, ws, K, N, s);
  if (e != hipSuccess) return fail_hip(e, "transpose launch");
  GemmArgs g{M, N, K, x, ws, b, r, act, out};
  g.dtype = dtype;
  e = gemm_launch(g, ncu, s);
  return e == hipSuccess ? GP_OK : fail_hip(e, "gemm launch");
}

int gp_gemm_out(int64_t M, int64_t N, int64_t K, const void* x, const void* w, const void* b, const void* r,
                int act, void* out, void* stream) {
  return gp_gemm_dtype_out(M, N, K, x, w, b, r, act, out, GP_DTYPE_F16, stream);
}

int gp_bert_ffn_dtype_out(int64_t M, int64_t H, int64_t FF, const void* x, const void* w1, const void* b1,
                          const void* w2, const void* b2, const void* gamma, const void* beta, float eps, int act,
                          void* out, int dtype, void* stream) {
  clear_error();
  int rc;
  if ((rc = check_dtype(dtype))) return rc;
  if (M < 0) return fail(GP_ERR_INVALID_ARG, "M must be >= 0 (got %lld)", (long long)M);
  if (H != 128 && H != 256 && H != 512 && H != 1024)
    return fail(GP_ERR_SHAPE, "H must be 128, 256, 512 or 1024 (got %lld)", (long long)H);
  if (FF < 128 || FF > kMaxDim || FF % 128)
    return fail(GP_ERR_SHAPE, "FF must be a multiple of 128 in [128, %lld] (got %lld)", (long long)kMaxDim,
                (long long)FF);
  if (M > kMaxRows) return fail(GP_ERR_SHAPE, "M too large (%lld)", (long long)M);
  if ((rc = check_act(act))) return rc;
  if (!(eps >= 0.f)) return fail(GP_ERR_INVALID_ARG, "eps must be >= 0");
  if ((rc = need16(w1, "w1")) || (rc = need16(w2, "w2")) || (rc = opt16(b1, "b1")) || (rc = opt16(b2, "b2")) ||
      (rc = opt16(gamma, "gamma")) || (rc = opt16(beta, "beta")))
    return rc;
  if (M == 0) return GP_OK;
  if ((rc = need16(x, "x")) || (rc = need16(out, "out"))) return rc;
  int dev = 0, ncu = 0;
  if ((rc = current_device_info(&dev, &ncu))) return rc;
  hipStream_t s = (hipStream_t)stream;

  // Workspace: w1^T [FF][H], w2^T [H][FF] (unless the GEMMs read w1 and w2
  // in place), then one chunk of activations [CH][FF] and, when the
  // LayerNorm is a launch of its own, of pre-LayerNorm rows [CH][H].
  const bool inplace = weights_in_place(4.0 * M * H * FF);
  const int64_t lnch = ln_chunk_rows(H, FF, ncu);
  const bool fuse_ln = lnch > 0;
  if (!fuse_ln && dtype != GP_DTYPE_F16)
    return fail(GP_ERR_SHAPE, "bf16 needs the LayerNorm in the GEMM epilogue, which this device's %d CUs cannot hold", ncu);
  const int64_t chmax = fuse_ln ? lnch : ffn_chunk_rows(FF + H);
  const int64_t CH = M < chmax ? M : chmax;
  const size_t o_w2t = inplace ? 0 : round_up((size_t)FF * H * 2);
  const size_t o_act = o_w2t + (inplace ? 0 : round_up((size_t)FF * H * 2));
  const size_t o_y = o_act + round_up((size_t)CH * FF * 2);
  const size_t total = o_y + (fuse_ln ? 0 : round_up((size_t)CH * H * 2));
  char* ws = nullptr;
  if ((rc = workspace_acquire(dev, s, total, (void**)&ws))) return rc;
  void *w1t = ws, *w2t = ws + o_w2t, *hbuf = ws + o_act, *ybuf = ws + o_y;

  hipError_t e = hipSuccess;
  if (!inplace) {
    const PrepSpec ps[2] = {{w1, w1t, nullptr, nullptr, H, FF, H, FF}, {w2, w2t, nullptr, nullptr, FF, H, FF, H}};
    e = prep_launch(ps, 2, s);
    if (e != hipSuccess) return fail_hip(e, "transpose launch");
  }
  // layer GEMM arguments: the weights in place or their transposed copies
  auto g = [&](int64_t rows, int64_t N, int64_t K, const void* a, const void* w, const void* wt, const void* b,
               const void* r, int ac, void* c) {
    GemmArgs ga = inplace ? gemm_w(rows, N, K, a, w, b, r, ac, c) : GemmArgs{rows, N, K, a, wt, b, r, ac, c};
    ga.dtype = dtype;
    return ga;
  };
  LnEpilogue lne;
  if (fuse_ln && (rc = lne.init(dev, s, CH, H))) return rc;
  for (int64_t r0 = 0; r0 < M; r0 += CH) {
    const int64_t rows = M - r0 < CH ? M - r0 : CH;
    const void* xc = at_row(x, r0, H);
    char* const oc = (char*)out + r0 * H * 2;
    e = gemm_launch(g(rows, FF, H, xc, w1, w1t, b1, nullptr, act, hbuf), ncu, s);
    if (e != hipSuccess) return fail_hip(e, "FFN GEMM1 launch");
    if (fuse_ln) {
      // GEMM2 + bias + residual + LayerNorm in one launch
      e = gemm_launch(lne.apply(g(rows, H, FF, hbuf, w2, w2t, b2, xc, GP_ACT_NONE, oc), gamma, beta, eps), ncu, s);
      if (e != hipSuccess) return fail_hip(e, "FFN GEMM2 + LayerNorm launch");
      continue;
    }
    e = gemm_launch(g(rows, H, FF, hbuf, w2, w2t, b2, xc, GP_ACT_NONE, ybuf), ncu, s);
    if (e != hipSuccess) return fail_hip(e, "FFN GEMM2 launch");
    e = layer_norm_launch(rows, H, ybuf, gamma, beta, eps, oc, ncu, s);
    if (e != hipSuccess) return fail_hip(e, "FFN LayerNorm launch");
  }
  return GP_OK;
}

int gp_bert_ffn_out(int64_t M, int64_t H, int64_t FF, const void* x, const void* w1, const void* b1,
                    const void* w2, const void* b2, const void* gamma, const void* beta, float eps, int act,
                    void* out, void* stream) {
  return gp_bert_ffn_dtype_out(M, H, FF, x, w1, b1, w2, b2, gamma, beta, eps, act, out, GP_DTYPE_F16, stream);
}

int gp_bert_ffn_impl_out(int64_t M, int64_t H, int64_t FF, const void* x, const void* w1, const void* b1,
                         const void* w2, const void* b2, const void* gamma, const void* beta, float eps, int act,
                         void* out, int impl, void* stream) {
  if (impl == GP_IMPL_FUSED)
    return gp_bert_ffn_dtype_out(M, H, FF, x, w1, b1, w2, b2, gamma, beta, eps, act, out, GP_DTYPE_F16, stream);
  clear_error();
  int rc;
  if (impl != GP_IMPL_PIPELINED) return fail(GP_ERR_INVALID_ARG, "unknown impl %d", impl);
  if (M < 0) return fail(GP_ERR_INVALID_ARG, "M must be >= 0 (got %lld)", (long long)M);
  if (H != 128 || FF != 512)
    return fail(GP_ERR_SHAPE, "the pipelined layout is built for the app's shape H = 128, FF = 512 (got %lld, %lld)",
                (long long)H, (long long)FF);
  if (M > kMaxRows) return fail(GP_ERR_SHAPE, "M too large (%lld)", (long long)M);
  if (act != GP_ACT_RELU && act != GP_ACT_GELU_TANH)
    return fail(GP_ERR_INVALID_ARG, "the pipelined layout supports ReLU and GELU(tanh) only");
  if (!(eps >= 0.f)) return fail(GP_ERR_INVALID_ARG, "eps must be >= 0");
  if ((rc = need16(w1, "w1")) || (rc = need16(w2, "w2")) || (rc = opt16(b1, "b1")) || (rc = opt16(b2, "b2")) ||
      (rc = opt16(gamma, "gamma")) || (rc = opt16(beta, "beta")))
    return rc;
  if (M == 0) return GP_OK;
  if ((rc = need16(x, "x")) || (rc = need16(out, "out"))) return rc;
  int dev = 0, ncu = 0;
  if ((rc = current_device_info(&dev, &ncu))) return rc;
  const BertFfnArgs a{M, H, FF, x, w1, b1, w2, b2, gamma, beta, eps, act, out};
  return bert_ffn_pipelined_run(a, dev, ncu, (hipStream_t)stream);
}

int gp_bert_addln_ffn_dtype_out(int64_t M, int64_t H, int64_t FF, const void* attn, const void* x,
                                const void* w0, const void* b0, const void* w1, const void* b1, const void* w2,
                                const void* b2, const void* ga0, const void* be0, const void* ga2, const void* be2,
                                float eps, int act, void* out, int impl, int dtype, void* stream) {
  clear_error();
  int rc;
  if ((rc = check_dtype(dtype))) return rc;
  if (dtype != GP_DTYPE_F16 && impl != GP_IMPL_FUSED)
    return fail(GP_ERR_INVALID_ARG, "bf16 runs the fused implementation only (the queue-chained layout is fp16)");
  if (M < 0) return fail(GP_ERR_INVALID_ARG, "M must be >= 0 (got %lld)", (long long)M);
  if (H != 128 && H != 256 && H != 512 && H != 1024)
    return fail(GP_ERR_SHAPE, "H must be 128, 256, 512 or 1024 (got %lld)", (long long)H);
  if (FF < 128 || FF > kMaxDim || FF % 128)
    return fail(GP_ERR_SHAPE, "FF must be a multiple of 128 in [128, %lld] (got %lld)", (long long)kMaxDim,
                (long long)FF);
  if (M > kMaxRows) return fail(GP_ERR_SHAPE, "M too large (%lld)", (long long)M);
  if ((rc = check_act(act))) return rc;
  if (impl != GP_IMPL_FUSED && impl != GP_IMPL_PIPELINED) return fail(GP_ERR_INVALID_ARG, "unknown impl %d", impl);
  if (!(eps >= 0.f)) return fail(GP_ERR_INVALID_ARG, "eps must be >= 0");
  if ((rc = need16(w0, "w0")) || (rc = need16(w1, "w1")) || (rc = need16(w2, "w2")) || (rc = opt16(b0, "b0")) ||
      (rc = opt16(b1, "b1")) || (rc = opt16(b2, "b2")) || (rc = opt16(ga0, "ga0")) || (rc = opt16(be0, "be0")) ||
      (rc = opt16(ga2, "ga2")) || (rc = opt16(be2, "be2")))
    return rc;
  if (M == 0) return GP_OK;
  if ((rc = need16(attn, "attn_out")) || (rc = need16(x, "x")) || (rc = need16(out, "out"))) return rc;
  int dev = 0, ncu = 0;
  if ((rc = current_device_info(&dev, &ncu))) return rc;
  hipStream_t s = (hipStream_t)stream;
  if (impl == GP_IMPL_PIPELINED) {
    const BertAddlnArgs a{M, H, FF, attn, x, w0, b0, w1, b1, w2, b2, ga0, be0, ga2, be2, eps, act, out};
    return bert_addln_pipelined_run(a, dev, ncu, s);
  }

  // Chain: per row chunk, GEMM0 (+ b0 + x), LN0, GEMM1 (+ b1, act), GEMM2 (+ b2 + h0), LN2.
  // Workspace: w0^T [H][H], w1^T [FF][H], w2^T [H][FF] (unless the GEMMs
  // read the weights in place), then for one chunk h0 [CH][H], the
  // activations [CH][FF] and, when the LayerNorms are launches of their own,
  // the pre-LayerNorm rows y [CH][H].
  const bool inplace = weights_in_place(2.0 * M * H * (H + 2.0 * FF));
  const int64_t lnch = ln_chunk_rows(H, FF + H, ncu);
  const bool fuse_ln = lnch > 0;
  if (!fuse_ln && dtype != GP_DTYPE_F16)
    return fail(GP_ERR_SHAPE, "bf16 needs the LayerNorm in the GEMM epilogue, which this device's %d CUs cannot hold", ncu);
  const int64_t chmax = fuse_ln ? lnch : ffn_chunk_rows(FF + 2 * H);
  const int64_t CH = M < chmax ? M : chmax;
  const size_t o_w1t = inplace ? 0 : round_up((size_t)H * H * 2);
  const size_t o_w2t = o_w1t + (inplace ? 0 : round_up((size_t)FF * H * 2));
  const size_t o_y = o_w2t + (inplace ? 0 : round_up((size_t)FF * H * 2));
  const size_t o_h0 = o_y + (fuse_ln ? 0 : round_up((size_t)CH * H * 2));
  const size_t o_act = o_h0 + round_up((size_t)CH * H * 2);
  const size_t total = o_act + round_up((size_t)CH * FF * 2);
  char* ws = nullptr;
  if ((rc = workspace_acquire(dev, s, total, (void**)&ws))) return rc;
  void *w0t = ws, *w1t = ws + o_w1t, *w2t = ws + o_w2t, *ybuf = ws + o_y, *h0 = ws + o_h0, *abuf = ws + o_act;
  hipError_t e = hipSuccess;
  if (!inplace) {
    const PrepSpec ps[3] = {{w0, w0t, nullptr, nullptr, H, H, H, H},
                            {w1, w1t, nullptr, nullptr, H, FF, H, FF},
                            {w2, w2t, nullptr, nullptr, FF, H, FF, H}};
    e = prep_launch(ps, 3, s);
    if (e != hipSuccess) return fail_hip(e, "transpose launch");
  }
  auto g = [&](int64_t rows, int64_t N, int64_t K, const void* a, const void* w, const void* wt, const void* b,
               const void* r, int ac, void* c) {
    GemmArgs ga = inplace ? gemm_w(rows, N, K, a, w, b, r, ac, c) : GemmArgs{rows, N, K, a, wt, b, r, ac, c};
    ga.dtype = dtype;
    return ga;
  };
  LnEpilogue lne;
  if (fuse_ln && (rc = lne.init(dev, s, CH, H))) return rc;
  for (int64_t r0 = 0; r0 < M; r0 += CH) {
    const int64_t rows = M - r0 < CH ? M - r0 : CH;
    if (fuse_ln) {
      // GEMM0 + b0 + x + LN0, GEMM1 + b1 + act, GEMM2 + b2 + h0 + LN2
      char* const oc = (char*)out + r0 * H * 2;
      e = gemm_launch(lne.apply(g(rows, H, H, at_row(attn, r0, H), w0, w0t, b0, at_row(x, r0, H), GP_ACT_NONE, h0),
                                ga0, be0, eps), ncu, s);
      if (e == hipSuccess) e = gemm_launch(g(rows, FF, H, h0, w1, w1t, b1, nullptr, act, abuf), ncu, s);
      if (e == hipSuccess)
        e = gemm_launch(lne.apply(g(rows, H, FF, abuf, w2, w2t, b2, h0, GP_ACT_NONE, oc), ga2, be2, eps), ncu, s);
      if (e != hipSuccess) return fail_hip(e, "bert_addln_ffn launch");
      continue;
    }
    e = gemm_launch(g(rows, H, H, at_row(attn, r0, H), w0, w0t, b0, at_row(x, r0, H), GP_ACT_NONE, ybuf), ncu, s);
    if (e == hipSuccess) e = layer_norm_launch(rows, H, ybuf, ga0, be0, eps, h0, ncu, s);
    if (e == hipSuccess) e = gemm_launch(g(rows, FF, H, h0, w1, w1t, b1, nullptr, act, abuf), ncu, s);
    if (e == hipSuccess) e = gemm_launch(g(rows, H, FF, abuf, w2, w2t, b2, h0, GP_ACT_NONE, ybuf), ncu, s);
    if (e == hipSuccess) e = layer_norm_launch(rows, H, ybuf, ga2, be2, eps, (char*)out + r0 * H * 2, ncu, s);
    if (e != hipSuccess) return fail_hip(e, "bert_addln_ffn launch");
  }
  return GP_OK;
}

int gp_bert_addln_ffn_out(int64_t M, int64_t H, int64_t FF, const void* attn, const void* x, const void* w0,
                          const void* b0, const void* w1, const void* b1, const void* w2, const void* b2,
                          const void* ga0, const void* be0, const void* ga2, const void* be2, float eps, int act,
                          void* out, int impl, void* stream) {
  return gp_bert_addln_ffn_dtype_out(M, H, FF, attn, x, w0, b0, w1, b1, w2, b2, ga0, be0, ga2, be2, eps, act, out,
                                     impl, GP_DTYPE_F16, stream);
}

}  // extern "C"
