// C ABI of the dense MLP chains: the DLRM MLPs (gp_mlp_out, gp_dlrm_botmlp_out,
// gp_dlrm_topmlp_out), the NeRF MLP (gp_nerf_full_out and its allocation-free
// form) and the NerfA trunk (gp_nerf_a_out).
//
// The reference builds each app as one pipelined kernel of GEMM stage blocks
// linked by queues (apps/dlrm_botmlp/pipelined/dlrm_botmlp_pl.cuh:79-137,
// apps/dlrm_topmlp/pipelined/dlrm_topmlp_pl.cuh:105-187,
// apps/nerf_full/pipelined/nerf_full_pl.cuh:122-274).  Their layers are 256 to
// 1024 wide, so the weights (0.34 to 6 MB) cannot stay resident in one CU;
// here every layer is one launch of the wide GEMM stage (gemm.hip) with its
// bias and activation fused, over row chunks of 262,144.
// Narrow and odd widths are handled by padding, never by special kernels:
//   * weights are transposed into the workspace with zero rows and columns up
//     to K a multiple of 64 and N a multiple of 128, biases zero-padded to N;
//   * an input whose width is not a multiple of 8 (or not 16-byte aligned) is
//     copied into a padded buffer; other inputs are read in place, and the
//     GEMM zero-fills the columns past their width;
//   * concatenated inputs ([h | x], [bottleneck | d]) are built in place --
//     the GEMM writes h into the first columns of the wider buffer;
//   * a layer narrower than 128 outputs (the DLRM click head, the NeRF density
//     and colour heads) runs at 128 and its first columns are copied out.
// Padded activation columns hold act(0) and meet zero weight rows, so they
// contribute nothing.
#include <hip/hip_runtime.h>

#include <mutex>
#include <vector>

#include "../../include/gpipes.h"
#include "gp_host.hpp"
#include "gp_kernels.hpp"

namespace gp {
namespace {

// Rows per chunk: 262,144 rows give a 256-wide layer 1,024 tiles (four per CU,
// so each CU's next tile is copied while the previous one's epilogue runs)
// and keep a 256-wide activation (128 MiB) MALL-sized.
constexpr int64_t kChunkRows = 262144;
constexpr int64_t kMaxRows = (int64_t(1) << 31) - 1;  // GEMM tile indices are 32-bit
constexpr int64_t kMaxWidth = 16384;

int64_t rup(int64_t v, int64_t m) { return (v + m - 1) / m * m; }

// Sequential carving of one workspace allocation (256-byte aligned pieces).
struct Carve {
  size_t off = 0;
  size_t take(size_t bytes) {
    const size_t o = off;
    off += (bytes + 255) & ~size_t(255);
    return o;
  }
};

int act_ok(int act) {
  return act == GP_ACT_NONE || act == GP_ACT_RELU || act == GP_ACT_GELU_TANH || act == GP_ACT_SIGMOID;
}

// One dense layer prepared for the GEMM stage: either its weights in place
// (w [kw][Np], read by the GEMM in their own layout) or a transposed,
// zero-padded copy (wt) when the output width is not a multiple of 128.
struct Prepared {
  const void* wt;  // [Np][Kin], zero-padded (nullptr: w in place)
  const void* b;   // [Np], zero-padded; the caller's bias when w is in place
  int64_t Kin, Np;
  int act;
  const void* w = nullptr;  // [kw][Np]
  int64_t kw = 0;
};

// A layer of a chain small enough to read its weights in place
// (weights_in_place) does so when its output width is a multiple of 128 and
// weights and bias are 16-byte aligned; otherwise they are prepared
// (transposed, zero-padded) into the workspace by the chain's prep launch.
bool in_place(bool chain, int64_t N, const void* w, const void* b) {
  return chain && N % 128 == 0 && aligned16(w) && (!b || aligned16(b));
}


// ka: columns of `a` read (a multiple of 8, <= L.Kin); the rest count as zero.
hipError_t layer(const Prepared& L, int64_t rows, const void* a, int64_t lda, void* c, int64_t ldc, int ncu,
                 hipStream_t s, int64_t ka = 0, int dtype = GP_DTYPE_F16) {
  GemmArgs g{rows, L.Np, L.Kin, a, L.wt, L.b, nullptr, L.act, c};
  g.dtype = dtype;
  g.w = L.w;
  g.kw = L.kw;
  g.lda = lda;
  g.ldc = ldc;
  g.ka = ka;
  return gemm_launch(g, ncu, s);
}

const char* row_ptr(const void* base, int64_t row, int64_t stride) { return (const char*)base + row * stride * 2; }

int common_checks(int64_t M, const void* x, const void* out) {
  if (M < 0) return fail(GP_ERR_INVALID_ARG, "M must be >= 0 (got %lld)", (long long)M);
  if (M > kMaxRows) return fail(GP_ERR_SHAPE, "M too large (%lld)", (long long)M);
  if (M > 0 && (!x || !out)) return fail(GP_ERR_INVALID_ARG, "x and out must be non-NULL when M > 0");
  return GP_OK;
}

// DlrmMlp-style chain: widths[0] -> widths[1] -> ... -> widths[nl], act[i] after layer i;
// every tensor of element type dtype.
int run_chain(int64_t M, int nl, const int64_t* widths, const void* const* w, const void* const* b, const int* acts,
              const void* x, void* out, hipStream_t s, int dtype = GP_DTYPE_F16) {
  int dev = 0, ncu = 0;
  int rc = current_device_info(&dev, &ncu);
  if (rc) return rc;
  if (nl == 3 && widths[1] == 512 && widths[2] == 256 && widths[3] == 128 && dlrm_bot_supported(widths[0], acts)) {
    // The DLRM bottom MLP's shape: one fused kernel, activations on chip.  An
    // input or output that is not 16-byte aligned (a row slice, say) goes
    // through the workspace, so results never depend on how tensors are sliced.
    const bool cx = !aligned16(x), co = !aligned16(out);
    Carve cv;
    const size_t o_pk = cv.take(dlrm_bot_workspace());
    const size_t o_x = cx ? cv.take((size_t)M * widths[0] * 2) : 0;
    const size_t o_o = co ? cv.take((size_t)M * widths[3] * 2) : 0;
    char* ws = nullptr;
    if ((rc = workspace_acquire(dev, s, cv.off, (void**)&ws))) return rc;
    hipError_t e = hipSuccess;
    if (cx) e = hipMemcpyAsync(ws + o_x, x, (size_t)M * widths[0] * 2, hipMemcpyDeviceToDevice, s);
    if (e != hipSuccess) return fail_hip(e, "DLRM input alignment copy");
    e = dlrm_bot_launch(M, (int)widths[0], cx ? ws + o_x : x, w, b, acts, co ? ws + o_o : out, ws + o_pk, ncu, s,
                        dtype);
    if (e != hipSuccess) return fail_hip(e, "DLRM bottom MLP fused kernel launch");
    if (co && (e = hipMemcpyAsync(out, ws + o_o, (size_t)M * widths[3] * 2, hipMemcpyDeviceToDevice, s)) != hipSuccess)
      return fail_hip(e, "DLRM output copy");
    return GP_OK;
  }
  const int64_t CH = M < kChunkRows ? M : kChunkRows;
  std::vector<int64_t> kin(nl), np(nl);
  int64_t maxnp = 0;
  for (int i = 0; i < nl; ++i) {
    kin[i] = i == 0 ? rup(widths[0], 64) : np[i - 1];
    np[i] = rup(widths[i + 1], 128);
    maxnp = np[i] > maxnp ? np[i] : maxnp;
  }
  // An input whose rows are whole 16-byte chunks is read in place; the GEMM
  // zero-fills its columns up to the padded width.
  const bool direct_in = widths[0] % 8 == 0 && aligned16(x);
  const bool direct_out = np[nl - 1] == widths[nl] && aligned16(out);
  // A one-output last layer (the DLRM click head) is a GEMV over the previous
  // activations, written straight to out.
  const bool gemv_head = widths[nl] == 1 && nl >= 2 && widths[nl - 1] % 8 == 0 && aligned16(w[nl - 1]);
  // ... -> K -> 256 -> 1 (the DLRM top MLP's tail): the last two layers as one
  // fused kernel, written straight to out.  Its input rows are K wide: the
  // chain input (read in place or padded to kin[0] = K) or a previous layer's
  // output (np = K).
  const int tl = nl - 2;  // first layer of the fused tail
  const bool fused_tail =
      widths[nl] == 1 && nl >= 2 && widths[nl - 1] == 256 && dlrm_tail_supported(widths[tl], acts[tl], acts[nl - 1]);
  Carve cv;
  std::vector<size_t> o_wt(nl), o_b(nl);
  for (int i = 0; i < nl; ++i) {
    o_wt[i] = cv.take((size_t)np[i] * kin[i] * 2);
    o_b[i] = cv.take((size_t)np[i] * 2);
  }
  const size_t o_x = direct_in ? 0 : cv.take((size_t)CH * kin[0] * 2);
  const size_t o_h0 = cv.take((size_t)CH * maxnp * 2);
  const size_t o_h1 = cv.take((size_t)CH * maxnp * 2);
  const size_t o_tail = fused_tail ? cv.take(dlrm_tail_workspace(widths[tl])) : 0;
  char* ws = nullptr;
  if ((rc = workspace_acquire(dev, s, cv.off, (void**)&ws))) return rc;

  // Layers whose weights cannot be read in place are transposed and padded
  // into the workspace (one launch for all of them); the fused tail packs its
  // own.
  std::vector<Prepared> L(nl);
  std::vector<PrepSpec> ps;
  double flop = 0;
  for (int i = 0; i < nl; ++i) flop += 2.0 * M * widths[i] * widths[i + 1];
  const bool chain = weights_in_place(flop);
  for (int i = 0; i < (fused_tail ? tl : nl); ++i) {
    if (in_place(chain, widths[i + 1], w[i], b[i])) {
      L[i] = {nullptr, b[i], kin[i], np[i], acts[i], w[i], widths[i]};
    } else {
      ps.push_back({w[i], ws + o_wt[i], b[i], ws + o_b[i], widths[i], widths[i + 1], kin[i], np[i]});
      L[i] = {ws + o_wt[i], ws + o_b[i], kin[i], np[i], acts[i]};
    }
  }
  if (!ps.empty())
    if (hipError_t e = prep_launch(ps.data(), (int)ps.size(), s); e != hipSuccess)
      return fail_hip(e, "MLP weight preparation");
  char* hb[2] = {ws + o_h0, ws + o_h1};
  for (int64_t r0 = 0; r0 < M; r0 += CH) {
    const int64_t rows = M - r0 < CH ? M - r0 : CH;
    const void* a = row_ptr(x, r0, widths[0]);
    int64_t lda = widths[0];
    hipError_t e = hipSuccess;
    if (!direct_in) {
      e = place_launch(rows, a, widths[0], widths[0], ws + o_x, kin[0], kin[0], GP_ACT_NONE, ncu, s);
      a = ws + o_x;
      lda = kin[0];
    }
    for (int i = 0; i < nl && e == hipSuccess; ++i) {
      const bool last = i == nl - 1;
      if (i == tl && fused_tail) {
        e = dlrm_tail_launch(rows, widths[tl], a, w[tl], b[tl], acts[tl], w[nl - 1], b[nl - 1], acts[nl - 1],
                             (void*)row_ptr(out, r0, 1), ws + o_tail, ncu, s, dtype, r0 == 0);
        break;
      }
      if (last && gemv_head) {
        e = gemv1_launch(rows, widths[i], a, lda, w[i], b[i], acts[i], (void*)row_ptr(out, r0, 1), ncu, s, dtype);
        break;
      }
      void* c = last && direct_out ? (void*)row_ptr(out, r0, widths[nl]) : (void*)hb[i % 2];
      e = layer(L[i], rows, a, lda, c, np[i], ncu, s, i == 0 && direct_in ? widths[0] : 0, dtype);
      a = c;
      lda = np[i];
    }
    if (e == hipSuccess && !direct_out && !gemv_head && !fused_tail)
      e = place_launch(rows, a, lda, widths[nl], (void*)row_ptr(out, r0, widths[nl]), widths[nl], widths[nl],
                       GP_ACT_NONE, ncu, s);
    if (e != hipSuccess) return fail_hip(e, "MLP layer launch");
  }
  return GP_OK;
}

int check_chain(int nl, const int64_t* widths, const void* const* w, const int* acts) {
  for (int i = 0; i <= nl; ++i)
    if (widths[i] < 1 || widths[i] > kMaxWidth)
      return fail(GP_ERR_SHAPE, "width %d must be in [1, %lld] (got %lld)", i, (long long)kMaxWidth,
                  (long long)widths[i]);
  for (int i = 0; i < nl; ++i) {
    if (!w[i]) return fail(GP_ERR_INVALID_ARG, "weight %d is NULL", i);
    if (!act_ok(acts[i])) return fail(GP_ERR_INVALID_ARG, "unknown activation %d for layer %d", acts[i], i);
  }
  return GP_OK;
}

}  // namespace
}  // namespace gp

using namespace gp;

extern "C" {

int gp_mlp_dtype_out(int64_t M, int nlayers, const int64_t* widths, const void* const* w, const void* const* b,
                     const int* acts, const void* x, void* out, int dtype, void* stream) {
  clear_error();
  if (dtype != GP_DTYPE_F16 && dtype != GP_DTYPE_BF16) return fail(GP_ERR_INVALID_ARG, "unknown dtype %d", dtype);
  if (nlayers < 1 || nlayers > 32) return fail(GP_ERR_INVALID_ARG, "nlayers must be in [1, 32] (got %d)", nlayers);
  if (!widths || !w || !b || !acts) return fail(GP_ERR_INVALID_ARG, "widths, w, b and acts must be non-NULL");
  int rc = common_checks(M, x, out);
  if (rc) return rc;
  if ((rc = check_chain(nlayers, widths, w, acts))) return rc;
  if (M == 0) return GP_OK;
  return run_chain(M, nlayers, widths, w, b, acts, x, out, (hipStream_t)stream, dtype);
}

int gp_mlp_out(int64_t M, int nlayers, const int64_t* widths, const void* const* w, const void* const* b,
               const int* acts, const void* x, void* out, void* stream) {
  return gp_mlp_dtype_out(M, nlayers, widths, w, b, acts, x, out, GP_DTYPE_F16, stream);
}

int gp_dlrm_botmlp_out(int64_t M, int64_t K0, const void* x, const void* w1, const void* b1, const void* w2,
                       const void* b2, const void* w3, const void* b3, void* out, void* stream) {
  const int64_t widths[4] = {K0, 512, 256, 128};
  const void* w[3] = {w1, w2, w3};
  const void* b[3] = {b1, b2, b3};
  const int acts[3] = {GP_ACT_RELU, GP_ACT_RELU, GP_ACT_RELU};
  return gp_mlp_out(M, 3, widths, w, b, acts, x, out, stream);
}

int gp_dlrm_topmlp_out(int64_t M, int64_t K0, int64_t N5, const void* x, const void* w1, const void* b1,
                       const void* w2, const void* b2, const void* w3, const void* b3, const void* w4,
                       const void* b4, const void* w5, const void* b5, int act5, void* out, void* stream) {
  const int64_t widths[6] = {K0, 1024, 1024, 512, 256, N5};
  const void* w[5] = {w1, w2, w3, w4, w5};
  const void* b[5] = {b1, b2, b3, b4, b5};
  const int acts[5] = {GP_ACT_RELU, GP_ACT_RELU, GP_ACT_RELU, GP_ACT_RELU, act5};
  return gp_mlp_out(M, 5, widths, w, b, acts, x, out, stream);
}

// Argument checks shared by both NeRF entry points.
static int nerf_checks(int64_t M, int64_t Kx, int64_t Kd, int64_t Na, int64_t Nrgb, const void* x, const void* d,
                       const void* const* w, const void* const* b, int rgb_act, void* out_r, void* out_rgb) {
  int rc = common_checks(M, x, out_r);
  if (rc) return rc;
  if (M > 0 && (!d || !out_rgb)) return fail(GP_ERR_INVALID_ARG, "d and out_rgb must be non-NULL when M > 0");
  if (!w || !b) return fail(GP_ERR_INVALID_ARG, "w and b must be non-NULL");
  if (Kx < 1 || Kx > 1024 || Kd < 1 || Kd > 1024 || Na < 1 || Na > 1024 || Nrgb < 1 || Nrgb > 1024)
    return fail(GP_ERR_SHAPE, "Kx, Kd, Na and Nrgb must be in [1, 1024]");
  for (int i = 0; i < 12; ++i)
    if (!w[i]) return fail(GP_ERR_INVALID_ARG, "weight %d is NULL", i + 1);
  if (!act_ok(rgb_act)) return fail(GP_ERR_INVALID_ARG, "unknown activation %d", rgb_act);
  return GP_OK;
}

int gp_nerf_full_dtype_out(int64_t M, int64_t Kx, int64_t Kd, int64_t Na, int64_t Nrgb, const void* x,
                           const void* d, const void* const* w, const void* const* b, int rgb_act, void* out_r,
                           void* out_rgb, int dtype, void* stream) {
  clear_error();
  if (dtype != GP_DTYPE_F16 && dtype != GP_DTYPE_BF16) return fail(GP_ERR_INVALID_ARG, "unknown dtype %d", dtype);
  int rc = nerf_checks(M, Kx, Kd, Na, Nrgb, x, d, w, b, rgb_act, out_r, out_rgb);
  if (rc) return rc;
  if (M == 0) return GP_OK;
  int dev = 0, ncu = 0;
  if ((rc = current_device_info(&dev, &ncu))) return rc;
  hipStream_t s = (hipStream_t)stream;

  if (nerf_fused_supported(Kx, Kd, Na, Nrgb)) {
    // The fused kernel copies x and d rows from 16-byte aligned bases; an
    // input that is not (a row slice of a [M, 27] tensor, say) is copied into
    // the workspace first, so results never depend on how inputs are sliced.
    const bool cx = !aligned16(x), cd = !aligned16(d);
    Carve cv;
    const size_t o_st = cv.take(nerf_fused_workspace());
    const size_t o_x = cx ? cv.take((size_t)M * Kx * 2) : 0;
    const size_t o_d = cd ? cv.take((size_t)M * Kd * 2) : 0;
    char* ws = nullptr;
    if ((rc = workspace_acquire(dev, s, cv.off, (void**)&ws))) return rc;
    hipError_t e = hipSuccess;
    if (cx) e = hipMemcpyAsync(ws + o_x, x, (size_t)M * Kx * 2, hipMemcpyDeviceToDevice, s);
    if (e == hipSuccess && cd) e = hipMemcpyAsync(ws + o_d, d, (size_t)M * Kd * 2, hipMemcpyDeviceToDevice, s);
    if (e != hipSuccess) return fail_hip(e, "NeRF input alignment copy");
    e = nerf_fused_launch(M, (int)Kx, (int)Kd, (int)Na, (int)Nrgb, cx ? ws + o_x : x, cd ? ws + o_d : d, w, b,
                          rgb_act, out_r, out_rgb, ws + o_st, ncu, s, dtype);
    if (e != hipSuccess) return fail_hip(e, "NeRF fused kernel launch");
    return GP_OK;
  }

  // Wider inputs or heads: one wide-GEMM launch per layer.
  // Layer shapes of apps/nerf_full/torch/model.py:5-46 with hidden 256:
  // 1: Kx->256, 2-5: 256->256 (ReLU); 6: [h | x] -> 256, 7-8: 256->256 (ReLU);
  // 9: 256->Na (density, linear); 10: 256->256 (bottleneck, linear);
  // 11: [bottleneck | d] -> 128 (ReLU); 12: 128->Nrgb (colour, rgb_act).
  const int64_t H = 256, H2 = 128;
  const int64_t kx = rup(Kx, 64), cat1 = rup(H + Kx, 64), cat2 = rup(H + Kd, 64);
  const int64_t np9 = rup(Na, 128), np12 = rup(Nrgb, 128);
  struct Shape {
    int64_t K, N, Kin, Np;
    int act;
  };
  const Shape sh[12] = {
      {Kx, H, kx, H, GP_ACT_RELU},      {H, H, H, H, GP_ACT_RELU},         {H, H, H, H, GP_ACT_RELU},
      {H, H, H, H, GP_ACT_RELU},        {H, H, H, H, GP_ACT_RELU},         {H + Kx, H, cat1, H, GP_ACT_RELU},
      {H, H, H, H, GP_ACT_RELU},        {H, H, H, H, GP_ACT_RELU},         {H, Na, H, np9, GP_ACT_NONE},
      {H, H, H, H, GP_ACT_NONE},        {H + Kd, H2, cat2, H2, GP_ACT_RELU}, {H2, Nrgb, H2, np12, rgb_act},
  };
  const int64_t CH = M < kChunkRows ? M : kChunkRows;
  Carve cv;
  size_t o_wt[12], o_b[12];
  for (int i = 0; i < 12; ++i) {
    o_wt[i] = cv.take((size_t)sh[i].Np * sh[i].Kin * 2);
    o_b[i] = cv.take((size_t)sh[i].Np * 2);
  }
  const size_t o_x = cv.take((size_t)CH * kx * 2);      // x, padded
  const size_t o_c1 = cv.take((size_t)CH * cat1 * 2);   // [h5 | x]
  const size_t o_c2 = cv.take((size_t)CH * cat2 * 2);   // [bottleneck | d]
  const size_t o_h0 = cv.take((size_t)CH * H * 2);
  const size_t o_h1 = cv.take((size_t)CH * H * 2);
  const size_t o_hd = cv.take((size_t)CH * (np9 > np12 ? np9 : np12) * 2);  // padded head outputs
  char* ws = nullptr;
  if ((rc = workspace_acquire(dev, s, cv.off, (void**)&ws))) return rc;
  Prepared L[12];
  PrepSpec ps[12];
  int nps = 0;
  double flop = 0;
  for (int i = 0; i < 12; ++i) flop += 2.0 * M * sh[i].K * sh[i].N;
  const bool chain = weights_in_place(flop);
  for (int i = 0; i < 12; ++i) {
    if (in_place(chain, sh[i].N, w[i], b[i])) {
      L[i] = {nullptr, b[i], sh[i].Kin, sh[i].Np, sh[i].act, w[i], sh[i].K};
    } else {
      ps[nps++] = {w[i], ws + o_wt[i], b[i], ws + o_b[i], sh[i].K, sh[i].N, sh[i].Kin, sh[i].Np};
      L[i] = {ws + o_wt[i], ws + o_b[i], sh[i].Kin, sh[i].Np, sh[i].act};
    }
  }
  if (nps)
    if (hipError_t e = prep_launch(ps, nps, s); e != hipSuccess) return fail_hip(e, "NeRF weight preparation");
  char *xb = ws + o_x, *c1 = ws + o_c1, *c2 = ws + o_c2, *h0 = ws + o_h0, *h1 = ws + o_h1, *hd = ws + o_hd;
  for (int64_t r0 = 0; r0 < M; r0 += CH) {
    const int64_t rows = M - r0 < CH ? M - r0 : CH;
    hipError_t e = place_launch(rows, row_ptr(x, r0, Kx), Kx, Kx, xb, kx, kx, GP_ACT_NONE, ncu, s);
    // the skip and view-direction inputs go into the tails of the concat buffers
    if (e == hipSuccess) e = place_launch(rows, row_ptr(x, r0, Kx), Kx, Kx, c1 + H * 2, cat1, cat1 - H, GP_ACT_NONE,
                                          ncu, s);
    if (e == hipSuccess) e = place_launch(rows, row_ptr(d, r0, Kd), Kd, Kd, c2 + H * 2, cat2, cat2 - H, GP_ACT_NONE,
                                          ncu, s);
    if (e == hipSuccess) e = layer(L[0], rows, xb, kx, h0, H, ncu, s, 0, dtype);
    if (e == hipSuccess) e = layer(L[1], rows, h0, H, h1, H, ncu, s, 0, dtype);
    if (e == hipSuccess) e = layer(L[2], rows, h1, H, h0, H, ncu, s, 0, dtype);
    if (e == hipSuccess) e = layer(L[3], rows, h0, H, h1, H, ncu, s, 0, dtype);
    // h5 -> the first 256 columns of [h5 | x]
    if (e == hipSuccess) e = layer(L[4], rows, h1, H, c1, cat1, ncu, s, 0, dtype);
    if (e == hipSuccess) e = layer(L[5], rows, c1, cat1, h0, H, ncu, s, 0, dtype);
    if (e == hipSuccess) e = layer(L[6], rows, h0, H, h1, H, ncu, s, 0, dtype);
    if (e == hipSuccess) e = layer(L[7], rows, h1, H, h0, H, ncu, s, 0, dtype);    // trunk output
    if (e == hipSuccess) e = layer(L[8], rows, h0, H, hd, np9, ncu, s, 0, dtype);  // density head
    if (e == hipSuccess)
      e = place_launch(rows, hd, np9, Na, (void*)row_ptr(out_r, r0, Na), Na, Na, GP_ACT_NONE, ncu, s);
    // bottleneck -> the first 256 columns of [bottleneck | d]
    if (e == hipSuccess) e = layer(L[9], rows, h0, H, c2, cat2, ncu, s, 0, dtype);
    if (e == hipSuccess) e = layer(L[10], rows, c2, cat2, h1, H2, ncu, s, 0, dtype);
    if (e == hipSuccess) e = layer(L[11], rows, h1, H2, hd, np12, ncu, s, 0, dtype);
    if (e == hipSuccess)
      e = place_launch(rows, hd, np12, Nrgb, (void*)row_ptr(out_rgb, r0, Nrgb), Nrgb, Nrgb, GP_ACT_NONE, ncu, s);
    if (e != hipSuccess) return fail_hip(e, "NeRF layer launch");
  }
  return GP_OK;
}

int gp_nerf_full_out(int64_t M, int64_t Kx, int64_t Kd, int64_t Na, int64_t Nrgb, const void* x, const void* d,
                     const void* const* w, const void* const* b, int rgb_act, void* out_r, void* out_rgb,
                     void* stream) {
  return gp_nerf_full_dtype_out(M, Kx, Kd, Na, Nrgb, x, d, w, b, rgb_act, out_r, out_rgb, GP_DTYPE_F16, stream);
}

int gp_nerf_a_dtype_out(int64_t M, int64_t Kx, const void* x, const void* const* w, const void* const* b, void* out,
                        int impl, int dtype, void* stream) {
  clear_error();
  if (dtype != GP_DTYPE_F16 && dtype != GP_DTYPE_BF16) return fail(GP_ERR_INVALID_ARG, "unknown dtype %d", dtype);
  int rc = common_checks(M, x, out);
  if (rc) return rc;
  if (!w || !b) return fail(GP_ERR_INVALID_ARG, "w and b must be non-NULL");
  if (Kx < 1 || Kx > 1024) return fail(GP_ERR_SHAPE, "Kx must be in [1, 1024] (got %lld)", (long long)Kx);
  for (int i = 0; i < 8; ++i)
    if (!w[i]) return fail(GP_ERR_INVALID_ARG, "weight %d is NULL", i + 1);
  if (impl != GP_IMPL_FUSED && impl != GP_IMPL_PIPELINED) return fail(GP_ERR_INVALID_ARG, "unknown impl %d", impl);
  if (impl == GP_IMPL_PIPELINED && dtype != GP_DTYPE_F16)
    return fail(GP_ERR_INVALID_ARG, "the queue-chained NerfA layout runs in fp16 only");
  if (M == 0) return GP_OK;
  // Every NerfA path writes out in 16-byte stores.
  if (!aligned16(out)) return fail(GP_ERR_ALIGN, "out must be 16-byte aligned");
  int dev = 0, ncu = 0;
  if ((rc = current_device_info(&dev, &ncu))) return rc;
  hipStream_t s = (hipStream_t)stream;
  if (impl == GP_IMPL_PIPELINED) {
    if (!aligned16(x)) return fail(GP_ERR_ALIGN, "x must be 16-byte aligned");
    for (int i = 0; i < 8; ++i)
      if (!aligned16(w[i])) return fail(GP_ERR_ALIGN, "weight %d must be 16-byte aligned", i + 1);
    NerfAArgs a{M, Kx, x, {}, {}, out};
    for (int i = 0; i < 8; ++i) {
      a.w[i] = w[i];
      a.b[i] = b[i];
    }
    return nerf_a_pipelined_run(a, dev, ncu, s);
  }

  if (nerf_trunk_supported(Kx) && M <= (int64_t(1) << 31) - 1) {
    // The NeRF kernel's trunk: all eight layers of a 256-row tile in one
    // kernel.  x rows that do not start 16-byte aligned are copied into the
    // workspace first (as gp_nerf_full_out does), so results never depend on
    // how the input is sliced.
    const bool cx = !aligned16(x);
    Carve cv;
    const size_t o_st = cv.take(nerf_fused_workspace());
    const size_t o_x = cx ? cv.take((size_t)M * Kx * 2) : 0;
    char* ws = nullptr;
    if ((rc = workspace_acquire(dev, s, cv.off, (void**)&ws))) return rc;
    if (cx)
      if (hipError_t e = hipMemcpyAsync(ws + o_x, x, (size_t)M * Kx * 2, hipMemcpyDeviceToDevice, s); e != hipSuccess)
        return fail_hip(e, "NerfA input alignment copy");
    if (hipError_t e = nerf_trunk_launch(M, (int)Kx, cx ? ws + o_x : x, w, b, out, ws + o_st, ncu, s, dtype);
        e != hipSuccess)
      return fail_hip(e, "NerfA fused kernel launch");
    return GP_OK;
  }

  // Wider inputs: one wide-GEMM launch per layer (apps/nerf_a/torch/model.py:5-38):
  // 1: Kx -> 256, 2-5: 256 -> 256; 6: [h5 | x] -> 256; 7-8: 256 -> 256; ReLU after each.
  const int64_t H = 256;
  const int64_t kx = rup(Kx, 64), cat1 = rup(H + Kx, 64);
  const int64_t kin[8] = {kx, H, H, H, H, cat1, H, H};
  const int64_t kreal[8] = {Kx, H, H, H, H, H + Kx, H, H};
  const int64_t CH = M < kChunkRows ? M : kChunkRows;
  Carve cv;
  size_t o_wt[8], o_b[8];
  for (int i = 0; i < 8; ++i) {
    o_wt[i] = cv.take((size_t)H * kin[i] * 2);
    o_b[i] = cv.take((size_t)H * 2);
  }
  const size_t o_x = cv.take((size_t)CH * kx * 2);     // x, padded
  const size_t o_c1 = cv.take((size_t)CH * cat1 * 2);  // [h5 | x]
  const size_t o_h0 = cv.take((size_t)CH * H * 2);
  const size_t o_h1 = cv.take((size_t)CH * H * 2);
  char* ws = nullptr;
  if ((rc = workspace_acquire(dev, s, cv.off, (void**)&ws))) return rc;
  Prepared L[8];
  PrepSpec ps[8];
  int nps = 0;
  double flop = 0;
  for (int i = 0; i < 8; ++i) flop += 2.0 * M * kreal[i] * H;
  const bool chain = weights_in_place(flop);
  for (int i = 0; i < 8; ++i) {
    if (in_place(chain, H, w[i], b[i])) {
      L[i] = {nullptr, b[i], kin[i], H, GP_ACT_RELU, w[i], kreal[i]};
    } else {
      ps[nps++] = {w[i], ws + o_wt[i], b[i], ws + o_b[i], kreal[i], H, kin[i], H};
      L[i] = {ws + o_wt[i], ws + o_b[i], kin[i], H, GP_ACT_RELU};
    }
  }
  if (nps)
    if (hipError_t e = prep_launch(ps, nps, s); e != hipSuccess) return fail_hip(e, "NerfA weight preparation");
  char *xb = ws + o_x, *c1 = ws + o_c1, *h0 = ws + o_h0, *h1 = ws + o_h1;
  for (int64_t r0 = 0; r0 < M; r0 += CH) {
    const int64_t rows = M - r0 < CH ? M - r0 : CH;
    hipError_t e = place_launch(rows, row_ptr(x, r0, Kx), Kx, Kx, xb, kx, kx, GP_ACT_NONE, ncu, s);
    if (e == hipSuccess) e = place_launch(rows, row_ptr(x, r0, Kx), Kx, Kx, c1 + H * 2, cat1, cat1 - H, GP_ACT_NONE,
                                          ncu, s);
    if (e == hipSuccess) e = layer(L[0], rows, xb, kx, h0, H, ncu, s, 0, dtype);
    if (e == hipSuccess) e = layer(L[1], rows, h0, H, h1, H, ncu, s, 0, dtype);
    if (e == hipSuccess) e = layer(L[2], rows, h1, H, h0, H, ncu, s, 0, dtype);
    if (e == hipSuccess) e = layer(L[3], rows, h0, H, h1, H, ncu, s, 0, dtype);
    // h5 -> the first 256 columns of [h5 | x]
    if (e == hipSuccess) e = layer(L[4], rows, h1, H, c1, cat1, ncu, s, 0, dtype);
    if (e == hipSuccess) e = layer(L[5], rows, c1, cat1, h0, H, ncu, s, 0, dtype);
    if (e == hipSuccess) e = layer(L[6], rows, h0, H, h1, H, ncu, s, 0, dtype);
    if (e == hipSuccess) e = layer(L[7], rows, h1, H, (void*)row_ptr(out, r0, H), H, ncu, s, 0, dtype);
    if (e != hipSuccess) return fail_hip(e, "NerfA layer launch");
  }
  return GP_OK;
}

int gp_nerf_a_out(int64_t M, int64_t Kx, const void* x, const void* const* w, const void* const* b, void* out, int impl,
                  void* stream) {
  return gp_nerf_a_dtype_out(M, Kx, x, w, b, out, impl, GP_DTYPE_F16, stream);
}

int gp_nerf_full_out_noalloc(int64_t M, int64_t Kx, int64_t Kd, int64_t Na, int64_t Nrgb, const void* x,
                             const void* d, const void* const* w, const void* const* b, int rgb_act, void* out_r,
                             void* out_rgb, void* stream) {
  clear_error();
  int rc = nerf_checks(M, Kx, Kd, Na, Nrgb, x, d, w, b, rgb_act, out_r, out_rgb);
  if (rc) return rc;
  if (!nerf_fused_supported(Kx, Kd, Na, Nrgb))
    return fail(GP_ERR_SHAPE,
                "the allocation-free NeRF call runs the fused kernel only, whose scratch is fixed: Kx <= 64, "
                "Kd <= 32, Na <= 64, Nrgb <= 64 (got %lld, %lld, %lld, %lld); use gp_nerf_full_out",
                (long long)Kx, (long long)Kd, (long long)Na, (long long)Nrgb);
  if (M == 0) return GP_OK;
  if (M > (int64_t(1) << 31) - 1) return fail(GP_ERR_SHAPE, "M must be < 2^31 (got %lld)", (long long)M);
  if (!aligned16(x) || !aligned16(d))
    return fail(GP_ERR_ALIGN, "x and d must be 16-byte aligned (the allocation-free call cannot copy them)");
  int dev = 0, ncu = 0;
  if ((rc = current_device_info(&dev, &ncu))) return rc;
  NerfScratch sc{};
  if ((rc = nerf_static_scratch(dev, &sc))) return rc;
  if (sc.bytes < nerf_fused_workspace())
    return fail(GP_ERR_SHAPE, "static scratch of %zu bytes is below the %zu the kernel needs", sc.bytes,
                nerf_fused_workspace());
  // An eager call waits for the previous call's kernels on this GPU (whatever
  // its stream) and records the event after its own; a call under capture is
  // not chained (a graph cannot wait on an event recorded outside it).
  const hipStream_t s = (hipStream_t)stream;
  std::lock_guard<std::mutex> lk(*sc.lock);
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  hipError_t e = hipStreamIsCapturing(s, &cs);
  if (e != hipSuccess) return fail_hip(e, "hipStreamIsCapturing");
  const bool eager = cs == hipStreamCaptureStatusNone;
  if (eager && (e = hipStreamWaitEvent(s, sc.last, 0)) != hipSuccess) return fail_hip(e, "hipStreamWaitEvent");
  e = nerf_fused_launch(M, (int)Kx, (int)Kd, (int)Na, (int)Nrgb, x, d, w, b, rgb_act, out_r, out_rgb, sc.ptr, ncu, s);
  if (e != hipSuccess) return fail_hip(e, "NeRF fused kernel launch");
  if (eager && (e = hipEventRecord(sc.last, s)) != hipSuccess) return fail_hip(e, "hipEventRecord");
  return GP_OK;
}

}  // extern "C"
