// Fused MeshGraphNet MLP for gfx950: Linear(K->128)+ReLU, Linear(128->128)+ReLU,
// Linear(128->128) [, LayerNorm(128)] in one persistent kernel.
//
// Reference behaviour: apps/mgn_fullmlp/pipelined/mgn_fullmlp_pl.cuh:83-252
// (three GEMM stage blocks + five LayerNorm blocks per pipeline row, chained by
// global-memory queues) and apps/mgn_linears/pipelined/mgn_linears_pl.cuh:176-212
// (the same chain without LayerNorm).  The oracle semantics are those of
// common/mlps.py:3-20 (MgnMlp), computed here with fp32 accumulation.
//
// MI355X design (one workgroup of 4 waves per CU, persistent over 64-row tiles):
//  * Weights live in VGPRs for the whole kernel.  Wave w owns output features
//    [32w, 32w+32) of every layer and keeps W1[:,32w:32w+32] (K/16 fragments),
//    W2 and W3 slices (8 fragments each) as MFMA A operands (W^T tiles).
//  * Each X tile (64 rows x K fp16) is streamed HBM->LDS with global_load_lds
//    (16 B per lane, whole 1 KiB wave transactions), double-buffered so the
//    next tile is in flight while this one is computed.  LDS chunks are
//    XOR-swizzled per row so the MFMA B-operand reads are bank-conflict free.
//  * The chain is computed transposed, Y^T = W^T X^T, with v_mfma_f32_32x32x16_f16.
//    Layer outputs (bias + ReLU + fp16 rounding fused in the epilogue) are
//    exchanged between the four waves through two small LDS tiles; they never
//    leave the CU.  Layer 3 keeps fp32 into the LayerNorm.
//  * LayerNorm is fused: each wave reduces its 32 features per row (in-lane +
//    one cross-half exchange), the four partial (mean, M2) pairs are combined
//    with Chan's parallel-variance formula through LDS.
//  * Output stores of tile t are issued at the start of the next tile, so the
//    wait for the next X tile never has to wait on fresh stores.
#include "gp_device.hpp"
#include "gp_kernels.hpp"

namespace gp {
namespace fused {

constexpr int TM = 64;          // rows per tile
constexpr int D = 128;          // hidden width of every MGN layer
constexpr int NWAVES = 4;
constexpr int NTHREADS = NWAVES * kWave;
constexpr int ACT_STRIDE = D * 2 + 16;  // padded LDS row (bytes) of a 128-wide fp16 tile
constexpr int SLAB_STRIDE = 64 * 2 + 16; // padded LDS row (bytes) of a transposed 64-k weight slab
constexpr int ACT_BYTES = (TM * ACT_STRIDE > D * SLAB_STRIDE) ? TM * ACT_STRIDE : D * SLAB_STRIDE;

template <int K>
struct Cfg {
  static_assert(K % 128 == 0 && K >= 128 && K <= 384, "K must be 128, 256 or 384");
  static constexpr int KS1 = K / 16;                 // MFMA k-steps of layer 1
  static constexpr int CPR = K / 8;                  // 16-byte chunks per X row
  static constexpr int XTILE = TM * K * 2;           // bytes per X tile
  static constexpr int DMA_INSTR = XTILE / 1024;     // wave-wide 1 KiB copies per tile
  static constexpr int DMA_PER_WAVE = DMA_INSTR / NWAVES;
  static_assert(DMA_INSTR % NWAVES == 0, "tile must split evenly over waves");
};

struct Params {
  const half_t* x;
  const half_t* w1;
  const half_t* b1;
  const half_t* w2;
  const half_t* b2;
  const half_t* w3;
  const half_t* b3;
  const half_t* gamma;
  const half_t* beta;
  half_t* out;
  int64_t M;
  float eps;
};

// Issue this wave's share of the copy of X tile `tile` into an LDS buffer.
// LDS chunk slot q = 64*i + lane holds row r = q / CPR, physical chunk p = q % CPR,
// which is logical chunk c = p ^ (r & 15) of that row.  Rows past M are clamped
// to the last row so every copy stays in bounds (their results are never stored).
template <int K>
__device__ __forceinline__ void issue_x_tile(const half_t* __restrict__ x, int64_t M, int64_t tile,
                                             GP_LDS char* buf, int wave, int lane) {
  using C = Cfg<K>;
  const int64_t row0 = tile * TM;
#pragma unroll
  for (int ii = 0; ii < C::DMA_PER_WAVE; ++ii) {
    const int i = ii * NWAVES + wave;
    const int q = i * kWave + lane;
    const int r = q / C::CPR;
    const int p = q - r * C::CPR;
    const int c = p ^ (r & 15);
    int64_t grow = row0 + r;
    grow = grow < M ? grow : M - 1;
    dma16(x + grow * K + c * 8, buf + i * 1024);
  }
}

template <int K, bool LN>
__global__ __launch_bounds__(NTHREADS) __attribute__((amdgpu_waves_per_eu(1, 1)))
void mgn_fused_kernel(Params p) {
  using C = Cfg<K>;
  __shared__ __attribute__((aligned(1024))) char xs0[C::XTILE];
  __shared__ __attribute__((aligned(1024))) char xs1[C::XTILE];
  __shared__ __attribute__((aligned(16))) char act1[ACT_BYTES];
  __shared__ __attribute__((aligned(16))) char act2[ACT_BYTES];
  __shared__ __attribute__((aligned(16))) f2 lnpart[TM][NWAVES];
  __shared__ __attribute__((aligned(16))) float prm[5][D];  // b1, b2, b3, gamma, beta

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int lr = lane & 31;   // row (B column / C column) within a 32-row block
  const int lh = lane >> 5;   // which half of the k-chunk / feature quad

  const int64_t M = p.M;
  const int64_t ntiles = (M + TM - 1) / TM;
  const int64_t G = gridDim.x;
  int64_t t = blockIdx.x;
  if (t >= ntiles) return;

  // Start streaming the first two tiles before anything else.
  issue_x_tile<K>(p.x, M, t, (GP_LDS char*)xs0, wave, lane);
  if (t + G < ntiles) issue_x_tile<K>(p.x, M, t + G, (GP_LDS char*)xs1, wave, lane);

  // Bias / LayerNorm parameters -> LDS (fp32).
  if (tid < D) {
    prm[0][tid] = (float)p.b1[tid];
    prm[1][tid] = (float)p.b2[tid];
    prm[2][tid] = (float)p.b3[tid];
    if (LN) {
      prm[3][tid] = (float)p.gamma[tid];
      prm[4][tid] = (float)p.beta[tid];
    }
  }

  // Weight fragments: A operand = W^T, lane holds W[k0 + 8*lh + e][32*wave + lr].
  // W is row-major [K][128]; 64-k slabs are transposed through LDS (the two
  // activation tiles, double-buffered) so every fragment is one 16-byte read.
  const int fcol = 32 * wave + lr;
  h8 w1f[C::KS1];
  h8 w2f[D / 16];
  h8 w3f[D / 16];
  {
    constexpr int NS1 = K / 64;
    constexpr int NS = NS1 + 4;  // W1 slabs, then two for W2, two for W3
    auto slab_src = [&](int j) -> const half_t* {
      return j < NS1 ? p.w1 + (64 * j) * D : (j < NS1 + 2 ? p.w2 + 64 * (j - NS1) * D : p.w3 + 64 * (j - NS1 - 2) * D);
    };
    h8 va[4], vb[4];
    auto load_slab = [&](int j, h8(&v)[4]) {
      const half_t* W = slab_src(j);
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = *(const h8*)(W + lane * D + 8 * (wave + 4 * i));
    };
    auto put_slab = [&](GP_LDS char* buf, const h8(&v)[4]) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int e = 0; e < 8; ++e)
          *(GP_LDS half_t*)(buf + (8 * (wave + 4 * i) + e) * SLAB_STRIDE + lane * 2) = v[i][e];
    };
    load_slab(0, va);
#pragma unroll
    for (int j = 0; j < NS; ++j) {
      GP_LDS char* buf = (j & 1) ? (GP_LDS char*)act2 : (GP_LDS char*)act1;
      if (j + 1 < NS) load_slab(j + 1, (j & 1) ? va : vb);
      put_slab(buf, (j & 1) ? vb : va);
      lds_barrier();
#pragma unroll
      for (int sl = 0; sl < 4; ++sl) {
        const h8 f = *(const GP_LDS h8*)(buf + fcol * SLAB_STRIDE + (16 * sl + 8 * lh) * 2);
        if (j < NS1) w1f[4 * j + sl] = f;
        else if (j < NS1 + 2) w2f[4 * (j - NS1) + sl] = f;
        else w3f[4 * (j - NS1 - 2) + sl] = f;
      }
    }
    // the activation tiles are reused below: every wave must be done reading
    lds_barrier();
  }

  // Per-lane LDS addressing.
  const int xr = lr & 15;
  const int xa = lh ^ xr;                 // chunk (2s+lh) lands at (2s ^ xa) within its 16-group
  const int xrow = lr * (K * 2);          // byte offset of this lane's row in block 0
  const int arow = lr * ACT_STRIDE;
  // features of accumulator group g: 32*wave + 8*g + 4*lh + (0..3)
  const int fq = 32 * wave + 4 * lh;

  // Deferred output of the previous tile (stored at the top of the next one).
  h4 pend[2][4];
  int64_t pend_row0 = -1;

  auto store_pending = [&]() {
    if (pend_row0 < 0) return;
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
      const int64_t row = pend_row0 + 32 * rb + lr;
      if (row < M) {
        half_t* o = p.out + row * D + fq;
#pragma unroll
        for (int g = 0; g < 4; ++g) *(h4*)(o + 8 * g) = pend[rb][g];
      }
    }
  };

  auto process = [&](GP_LDS char* xs, int64_t tile, bool next_inflight, bool issue_next, int64_t next_tile) {
    // 1. this tile's X has landed (only the following tile's copies may remain).
    if (next_inflight) wait_vmcnt<C::DMA_PER_WAVE>();
    else wait_vmcnt<0>();
    lds_barrier();
    store_pending();

    // 2. layer 1: acc[rb] = W1^T X^T over K.
    f16x acc0 = {}, acc1 = {};
#pragma unroll
    for (int s = 0; s < C::KS1; ++s) {
      const int off = ((2 * s) & ~15) * 16 + (((2 * s) ^ xa) & 15) * 16;
      const h8 b0 = *(const GP_LDS h8*)(xs + xrow + off);
      const h8 b1 = *(const GP_LDS h8*)(xs + xrow + 32 * K * 2 + off);
      acc0 = mfma32(w1f[s], b0, acc0);
      acc1 = mfma32(w1f[s], b1, acc1);
    }
    // epilogue 1: + b1, ReLU, fp16 -> act1[row][feature]
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const f4 bias = *(const f4*)&prm[0][fq + 8 * g];
      h4 o0, o1;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        o0[e] = (half_t)relu(acc0[4 * g + e] + bias[e]);
        o1[e] = (half_t)relu(acc1[4 * g + e] + bias[e]);
      }
      *(GP_LDS h4*)((GP_LDS char*)act1 + arow + (fq + 8 * g) * 2) = o0;
      *(GP_LDS h4*)((GP_LDS char*)act1 + arow + 32 * ACT_STRIDE + (fq + 8 * g) * 2) = o1;
    }
    lds_barrier();
    // The X buffer is free again: start the copy of the tile two steps ahead.
    if (issue_next) issue_x_tile<K>(p.x, M, next_tile, xs, wave, lane);

    // 3. layer 2
    acc0 = f16x{};
    acc1 = f16x{};
#pragma unroll
    for (int s = 0; s < D / 16; ++s) {
      const int off = (2 * s + lh) * 16;
      const h8 b0 = *(const GP_LDS h8*)((GP_LDS char*)act1 + arow + off);
      const h8 b1 = *(const GP_LDS h8*)((GP_LDS char*)act1 + arow + 32 * ACT_STRIDE + off);
      acc0 = mfma32(w2f[s], b0, acc0);
      acc1 = mfma32(w2f[s], b1, acc1);
    }
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const f4 bias = *(const f4*)&prm[1][fq + 8 * g];
      h4 o0, o1;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        o0[e] = (half_t)relu(acc0[4 * g + e] + bias[e]);
        o1[e] = (half_t)relu(acc1[4 * g + e] + bias[e]);
      }
      *(GP_LDS h4*)((GP_LDS char*)act2 + arow + (fq + 8 * g) * 2) = o0;
      *(GP_LDS h4*)((GP_LDS char*)act2 + arow + 32 * ACT_STRIDE + (fq + 8 * g) * 2) = o1;
    }
    lds_barrier();

    // 4. layer 3 (+ bias), fp32 kept for the LayerNorm
    acc0 = f16x{};
    acc1 = f16x{};
#pragma unroll
    for (int s = 0; s < D / 16; ++s) {
      const int off = (2 * s + lh) * 16;
      const h8 b0 = *(const GP_LDS h8*)((GP_LDS char*)act2 + arow + off);
      const h8 b1 = *(const GP_LDS h8*)((GP_LDS char*)act2 + arow + 32 * ACT_STRIDE + off);
      acc0 = mfma32(w3f[s], b0, acc0);
      acc1 = mfma32(w3f[s], b1, acc1);
    }
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const f4 bias = *(const f4*)&prm[2][fq + 8 * g];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        acc0[4 * g + e] += bias[e];
        acc1[4 * g + e] += bias[e];
      }
    }

    if constexpr (LN) {
      // Per-wave statistics over this wave's 32 features of each row.
      float s0 = 0.f, s1 = 0.f;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        s0 += acc0[v];
        s1 += acc1[v];
      }
      s0 += xor_lane32(s0);
      s1 += xor_lane32(s1);
      const float m0 = s0 * (1.f / 32.f), m1 = s1 * (1.f / 32.f);
      float q0 = 0.f, q1 = 0.f;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const float d0 = acc0[v] - m0, d1 = acc1[v] - m1;
        q0 += d0 * d0;
        q1 += d1 * d1;
      }
      q0 += xor_lane32(q0);
      q1 += xor_lane32(q1);
      if (lh == 0) {
        lnpart[lr][wave] = f2{m0, q0};
        lnpart[32 + lr][wave] = f2{m1, q1};
      }
      lds_barrier();
      // Combine the four (mean, M2) partials of each row (Chan et al.).
      float mean[2], rstd[2];
#pragma unroll
      for (int rb = 0; rb < 2; ++rb) {
        const f4 pa = *(const f4*)&lnpart[32 * rb + lr][0];
        const f4 pb = *(const f4*)&lnpart[32 * rb + lr][2];
        const float mu = 0.25f * ((pa[0] + pa[2]) + (pb[0] + pb[2]));
        const float da = pa[0] - mu, db = pa[2] - mu, dc = pb[0] - mu, dd = pb[2] - mu;
        const float m2 = (pa[1] + pa[3]) + (pb[1] + pb[3]) + 32.f * (da * da + db * db + dc * dc + dd * dd);
        const float var = m2 * (1.f / D);
        mean[rb] = mu;
        rstd[rb] = 1.f / sqrtf(var + p.eps);
      }
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const f4 gm = *(const f4*)&prm[3][fq + 8 * g];
        const f4 bt = *(const f4*)&prm[4][fq + 8 * g];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          pend[0][g][e] = (half_t)((acc0[4 * g + e] - mean[0]) * rstd[0] * gm[e] + bt[e]);
          pend[1][g][e] = (half_t)((acc1[4 * g + e] - mean[1]) * rstd[1] * gm[e] + bt[e]);
        }
      }
    } else {
#pragma unroll
      for (int g = 0; g < 4; ++g)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          pend[0][g][e] = (half_t)acc0[4 * g + e];
          pend[1][g][e] = (half_t)acc1[4 * g + e];
        }
    }
    pend_row0 = tile * TM;
  };

  // Tiles alternate between the two X buffers; the loop is unrolled by two so
  // each buffer is a distinct LDS object at every access.
  for (;;) {
    {
      const bool inflight = t + G < ntiles;
      const bool issue = t + 2 * G < ntiles;
      process((GP_LDS char*)xs0, t, inflight, issue, t + 2 * G);
    }
    t += G;
    if (t >= ntiles) break;
    {
      const bool inflight = t + G < ntiles;
      const bool issue = t + 2 * G < ntiles;
      process((GP_LDS char*)xs1, t, inflight, issue, t + 2 * G);
    }
    t += G;
    if (t >= ntiles) break;
  }
  store_pending();
}

}  // namespace fused

// ---------------------------------------------------------------------------
// Host launcher
// ---------------------------------------------------------------------------
template <int K, bool LN>
static hipError_t launch_fused(const MgnArgs& a, int grid, hipStream_t stream) {
  fused::Params p{(const half_t*)a.x,  (const half_t*)a.w1, (const half_t*)a.b1, (const half_t*)a.w2,
                  (const half_t*)a.b2, (const half_t*)a.w3, (const half_t*)a.b3, (const half_t*)a.gamma,
                  (const half_t*)a.beta, (half_t*)a.out, a.M, a.eps};
  hipLaunchKernelGGL((fused::mgn_fused_kernel<K, LN>), dim3(grid), dim3(fused::NTHREADS), 0, stream, p);
  return hipGetLastError();
}

hipError_t mgn_fused_launch(const MgnArgs& a, int num_cus, hipStream_t stream) {
  const int64_t ntiles = (a.M + fused::TM - 1) / fused::TM;
  const int grid = (int)(ntiles < num_cus ? ntiles : num_cus);
  const bool ln = a.gamma != nullptr;
  switch (a.K) {
    case 384: return ln ? launch_fused<384, true>(a, grid, stream) : launch_fused<384, false>(a, grid, stream);
    case 256: return ln ? launch_fused<256, true>(a, grid, stream) : launch_fused<256, false>(a, grid, stream);
    case 128: return ln ? launch_fused<128, true>(a, grid, stream) : launch_fused<128, false>(a, grid, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace gp
