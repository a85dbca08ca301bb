// Fused MeshGraphNet MLP for gfx950: Linear(K->128)+ReLU, Linear(128->128)+ReLU,
// Linear(128->128) [, LayerNorm(128)] in one persistent kernel.
//
// Reference behaviour: apps/mgn_fullmlp/pipelined/mgn_fullmlp_pl.cuh:83-252
// (three GEMM stage blocks + five LayerNorm blocks per pipeline row, chained by
// global-memory queues) and apps/mgn_linears/pipelined/mgn_linears_pl.cuh:176-212
// (the same chain without LayerNorm).  The oracle semantics are those of
// common/mlps.py:3-20 (MgnMlp), computed here with fp32 accumulation.
//
// MI355X design (one workgroup of 8 waves per CU, persistent over 64-row tiles):
//  * Wave w owns output features [32n, 32n+32) (n = w % 4) of every layer for
//    the 32-row block m = w / 4 of each tile, so each SIMD runs two waves with
//    the same weights: while one waits on LDS, the other issues MFMAs.
//  * Weights stay resident for the whole kernel in AGPRs (MFMA takes its A
//    operand from AGPRs on gfx950): W1[:,32n:32n+32] as K/16 fragments plus the
//    W2 and W3 slices (8 fragments each) -- 160 registers per wave.
//  * Each X tile (64 rows x K fp16) is streamed HBM->LDS with global_load_lds
//    (16 B per lane, whole 1 KiB wave transactions), double-buffered so the
//    next tile is in flight while this one is computed.  LDS chunks are
//    XOR-swizzled per row so the MFMA B-operand reads are bank-conflict free.
//  * The chain is computed transposed, Y^T = W^T X^T, with
//    v_mfma_f32_32x32x16_f16; the bias is the accumulator's initial value.
//    Layer outputs (ReLU + fp16 rounding in the epilogue) are exchanged between
//    the four feature slices through two small LDS tiles; they never leave the
//    CU.  Layer 3 stays fp32 into the LayerNorm.
//  * LayerNorm is fused: each wave reduces its 32 features per row (in-lane +
//    one cross-half exchange), and the four partial (mean, M2) pairs of a row
//    are combined with Chan's parallel-variance formula through LDS.
//  * The finished output tile is staged in LDS and written out as whole rows at
//    the start of the next tile, so the wait for the next X tile never waits on
//    fresh stores.
#include "gp_device.hpp"
#include "gp_kernels.hpp"

namespace gp {
namespace fused {

constexpr int TM = 64;          // rows per tile (two 32-row MFMA blocks)
constexpr int D = 128;          // hidden width of every MGN layer
constexpr int NWAVES = 8;       // 4 feature slices x 2 row blocks
constexpr int NTHREADS = NWAVES * kWave;
constexpr int ACT_STRIDE = D * 2 + 16;   // padded LDS row (bytes) of a 128-wide fp16 tile
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
// which is logical chunk c = p ^ (r & 15) of that row.  The copy goes through a
// buffer descriptor whose base is the tile and whose size ends at row M, so
// rows past M are zero-filled by the hardware range check (their results are
// never stored) and every per-lane offset is a 32-bit value.
template <int K>
__device__ __forceinline__ void issue_x_tile(const half_t* __restrict__ x, int64_t M, int64_t tile,
                                             GP_LDS char* buf, int wave, int lane) {
  using C = Cfg<K>;
  const int64_t row0 = tile * TM;
  const int64_t left = (M - row0) * (K * 2);
  const int nbytes = left < C::XTILE ? (int)left : C::XTILE;
  const __amdgpu_buffer_rsrc_t rsrc = make_rsrc(x + row0 * K, nbytes);
#pragma unroll
  for (int ii = 0; ii < C::DMA_PER_WAVE; ++ii) {
    const int i = ii * NWAVES + wave;
    const int q = i * kWave + lane;
    const int r = q / C::CPR;
    const int p = q - r * C::CPR;
    const int c = p ^ (r & 15);
    dma16_buf(rsrc, (r * K + c * 8) * 2, buf + i * 1024);
  }
}

// Accumulator initialised with the bias: C element 4g+e of a lane holds the
// bias of feature fq + 8g + e (every row of the block shares it).
__device__ __forceinline__ f16x bias_frag(const float* bias, int fq) {
  f16x c;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const f4 v = *(const f4*)&bias[fq + 8 * g];
#pragma unroll
    for (int e = 0; e < 4; ++e) c[4 * g + e] = v[e];
  }
  return c;
}

// One 32-row block: acc += W^T(fragments wf[0..KS)) * B, B fragments read from
// LDS through ld(s) two k-steps ahead of their MFMA.
template <int KS, typename LD>
__device__ __forceinline__ void gemm_blk(const h8* wf, LD ld, f16x& acc) {
  h8 q[2];
  q[0] = ld(0);
  q[1] = ld(1);
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    acc = mfma32(wf[s], q[s & 1], acc);
    if (s + 2 < KS) q[s & 1] = ld(s + 2);
  }
}

// ReLU + fp16 rounding of the accumulator into this lane's row of an LDS
// activation tile.  relu(round(x)) == round(relu(x)), so ReLU runs on the
// packed fp16 values.
__device__ __forceinline__ void store_relu_row(GP_LDS char* act_row, int fq, const f16x& a) {
  const h4 zero = {0, 0, 0, 0};
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const h4 o = __builtin_elementwise_max(
        __builtin_convertvector((f4){a[4 * g], a[4 * g + 1], a[4 * g + 2], a[4 * g + 3]}, h4), zero);
    *(GP_LDS h4*)(act_row + (fq + 8 * g) * 2) = o;
  }
}

template <int K, bool LN>
__global__ __launch_bounds__(NTHREADS) __attribute__((amdgpu_waves_per_eu(2, 2)))
void mgn_fused_kernel(Params p) {
  using C = Cfg<K>;
  __shared__ __attribute__((aligned(1024))) char xs0[C::XTILE];
  __shared__ __attribute__((aligned(1024))) char xs1[C::XTILE];
  __shared__ __attribute__((aligned(16))) char act1[ACT_BYTES];
  __shared__ __attribute__((aligned(16))) char act2[ACT_BYTES];
  __shared__ __attribute__((aligned(16))) char ostage[TM * ACT_STRIDE];  // finished output tile
  __shared__ __attribute__((aligned(16))) f2 lnpart[TM][4];
  __shared__ __attribute__((aligned(16))) float prm[5][D];  // b1, b2, b3, gamma, beta

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int lr = lane & 31;   // row within the 32-row block (B / C column)
  const int lh = lane >> 5;   // half of the k-chunk / feature quad
  const int n = wave & 3;     // feature slice
  const int m = wave >> 2;    // row block

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

  // Weight fragments: A operand = W^T, lane holds W[k0 + 8*lh + e][32*n + lr].
  // W is row-major [K][128]; 64-k slabs are transposed through LDS (the two
  // activation tiles, double-buffered) so every fragment is one 16-byte read.
  const int fcol = 32 * n + lr;
  h8 w1f[C::KS1];
  h8 w2f[D / 16];
  h8 w3f[D / 16];
  {
    constexpr int NS1 = K / 64;
    constexpr int NS = NS1 + 4;  // W1 slabs, then two for W2, two for W3
    auto slab_src = [&](int j) -> const half_t* {
      return j < NS1 ? p.w1 + (64 * j) * D : (j < NS1 + 2 ? p.w2 + 64 * (j - NS1) * D : p.w3 + 64 * (j - NS1 - 2) * D);
    };
    // 64 rows x 16 feature octets per slab: wave w copies octets w and w + 8.
    h8 va[2], vb[2];
    auto load_slab = [&](int j, h8(&v)[2]) {
      const half_t* W = slab_src(j);
#pragma unroll
      for (int i = 0; i < 2; ++i) v[i] = *(const h8*)(W + lane * D + 8 * (wave + 8 * i));
    };
    auto put_slab = [&](GP_LDS char* buf, const h8(&v)[2]) {
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int e = 0; e < 8; ++e)
          *(GP_LDS half_t*)(buf + (8 * (wave + 8 * i) + e) * SLAB_STRIDE + lane * 2) = v[i][e];
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
  // Register placement with two waves per SIMD (128 VGPRs + 128 AGPRs each):
  // W1 and W3 live in AGPRs (MFMA reads its A operand from AGPRs on gfx950),
  // W2, the accumulator and the LDS operand pipeline in VGPRs.
#pragma unroll
  for (int s = 0; s < C::KS1; ++s) asm volatile("" : "+a"(w1f[s]));
#pragma unroll
  for (int s = 0; s < D / 16; ++s) {
    asm volatile("" : "+v"(w2f[s]));
    asm volatile("" : "+a"(w3f[s]));
  }

  // Per-lane LDS addressing for this wave's row block.
  const int row = 32 * m + lr;                  // tile row covered by this lane's accumulator column
  const int xa = lh ^ (lr & 15);                // chunk (2s+lh) lands at (2s ^ xa) within its 16-group
  const int xrow = row * (K * 2);
  const int arow = row * ACT_STRIDE;
  const int fq = 32 * n + 4 * lh;               // features of accumulator group g: fq + 8g + (0..3)

  // The finished output tile waits in LDS and is stored at the top of the
  // next tile as whole 256-byte rows (thread t copies 16-byte chunks t, t+512).
  int64_t pend_tile = -1;
  auto store_pending = [&]() {
    if (pend_tile < 0) return;
    const int tid_l = opaque(tid);  // recompute the offsets per tile rather than keep them live
#pragma unroll
    for (int j = 0; j < (TM * D * 2 / 16) / NTHREADS; ++j) {
      const int c = tid_l + NTHREADS * j;
      const int r = c >> 4, col = (c & 15) * 8;
      const int64_t grow = pend_tile * TM + r;
      const h8 v = *(const GP_LDS h8*)((GP_LDS char*)ostage + r * ACT_STRIDE + col * 2);
      if (grow < M) *(h8*)(p.out + grow * D + col) = v;
    }
  };
  auto put_out = [&](int g, h4 v) { *(GP_LDS h4*)((GP_LDS char*)ostage + arow + (fq + 8 * g) * 2) = v; };

  auto process = [&](GP_LDS char* xs, int64_t tile, bool next_inflight, bool issue_next, int64_t next_tile) {
    // 1. this tile's X has landed (only the following tile's copies may remain).
    if (next_inflight) wait_vmcnt<C::DMA_PER_WAVE>();
    else wait_vmcnt<0>();
    lds_barrier();
    store_pending();

    // 2. layer 1: acc = b1 + W1^T X^T over K.
    f16x acc = bias_frag(prm[0], fq);
    gemm_blk<C::KS1>(w1f, [&](int s) {
      const int off = ((2 * s) & ~15) * 16 + (((2 * s) ^ xa) & 15) * 16;
      return *(const GP_LDS h8*)(xs + xrow + off);
    }, acc);
    store_relu_row((GP_LDS char*)act1 + arow, fq, acc);
    lds_barrier();
    // The X buffer is free again: start the copy of the tile two steps ahead.
    if (issue_next) issue_x_tile<K>(p.x, M, next_tile, xs, wave, opaque(lane));

    // 3. layer 2
    acc = bias_frag(prm[1], fq);
    gemm_blk<D / 16>(w2f, [&](int s) {
      return *(const GP_LDS h8*)((GP_LDS char*)act1 + arow + (2 * s + lh) * 16);
    }, acc);
    store_relu_row((GP_LDS char*)act2 + arow, fq, acc);
    lds_barrier();

    // 4. layer 3 (+ bias), fp32 kept for the LayerNorm
    acc = bias_frag(prm[2], fq);
    gemm_blk<D / 16>(w3f, [&](int s) {
      return *(const GP_LDS h8*)((GP_LDS char*)act2 + arow + (2 * s + lh) * 16);
    }, acc);

    if constexpr (LN) {
      // Statistics of this wave's 32 features of the row.
      float s0 = 0.f;
#pragma unroll
      for (int v = 0; v < 16; ++v) s0 += acc[v];
      s0 += xor_lane32(s0);
      const float m0 = s0 * (1.f / 32.f);
      float q0 = 0.f;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const float d0 = acc[v] - m0;
        q0 = __builtin_fmaf(d0, d0, q0);
      }
      q0 += xor_lane32(q0);
      if (lh == 0) lnpart[row][n] = f2{m0, q0};
      lds_barrier();
      // Combine the four (mean, M2) partials of the row (Chan et al.).
      const f4 pa = *(const f4*)&lnpart[row][0];
      const f4 pb = *(const f4*)&lnpart[row][2];
      const float mu = 0.25f * ((pa[0] + pa[2]) + (pb[0] + pb[2]));
      const float da = pa[0] - mu, db = pa[2] - mu, dc = pb[0] - mu, dd = pb[2] - mu;
      const float m2 = (pa[1] + pa[3]) + (pb[1] + pb[3]) + 32.f * (da * da + db * db + dc * dc + dd * dd);
      const float rstd = 1.f / sqrtf(m2 * (1.f / D) + p.eps);
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const f4 gm = *(const f4*)&prm[3][fq + 8 * g];
        const f4 bt = *(const f4*)&prm[4][fq + 8 * g];
        f4 y;
#pragma unroll
        for (int e = 0; e < 4; ++e) y[e] = __builtin_fmaf((acc[4 * g + e] - mu) * rstd, gm[e], bt[e]);
        put_out(g, __builtin_convertvector(y, h4));
      }
    } else {
#pragma unroll
      for (int g = 0; g < 4; ++g)
        put_out(g, __builtin_convertvector((f4){acc[4 * g], acc[4 * g + 1], acc[4 * g + 2], acc[4 * g + 3]}, h4));
    }
    pend_tile = tile;
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
  lds_barrier();
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
