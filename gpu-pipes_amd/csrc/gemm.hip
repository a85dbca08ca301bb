// Wide fp16 GEMM stage with fused epilogues for gfx950:
//
//   C[M][N] = act(A[M][K] . B[K][N] + bias[N]) (+ R[M][N])      fp32 accumulate
//
// This is the stage the reference composes its BERT FFN from: GEMM blocks
// split along N (and K, through an accumulator queue) with a bias + ReLU
// epilogue, and the residual brought in as the accumulator of the second
// GEMM (apps/bert_ffn/pipelined/bert_ffn_pl.cuh:79-116,
// common/pipe_gemm.cuh:128-146).  At BERT-large width (H = 1024, ff = 4096)
// the weights (16 MB) cannot stay resident on chip, so on MI355X each GEMM is
// one streaming kernel over 256 x 256 output tiles with its epilogue fused.
//
// Kernel design.  B is consumed transposed (Bt[N][K], from transpose_kernel),
// so both MFMA operands are rows of consecutive k.  The product is computed
// transposed, C^T = Bt A^T, with v_mfma_f32_32x32x16_f16: the MFMA A operand
// is a 32-feature block of Bt, the MFMA B operand a 32-row block of A, and
// each accumulator lane ends up holding 4 consecutive features of one row
// (8-byte stores).  A workgroup of four waves -- one per SIMD, so the 256
// accumulator registers of a wave fit beside its operand fragments --
// computes a BN x BM tile; wave (wn, wm) owns 32 NBW features and 32 MBW
// rows.  K advances in 32-wide slabs, each slab holding the tile's BM rows of
// A and BN rows of Bt (64 bytes per row, 16-byte chunks XOR-swizzled by row so
// that 16 consecutive rows read at one chunk hit 16 distinct bank groups).
// Slabs are copied HBM->LDS with buffer_load ... lds into a ring of four, so
// the copies of three slabs are in flight while one is multiplied; operand
// fragments are double-buffered in registers, and the one LDS barrier per
// slab sits between the two 16-k steps, where it overlaps running MFMAs.
#include <hip/hip_runtime.h>

#include <type_traits>

#include "../../include/gpipes.h"
#include "gp_device.hpp"
#include "gp_kernels.hpp"
#include "stages.hpp"

namespace gp {
namespace gemm {

constexpr int BK = 32;     // k per slab
constexpr int ROWB = 64;   // bytes per slab row (BK fp16)
constexpr int NBUF = 4;    // slab ring depth
constexpr int NW = 4;      // waves per workgroup
constexpr int NT = NW * kWave;

template <int NBW_, int MBW_, int WN_>
struct Cfg {
  static constexpr int NBW = NBW_, MBW = MBW_, WN = WN_, WM = NW / WN_;
  static constexpr int BN = 32 * NBW * WN;         // features per tile
  static constexpr int BM = 32 * MBW * WM;         // rows per tile
  static constexpr int ROWS = BM + BN;             // slab rows: A rows, then Bt rows
  static constexpr int SLAB = ROWS * ROWB;         // bytes per slab
  static constexpr int NCOPY = ROWS / 16;          // 1 KiB copies per slab (16 rows each)
  static constexpr int DPW = NCOPY / NW;           // copies per wave per slab
  static constexpr int MFMAS = 2 * NBW * MBW;      // MFMAs per wave per slab
  static_assert(NCOPY % NW == 0 && (BM / 16) % NW == 0, "copy split must be uniform per wave");
  static_assert(NBUF * SLAB <= 160 * 1024, "LDS");
};
using Wide = Cfg<4, 4, 2>;    // 256 features x 256 rows
using Narrow = Cfg<4, 2, 1>;  // 128 features x 256 rows (N = 128)

struct Args {
  const half_t* a;     // [M][K]
  const half_t* bt;    // [N][K]
  const half_t* bias;  // [N] or null
  const half_t* r;     // [M][N] residual or null
  half_t* c;           // [M][N]
  int64_t M;
  int N;
  int K;
};

// Byte offset of logical 16-byte chunk c (0..3) of slab row r.
__device__ __forceinline__ int slab_off(int r, int c) { return r * ROWB + ((c ^ ((r >> 2) & 3)) << 4); }

template <class C, int ACT, bool RESID>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(1, 1))) void gemm_kernel(Args p) {
  __shared__ __attribute__((aligned(1024))) char ring[NBUF * C::SLAB];
  __shared__ __attribute__((aligned(1024))) char bias_lds[2][1024];  // bias of a tile, by tile parity

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int lr = lane & 31, lh = lane >> 5;
  const int wn = wave % C::WN, wm = wave / C::WN;
  const int K = p.K;
  const int nslab = K / BK;
  const int npre = nslab < NBUF ? nslab : NBUF;  // slabs copied ahead of a tile's main loop

  // Persistent workers.  Workgroup b is taken to run on XCD b % 8 (the
  // dispatch order); the tiles are split into contiguous ranges, one per XCD,
  // and the workers of an XCD deal out their range, so the tiles that run at
  // the same time on one XCD share A and Bt panels in its L2.
  // Tile indices fit in 32 bits: the host limits M to 2^31 - 1 rows.
  const int tiles_n = p.N / C::BN;
  const int ntiles = (int)((p.M + C::BM - 1) / C::BM) * tiles_n;
  const int G = gridDim.x;
  const int NX = G < 8 ? G : 8;
  const int xcd = blockIdx.x % NX, wid = blockIdx.x / NX;
  const int nwx = (G - xcd + NX - 1) / NX;
  const int hi = (int)((int64_t)ntiles * (xcd + 1) / NX);
  int t = (int)((int64_t)ntiles * xcd / NX) + wid;
  if (t >= hi) return;

  // Copies.  Copy q of a slab fills slab rows 16q .. 16q+15; lane l writes
  // row 16q + l/4 at chunk position l%4, i.e. logical chunk (l%4) ^ ((row>>2)&3).
  // Wave w issues copies q = j NW + w; since BM/16 is a multiple of NW, copies
  // j < BM/(16 NW) are rows of A, the rest rows of Bt.  Rows of A past M lie
  // outside the descriptor's range and read as zero.
  constexpr int JA = C::BM / 16 / NW;
  int voff[C::DPW];
#pragma unroll
  for (int j = 0; j < C::DPW; ++j) {
    const int row = 16 * (j * NW + wave) + (lane >> 2);  // slab row
    const int orow = j < JA ? row : row - C::BM;           // row of A or of Bt
    voff[j] = orow * K * 2 + (((lane & 3) ^ ((row >> 2) & 3)) << 4);
  }
  GP_LDS char* const lds = (GP_LDS char*)ring;

  struct Tile {
    int64_t m0;
    int n0, rows;
    __amdgpu_buffer_rsrc_t ra, rb;
  };
  auto tile_at = [&](int tt) {
    Tile T;
    const int tm = tt / tiles_n;
    T.n0 = (tt - tm * tiles_n) * C::BN;
    T.m0 = (int64_t)tm * C::BM;
    const int64_t mrows = p.M - T.m0;
    T.rows = (int)(mrows < C::BM ? mrows : C::BM);
    T.ra = make_rsrc(p.a + T.m0 * K, T.rows * K * 2);
    T.rb = make_rsrc(p.bt + (int64_t)T.n0 * K, C::BN * K * 2);
    return T;
  };
  auto issue = [&](const Tile& T, int kt) {
    GP_LDS char* const s = lds + (kt % NBUF) * C::SLAB;
#pragma unroll
    for (int j = 0; j < C::DPW; ++j)
      dma16_buf(j < JA ? T.ra : T.rb, voff[j] + kt * ROWB, s + (j * NW + wave) * 1024);  // panels are re-read from L2
  };
  // A tile's copies ahead of its main loop: its bias (every wave copies the
  // same 1 KiB, which keeps the per-wave copy counts uniform; a null bias is a
  // zero-length range and reads as zeros), then slabs 0 .. npre-1.
  auto prefetch = [&](const Tile& T, int par) {
    dma16_buf(make_rsrc(p.bias ? p.bias + T.n0 : p.bias, p.bias ? C::BN * 2 : 0), lane * 16,
              (GP_LDS char*)bias_lds[par]);
    for (int kt = 0; kt < npre; ++kt) issue(T, kt);
  };

  // Operand fragments of one 16-k step: NBW of Bt, MBW of A.
  struct Frags {
    h8 a[C::NBW], b[C::MBW];
  };
  const int frow = C::BM + 32 * C::NBW * wn + lr;  // slab row of Bt fragment nb: frow + 32 nb
  const int arow = 32 * C::MBW * wm + lr;          // slab row of A fragment mb: arow + 32 mb
  auto load = [&](Frags& f, int kt, int ks) {
    GP_LDS const char* const s = lds + (kt % NBUF) * C::SLAB;
#pragma unroll
    for (int nb = 0; nb < C::NBW; ++nb) f.a[nb] = *(GP_LDS const h8*)(s + slab_off(frow + 32 * nb, 2 * ks + lh));
#pragma unroll
    for (int mb = 0; mb < C::MBW; ++mb) f.b[mb] = *(GP_LDS const h8*)(s + slab_off(arow + 32 * mb, 2 * ks + lh));
  };
  f16x acc[C::NBW][C::MBW];
  // MFMAs of one step; the NFR fragment reads issued just before are spread
  // over the first MFMAs so that their latency hides behind the matrix pipe.
  auto mma = [&](const Frags& f, auto nfr_c) {
    constexpr int nfr = decltype(nfr_c)::value;
#pragma unroll
    for (int nb = 0; nb < C::NBW; ++nb)
#pragma unroll
      for (int mb = 0; mb < C::MBW; ++mb) acc[nb][mb] = mfma32(f.a[nb], f.b[mb], acc[nb][mb]);
#pragma unroll
    for (int i = 0; i < nfr; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, C::NBW * C::MBW - nfr, 0);
  };
  // Waits until slab kt's copies (this wave's) have landed, given how many
  // later slabs of the tile have copies in flight.
  auto wait_slab = [&](int kt) {
    const int later = nslab - 1 - kt;
    if (later >= NBUF - 2)
      wait_vmcnt<(NBUF - 2) * C::DPW>();
    else if (later == 1)
      wait_vmcnt<C::DPW>();
    else
      wait_vmcnt<0>();
  };
  static_assert(NBUF == 4, "wait_slab covers up to two later slabs in flight");
  // Memory operations of one epilogue: a store (and a residual load) per
  // fragment and element group.
  constexpr int EPI_OPS = C::NBW * 4 * C::MBW * (RESID ? 2 : 1);
  // Waits until a tile's bias and slab 0 have landed.  Issued after them:
  // the tile's other npre-1 slabs and, from the second tile on, the previous
  // tile's epilogue.  The counter field holds at most 63, which still implies
  // slab 0 whenever more than 63 operations followed it.
  auto wait_first = [&](bool after_epi) {
    const int g = npre - 1;
    if (after_epi) {
      if constexpr (EPI_OPS >= 63) {
        wait_vmcnt<63>();
      } else {
        if (g >= 3) wait_vmcnt<(3 * C::DPW + EPI_OPS > 63 ? 63 : 3 * C::DPW + EPI_OPS)>();
        else if (g == 2) wait_vmcnt<(2 * C::DPW + EPI_OPS > 63 ? 63 : 2 * C::DPW + EPI_OPS)>();
        else if (g == 1) wait_vmcnt<(C::DPW + EPI_OPS > 63 ? 63 : C::DPW + EPI_OPS)>();
        else wait_vmcnt<EPI_OPS>();
      }
    } else {
      if (g >= 3) wait_vmcnt<3 * C::DPW>();
      else if (g == 2) wait_vmcnt<2 * C::DPW>();
      else if (g == 1) wait_vmcnt<C::DPW>();
      else wait_vmcnt<0>();
    }
  };
  static_assert(3 * C::DPW <= 63, "slab copies in flight exceed the counter field");

  constexpr int NFR = C::NBW + C::MBW;  // fragment reads per step
  static_assert(NFR <= C::NBW * C::MBW, "reads are spread one per MFMA");
  Tile T = tile_at(t);
  int par = 0;
  prefetch(T, par);
#pragma unroll
  for (int nb = 0; nb < C::NBW; ++nb)
#pragma unroll
    for (int mb = 0; mb < C::MBW; ++mb) acc[nb][mb] = f16x{};
  wait_first(false);
  for (;;) {
    // Main loop.  Iteration kt holds step 0 of slab kt in registers (f0):
    //   read step 1 of slab kt (f1)          | MFMAs of f0
    //   wait for slab kt+1, barrier          | (MFMAs of f0 still running)
    //   refill slab kt's buffer with kt+4, read step 0 of slab kt+1 (f0) | MFMAs of f1
    // The barrier certifies that every wave's copies of slab kt+1 landed and
    // that every wave has read slab kt into registers, so its buffer is free.
    Frags f0, f1;
    lds_barrier();
    load(f0, 0, 0);
    for (int kt = 0; kt + 1 < nslab; ++kt) {
      load(f1, kt, 1);
      mma(f0, std::integral_constant<int, NFR>{});
      wait_slab(kt + 1);
      lds_barrier();
      if (kt + NBUF < nslab) issue(T, kt + NBUF);
      load(f0, kt + 1, 0);
      mma(f1, std::integral_constant<int, NFR>{});
    }
    load(f1, nslab - 1, 1);
    mma(f0, std::integral_constant<int, NFR>{});
    mma(f1, std::integral_constant<int, 0>{});

    // The next tile's copies go out before this tile's epilogue, once every
    // wave has read the last slab (the barrier), so their latency hides
    // behind it.
    const int tnext = t + nwx;
    const bool more = tnext < hi;
    Tile Nx;
    if (more) {
      Nx = tile_at(tnext);
      lds_barrier();
      prefetch(Nx, par ^ 1);
    }

    // Epilogue.  For fragment (nb, mb) the lane holds row arow + 32 mb of the
    // tile and, in elements 4g .. 4g+3, features
    // n0 + 32 NBW wn + 32 nb + 8 g + 4 lh + (0..3).  Output and residual go
    // through buffer descriptors limited to the tile's valid rows, so a
    // partial tile needs no per-row branch; the residual loads of one nb are
    // all issued before the first is used.
    const __amdgpu_buffer_rsrc_t rc = make_rsrc(p.c + T.m0 * p.N, T.rows * p.N * 2);
    const __amdgpu_buffer_rsrc_t rr = make_rsrc(RESID ? p.r + T.m0 * p.N : p.c, RESID ? T.rows * p.N * 2 : 0);
    // Per-row byte offsets, computed here (opaque: not hoisted out of the tile
    // loop as 64 live registers); the nb / g part is an instruction offset.
    int ebase[C::MBW];
#pragma unroll
    for (int mb = 0; mb < C::MBW; ++mb) ebase[mb] = opaque(((arow + 32 * mb) * p.N + T.n0 + 32 * C::NBW * wn + 4 * lh) * 2);
    auto eoff = [&](int nb, int g, int mb) { return ebase[mb] + (32 * nb + 8 * g) * 2; };
#pragma unroll
    for (int nb = 0; nb < C::NBW; ++nb) {
      h4 res[4][C::MBW];
      if constexpr (RESID) {
#pragma unroll
        for (int g = 0; g < 4; ++g)
#pragma unroll
          for (int mb = 0; mb < C::MBW; ++mb) res[g][mb] = buf_load_h4(rr, eoff(nb, g, mb));
      }
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const h4 bv = *(GP_LDS const h4*)(bias_lds[par] + (32 * C::NBW * wn + 32 * nb + 8 * g + 4 * lh) * 2);
#pragma unroll
        for (int mb = 0; mb < C::MBW; ++mb) {
          f4 v;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            v[e] = apply_act(acc[nb][mb][4 * g + e] + (float)bv[e], ACT);
            if constexpr (RESID) v[e] += (float)res[g][mb][e];
          }
          buf_store_h4(rc, eoff(nb, g, mb), __builtin_convertvector(v, h4));
        }
      }
#pragma unroll
      for (int mb = 0; mb < C::MBW; ++mb) acc[nb][mb] = f16x{};  // ready for the next tile
    }
    if (!more) break;
    wait_first(true);
    t = tnext;
    T = Nx;
    par ^= 1;
  }
}

// out[N][K] = in[K][N] (fp16), 64 x 64 tiles through LDS; K and N multiples of 64.
__global__ __launch_bounds__(256) void transpose_kernel(const half_t* in, half_t* out, int K, int N) {
  __shared__ half_t tile[64][66];
  const int k0 = blockIdx.y * 64, n0 = blockIdx.x * 64;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  for (int r = ty; r < 64; r += 4) tile[r][tx] = in[(int64_t)(k0 + r) * N + n0 + tx];
  __syncthreads();
  for (int r = ty; r < 64; r += 4) out[(int64_t)(n0 + r) * K + k0 + tx] = tile[tx][r];
}

template <class C, int ACT, bool RESID>
static hipError_t launch(const Args& a, int num_cus, hipStream_t s) {
  const int64_t tiles = ((a.M + C::BM - 1) / C::BM) * (a.N / C::BN);
  const int64_t grid = tiles < num_cus ? tiles : num_cus;  // one persistent workgroup per CU
  hipLaunchKernelGGL((gemm_kernel<C, ACT, RESID>), dim3((unsigned)grid), dim3(NT), 0, s, a);
  return hipGetLastError();
}

template <class C>
static hipError_t dispatch(const Args& g, int act, int ncu, hipStream_t s) {
  if (g.r) return act == ACT_NONE ? launch<C, ACT_NONE, true>(g, ncu, s) : hipErrorInvalidValue;
  switch (act) {
    case ACT_NONE: return launch<C, ACT_NONE, false>(g, ncu, s);
    case ACT_RELU: return launch<C, ACT_RELU, false>(g, ncu, s);
    case ACT_GELU_TANH: return launch<C, ACT_GELU_TANH, false>(g, ncu, s);
    case ACT_SIGMOID: return launch<C, ACT_SIGMOID, false>(g, ncu, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace gemm

hipError_t gemm_launch(const GemmArgs& a, int num_cus, hipStream_t s) {
  using namespace gemm;
  if (a.M <= 0) return hipSuccess;
  const Args g{(const half_t*)a.x, (const half_t*)a.wt, (const half_t*)a.b, (const half_t*)a.r, (half_t*)a.out,
               a.M, (int)a.N, (int)a.K};
  if (a.N % Wide::BN == 0) return dispatch<Wide>(g, a.act, num_cus, s);
  return dispatch<Narrow>(g, a.act, num_cus, s);
}

hipError_t transpose_launch(const void* in, void* out, int64_t K, int64_t N, hipStream_t s) {
  hipLaunchKernelGGL(gemm::transpose_kernel, dim3((unsigned)(N / 64), (unsigned)(K / 64)), dim3(256), 0, s,
                     (const half_t*)in, (half_t*)out, (int)K, (int)N);
  return hipGetLastError();
}

}  // namespace gp
