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
// one streaming kernel over output tiles with its epilogue fused.
//
// Kernel design.
//  * B is consumed transposed (Bt[N][K], from prep_kernel),
//    so both MFMA operands are rows of consecutive k -- or, for calls small
//    enough that the transpose launch would cost more than it saves, in its
//    own [K][N] layout, its fragments read with the transposing LDS read
//    (the BROW kernels).  The product is computed transposed,
//    C^T = Bt A^T, with v_mfma_f32_32x32x16_f16: the MFMA A operand is a
//    32-feature block of Bt, the MFMA B operand a 32-row block of A, and each
//    accumulator lane ends up holding 4 consecutive features of one row.
//  * A workgroup of four waves -- one per SIMD, so the 256 accumulator
//    registers of a wave fit beside its operand fragments -- computes a
//    BN x BM tile (256 x 256, or 128 x 256 when N is an odd multiple of 128);
//    wave (wn, wm) owns 32 NBW features and 32 MBW rows.
//  * K advances in 64-wide slabs.  A slab is two LDS units -- the tile's BM
//    rows of A and its BN rows of Bt, 128 bytes per row, copied HBM->LDS with
//    buffer_load ... lds -- and units live in a ring of five (160 KiB), so
//    three units are in flight while a slab is multiplied.  128-byte row
//    segments are whole L2 lines: a copy instruction moves eight of them.
//    16-byte chunks are XOR-swizzled by row so that 16 consecutive rows read
//    at one chunk hit 16 distinct bank groups (conflict-free ds_read_b128).
//  * Operand fragments are double-buffered in registers across the four
//    16-k steps of a slab; the one LDS barrier per slab sits before the last
//    step, where it overlaps the running MFMAs, and releases the two units
//    of the slab for the copies of the slab two ahead.
//  * Workgroups are persistent (one per CU).  A tile's first units are copied
//    while the previous tile's epilogue runs.  The epilogue (bias, activation
//    or residual, fp16 rounding) stores through buffer descriptors limited to
//    the tile's valid rows, so partial tiles need no per-row branches.
#include <hip/hip_runtime.h>

#include <type_traits>
#include <utility>

#include "../../include/gpipes.h"
#include "gp_device.hpp"
#include "gp_kernels.hpp"
#include "stages.hpp"

namespace gp {
namespace gemm {

constexpr int BK = 64;              // k per slab
constexpr int ROWB = BK * 2;        // bytes per unit row (one 128-byte L2 line)
constexpr int CPR = ROWB / 16;      // 16-byte chunks per row
constexpr int RPC = 1024 / ROWB;    // rows per 1 KiB copy instruction
constexpr int KS = BK / 16;         // MFMA k-steps per slab
constexpr int NU = 5;               // units in the LDS ring
constexpr int NW = 4;               // waves per workgroup
constexpr int kLnPasses = 4;        // passes over the grid one LayerNorm-exchange launch may run
constexpr int NT = NW * kWave;
static_assert(KS % 2 == 0, "fragments alternate between two register sets per step");

template <int NBW_, int MBW_, int WN_>
struct Cfg {
  static constexpr int NBW = NBW_, MBW = MBW_, WN = WN_, WM = NW / WN_;
  static constexpr int BN = 32 * NBW * WN;                     // features per tile
  static constexpr int BM = 32 * MBW * WM;                     // rows per tile
  static constexpr int UNIT = (BM > BN ? BM : BN) * ROWB;      // bytes per ring slot
  static constexpr int UA = BM / RPC / NW, UB = BN / RPC / NW;  // copies per wave of an A / Bt unit
  static_assert(BM % (RPC * NW) == 0 && BN % (RPC * NW) == 0, "copy split must be uniform per wave");
  static_assert(NU * UNIT <= 160 * 1024, "LDS");
  static_assert(2 * UA + UB <= 63, "copies in flight exceed the counter field");
};
using Wide = Cfg<4, 4, 2>;    // 256 features x 256 rows
using Narrow = Cfg<4, 2, 1>;  // 128 features x 256 rows
using Short = Cfg<4, 1, 1>;   // 128 features x 128 rows: N = 128 LayerNorm launches of fewer rows than 256 per CU

// Element types: F16 / BF16 (gp_device.hpp).


struct Args {
  const half_t* a;     // [M][lda], the first K columns used
  const half_t* bt;    // [N][K] (transposed weights), or
  const half_t* w;     // [kw][ldw] (the weights in their own layout, BROW kernels)
  int ldw, kw;         // row stride and rows of w; rows [kw, K) read as zero
  const half_t* bias;  // [N] or null
  const half_t* r;     // [M][ldr] residual or null
  half_t* c;           // [M][ldc], the first N columns written
  int64_t M;
  int N;
  int K;
  int ka;              // columns of A read (a multiple of 8, <= K); columns [ka, K) read as zero
  int lda, ldc, ldr;   // row strides in elements
  // LayerNorm epilogue (LNM kernels): gamma / beta [N] or null (1 / 0), eps.
  const half_t* gamma;
  const half_t* beta;
  float eps;
  // LNM 2: per-row partial statistics [M][N / 128] ((mean, M2) of one wave's
  // 128 features, as 64-bit words), per-row-block commit counters, and the
  // launch context (epoch, status word, poll bound).
  unsigned long long* stats;
  QCounter* cnt;
  QueueCtx ctx;
  uint32_t ln_target;  // count of a row block's counter once this launch's waves have all committed
};

// Byte offset of logical 16-byte chunk c of unit row r: the chunk position is
// XOR-swizzled with (r / 2) so 16 consecutive rows (two per 256-byte bank
// window) read at one logical chunk cover 16 distinct 16-byte bank groups.
__device__ __forceinline__ int unit_off(int r, int c) { return r * ROWB + ((c ^ ((r >> 1) & 7)) << 4); }

template <typename F, int... I>
__device__ __forceinline__ void static_for(std::integer_sequence<int, I...>, F&& f) {
  (f(std::integral_constant<int, I>{}), ...);
}

// BROW: the weights are read in their own [K][N] layout.  A Bt unit then
// holds the slab's 64 weight rows, BN features each (2 BN bytes per row, four
// or two rows per 1 KiB copy), in the staged-rows layout of gp_device.hpp
// (16-byte chunk c of row r at chunk position c ^ 4 (r % 4)), and the MFMA A
// fragments -- columns of W -- are read with ds_read_b64_tr_b16, two reads
// per fragment.  No transposed copy of W is made.
//
// LNM (LayerNorm epilogue): 0 none; 1 the tile holds whole rows and each
// wave all 128 features of its rows (N = 128, Narrow), so the row statistics
// stay in the wave; 2 (Wide, N = 256 .. 1024) a row spans N / 128 waves of
// N / BN workgroups, which publish
// per-wave partial statistics and combine them (at most kLnPasses passes of
// one tile per workgroup, every workgroup resident).  Launches of one epoch
// share the counters: launch round r of the epoch waits for (r + 1) N / BN NW
// commits.
//
// E: the element type (F16 or BF16).
template <class C, int ACT, bool RESID, bool BROW = false, int LNM = 0, typename E = F16>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(1, 1))) void gemm_kernel(Args p) {
  __shared__ __attribute__((aligned(1024))) char ring[NU * C::UNIT];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int lr = lane & 31, lh = lane >> 5;
  const int wn = wave % C::WN, wm = wave / C::WN;
  const int K = p.K;
  const int nslab = K / BK;
  const int nunit = 2 * nslab;  // unit 2s: A rows of slab s; unit 2s+1: Bt rows of slab s
  const int npre = nunit < NU ? nunit : NU;  // units copied ahead of a tile's main loop

  // Persistent workers.  Workgroup b is taken to run on XCD b % 8 (the
  // dispatch order); the tiles are split into contiguous ranges, one per XCD,
  // and the workers of an XCD deal out their range, so the tiles that run at
  // the same time on one XCD share A and Bt panels in its L2.  Tile indices
  // fit in 32 bits: the host limits M to 2^31 - 1 rows.
  const int tiles_n = p.N / C::BN;
  const int ntiles = (int)((p.M + C::BM - 1) / C::BM) * tiles_n;
  const int G = gridDim.x;
  const int NX = G < 8 ? G : 8;
  const int xcd = blockIdx.x % NX, wid = blockIdx.x / NX;
  int nwx = (G - xcd + NX - 1) / NX;
  int hi = (int)((int64_t)ntiles * (xcd + 1) / NX);
  int t = (int)((int64_t)ntiles * xcd / NX) + wid;
  if constexpr (LNM == 2) {
    // Passes of G tiles: workgroup b takes tile f(b) of every pass, j G +
    // f(b).  A pass holds whole row blocks (the host keeps G a multiple of
    // N / BN when there is more than one), so the N / BN tiles of a row block,
    // which wait for each other's LayerNorm statistics, all run in the same
    // pass on workgroups that are all resident; pass j + 1 waits on nothing
    // that pass j has not finished.  With a grid of whole multiples of 8, XCD
    // x takes tiles [x G/8, (x+1) G/8) of a pass, so the workgroups of one row
    // block mostly share an L2.
    t = G % 8 == 0 ? (int)(blockIdx.x % 8) * (G / 8) + (int)(blockIdx.x / 8) : (int)blockIdx.x;
    hi = ntiles;
    nwx = G;
  }
  if (t >= hi) return;

  // Copies.  Copy j of a wave fills unit rows RPC (j NW + w) .. + RPC-1; lane
  // l writes row RPC (j NW + w) + l / CPR at chunk position l % CPR, which
  // holds the logical chunk the unit_off swizzle maps there.  Rows of
  // consecutive j are RPC NW = 32 apart, which leaves the swizzle unchanged,
  // so the source offset of every copy of a lane is voff plus the
  // wave-uniform (j RPC NW) K 2 + 128 s, passed in an SGPR.  Rows of A past M
  // lie outside the descriptor's range and read as zero.
  static_assert((RPC * NW / 2) % CPR == 0, "copies of one lane share a swizzle");
  const int vrow = RPC * wave + lane / CPR;
  const int vswz = ((lane % CPR) ^ ((vrow >> 1) & 7)) << 4;
  const int voffa = vrow * p.lda * 2 + vswz;
  // BROW copies: CPRB 16-byte chunks per weight row, RPCB rows per copy; copy
  // j of a wave covers rows RPCB (j NW + w) .. + RPCB - 1 of the slab, whose
  // row % 4 does not depend on j, so again only an SGPR offset changes.
  constexpr int CPRB = C::BN / 8, RPCB = 64 / CPRB;
  const int rq = RPCB * wave + lane / CPRB;
  const int voffb = BROW ? rq * p.ldw * 2 + (((lane % CPRB) ^ (4 * (rq & 3))) << 4) : vrow * K * 2 + vswz;
  // A slabs that reach past column ka: a lane whose chunk starts at or past
  // ka reads from an offset beyond every descriptor's range, so the copy
  // writes zeros (the weight rows it meets are zero too).
  const int lck = (vswz >> 4) * 8;  // the lane's first column within a slab
  constexpr int kBeyond = 0x40000000;
  const int jstra = RPC * NW * p.lda * 2, jstrb = BROW ? RPCB * NW * p.ldw * 2 : RPC * NW * K * 2;
  const int slabb = BROW ? 64 * p.ldw * 2 : ROWB;  // source offset of the next slab's B unit
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
    T.ra = make_rsrc(p.a + T.m0 * p.lda, T.rows * p.lda * 2);
    if constexpr (BROW)
      T.rb = make_rsrc(p.w + T.n0, (int)((int64_t)p.kw * p.ldw * 2 - (int64_t)T.n0 * 2));
    else
      T.rb = make_rsrc(p.bt + (int64_t)T.n0 * K, C::BN * K * 2);
    return T;
  };
  // Copies [j0, j1) of unit u (default: all of them).
  auto issue = [&](const Tile& T, int u, int j0 = 0, int j1 = 64) {
    GP_LDS char* const s = lds + (u % NU) * C::UNIT;
    const int so = (u >> 1) * ROWB;
    if (u & 1) {
      const int sob = (u >> 1) * slabb;
#pragma unroll
      for (int j = 0; j < C::UB; ++j)
        if (j >= j0 && j < j1) dma16_buf_so(T.rb, voffb, j * jstrb + sob, s + (j * NW + wave) * 1024);
    } else {
      const int k0 = (u >> 1) * BK;
      const int vo = k0 + BK <= p.ka || k0 + lck < p.ka ? voffa : kBeyond;
#pragma unroll
      for (int j = 0; j < C::UA; ++j)
        if (j >= j0 && j < j1) dma16_buf_so(T.ra, vo, j * jstra + so, s + (j * NW + wave) * 1024);
    }
  };
  auto prefetch = [&](const Tile& T) {
    for (int u = 0; u < npre; ++u) issue(T, u);
  };

  // Operand fragments of one 16-k step: NBW of Bt, MBW of A.
  struct Frags {
    h8 a[C::NBW], b[C::MBW];
  };
  const int frow = 32 * C::NBW * wn + lr;  // Bt unit row of fragment nb: frow + 32 nb
  const int arow = 32 * C::MBW * wm + lr;  // A unit row of fragment mb: arow + 32 mb
  // Rows 32 apart share the unit_off swizzle, so fragment nb (mb) of step ks
  // is at a per-lane offset for ks plus the constant 32 nb ROWB (32 mb ROWB).
  // BROW: lane part of the first transposed read of fragment nb (rows
  // 8 lh + m / 4 of the step, features 32 (NBW wn + nb) + 16 (group % 2) +
  // 4 (m % 4) .. +3, m = lane % 16); the second read is four rows further.
  // With NBW = 4 the swizzled chunk of fragment nb is that of fragment 0
  // with bits 2-3 xor-ed by nb, so lb(nb) = lb(0) ^ 64 nb.
  static_assert(!BROW || C::NBW == 4, "fragment offsets assume four fragments per wave");
  int lb0 = 0;
  if constexpr (BROW) {
    const int m = lane & 15, r4 = m >> 2;
    const int f = 32 * C::NBW * wn + 16 * ((lane >> 4) & 1) + 4 * (m & 3);
    lb0 = (8 * lh + r4) * (C::BN * 2) + (((f >> 3) ^ (4 * r4)) << 4) + (f & 7) * 2;
  }
  auto load = [&](Frags& f, int kt, int ks) {
    GP_LDS const char* const ua = lds + ((2 * kt) % NU) * C::UNIT + unit_off(arow, 2 * ks + lh);
    if constexpr (BROW) {
      GP_LDS const char* const ub = lds + ((2 * kt + 1) % NU) * C::UNIT + ks * 16 * (C::BN * 2);
#pragma unroll
      for (int nb = 0; nb < C::NBW; ++nb) {
        const int lb = lb0 ^ (64 * nb);
        const s4 x0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((GP_LDS s4*)(ub + lb));
        const s4 x1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((GP_LDS s4*)(ub + lb + 4 * (C::BN * 2)));
        f.a[nb] = __builtin_bit_cast(h8, __builtin_shufflevector(x0, x1, 0, 1, 2, 3, 4, 5, 6, 7));
      }
    } else {
      GP_LDS const char* const ub = lds + ((2 * kt + 1) % NU) * C::UNIT + unit_off(frow, 2 * ks + lh);
#pragma unroll
      for (int nb = 0; nb < C::NBW; ++nb) f.a[nb] = *(GP_LDS const h8*)(ub + 32 * nb * ROWB);
    }
#pragma unroll
    for (int mb = 0; mb < C::MBW; ++mb) f.b[mb] = *(GP_LDS const h8*)(ua + 32 * mb * ROWB);
  };
  f16x acc[C::NBW][C::MBW];
  // MFMAs of one step; the nfr fragment reads and nv copies issued just
  // before are spread one per MFMA over the first MFMAs, so that their
  // latency hides behind the matrix pipe.
  auto mma = [&](const Frags& f, auto nfr_c, auto nv_c) {
    constexpr int nfr = decltype(nfr_c)::value, nv = decltype(nv_c)::value;
#pragma unroll
    for (int nb = 0; nb < C::NBW; ++nb)
#pragma unroll
      for (int mb = 0; mb < C::MBW; ++mb) acc[nb][mb] = E::mma(f.a[nb], f.b[mb], acc[nb][mb]);
    constexpr int nm = C::NBW * C::MBW;
#pragma unroll
    for (int i = 0; i < nm; ++i) {
      if (i < nfr) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      if (i + nm < nfr) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // more reads than MFMAs: two per MFMA
      if (i + 2 * nm < nfr) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // (three: Short tiles reading W in place)
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      if (i < nv) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
    }
  };
  using I0 = std::integral_constant<int, 0>;

  // Memory operations of one epilogue: a store (and a residual load) per
  // fragment and element group.
  constexpr int EPI_OPS = C::NBW * C::MBW * (RESID ? 6 : 2);
  // Waits until units 0 and 1 of a tile have landed.  Issued after them: the
  // tile's units 2 .. npre-1 (A, Bt, A) and, from the second tile on, the
  // previous tile's epilogue.  The counter field holds at most 63, which still
  // implies units 0 and 1 whenever more than 63 operations followed them.
  auto wait_first = [&](bool after_epi) {
    if (after_epi) {
      if constexpr (EPI_OPS >= 63) {
        wait_vmcnt<63>();
      } else {
        if (npre == NU) wait_vmcnt<(2 * C::UA + C::UB + EPI_OPS > 63 ? 63 : 2 * C::UA + C::UB + EPI_OPS)>();
        else if (npre == 4) wait_vmcnt<(C::UA + C::UB + EPI_OPS > 63 ? 63 : C::UA + C::UB + EPI_OPS)>();
        else wait_vmcnt<EPI_OPS>();
      }
    } else {
      if (npre == NU) wait_vmcnt<2 * C::UA + C::UB>();
      else if (npre == 4) wait_vmcnt<C::UA + C::UB>();
      else wait_vmcnt<0>();
    }
  };

  constexpr int NFR = (BROW ? 2 : 1) * C::NBW + C::MBW;  // fragment reads per step
  static_assert(NFR <= 3 * C::NBW * C::MBW, "reads are spread at most three per MFMA");
  Tile T = tile_at(t);
  prefetch(T);
#pragma unroll
  for (int nb = 0; nb < C::NBW; ++nb)
#pragma unroll
    for (int mb = 0; mb < C::MBW; ++mb) acc[nb][mb] = f16x{};
  wait_first(false);
  for (;;) {
    // Main loop.  Fragments of k-step ks live in f[ks % 2]; the reads of step
    // ks+1 are issued just before the MFMAs of step ks.  Before the last step
    // of slab kt: wait for slab kt+1 (units 2kt+2, 2kt+3; unit 2kt+4 may still
    // be in flight), barrier, and read step 0 of slab kt+1.  The barrier
    // certifies that every wave's copies of slab kt+1 landed and that every
    // wave has read slab kt into registers, so units 2kt+5 and 2kt+6 may go
    // into slab kt's slots.  Their copies are issued during the first three
    // steps of slab kt+1 (the Bt unit over steps 0-1, then the A unit over
    // steps 1-2), one copy after each of the first MFMAs of a step, so no
    // step's MFMAs wait behind a burst of copy issues; the A unit is still
    // the last one issued at the next wait.  Which units a slab copies
    // depends only on its position in the tile, so the slab body is
    // instantiated per case and stays branch-free for the scheduler.
    static_assert(KS == 4, "the copies of two units are spread over three steps");
    Frags f[2];
    lds_barrier();
    load(f[0], 0, 0);
    // One slab kt < nslab - 1; MODE: which freed units are copied during it
    // (0 none, 1 the Bt unit 2kt+3, 2 both 2kt+3 and the A unit 2kt+4).
    auto slab = [&](int kt, auto mode_c) {
      constexpr int MODE = decltype(mode_c)::value;
      const int pb = 2 * kt + 3, pa = 2 * kt + 4;
      static_for(std::make_integer_sequence<int, KS - 1>{}, [&](auto ks_c) {
        constexpr int ks = decltype(ks_c)::value;
        load(f[(ks + 1) % 2], kt, ks + 1);
        if constexpr (MODE >= 1 && ks == 0) issue(T, pb, 0, C::UB / 2);
        if constexpr (MODE >= 1 && ks == 1) issue(T, pb, C::UB / 2, C::UB);
        if constexpr (MODE == 2 && ks == 1) issue(T, pa, 0, C::UA / 2);
        if constexpr (MODE == 2 && ks == 2) issue(T, pa, C::UA / 2, C::UA);
        constexpr int nv = (MODE >= 1 && ks < 2 ? C::UB / 2 : 0) + (MODE == 2 && ks > 0 ? C::UA / 2 : 0);
        mma(f[ks % 2], std::integral_constant<int, NFR>{}, std::integral_constant<int, nv>{});
      });
      if (kt + 3 <= nslab)
        wait_vmcnt<C::UA>();
      else
        wait_vmcnt<0>();
      lds_barrier();
      load(f[0], kt + 1, 0);
      mma(f[1], std::integral_constant<int, NFR>{}, I0{});
    };
    if (nslab >= 2) slab(0, I0{});
    for (int kt = 1; kt + 2 < nslab; ++kt) slab(kt, std::integral_constant<int, 2>{});
    if (nslab >= 3) slab(nslab - 2, std::integral_constant<int, 1>{});
#pragma unroll
    for (int ks = 0; ks + 1 < KS; ++ks) {
      load(f[(ks + 1) % 2], nslab - 1, ks + 1);
      mma(f[ks % 2], std::integral_constant<int, NFR>{}, I0{});
    }
    mma(f[1], I0{}, I0{});

    // Bias of the features this lane holds (see the epilogue), loaded before
    // the next tile's copies so that waiting for it does not wait for them.
    h4 bias[C::NBW][4];
#pragma unroll
    for (int nb = 0; nb < C::NBW; ++nb)
#pragma unroll
      for (int g = 0; g < 4; ++g)
        bias[nb][g] = p.bias ? *(const h4*)(p.bias + T.n0 + 32 * C::NBW * wn + 32 * nb + 8 * g + 4 * lh) : h4{};
    // LayerNorm affine of the same features.
    h4 gam[LNM ? C::NBW : 1][4], bet[LNM ? C::NBW : 1][4];
    if constexpr (LNM != 0) {
#pragma unroll
      for (int nb = 0; nb < C::NBW; ++nb)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int f = T.n0 + 32 * C::NBW * wn + 32 * nb + 8 * g + 4 * lh;
          const half_t one_h = __builtin_bit_cast(half_t, E::kOne);
          gam[nb][g] = p.gamma ? *(const h4*)(p.gamma + f) : h4{one_h, one_h, one_h, one_h};
          bet[nb][g] = p.beta ? *(const h4*)(p.beta + f) : h4{};
        }
    }

    // The next tile's first units go out before this tile's epilogue, once
    // every wave has read the last slab (the barrier), so their latency hides
    // behind it.
    const int tnext = t + nwx;
    const bool more = tnext < hi;
    Tile Nx;
    if (more) {
      Nx = tile_at(tnext);
      lds_barrier();
      prefetch(Nx);
    }

    // Epilogue.  For fragment (nb, mb) the lane holds row arow + 32 mb of the
    // tile and, in elements 4g .. 4g+3, features
    // n0 + 32 NBW wn + 32 nb + 8 g + 4 lh + (0..3).  After bias, activation
    // and residual, v_permlane32_swap trades groups g = 2q+1 of the lanes in
    // the lower half for groups g = 2q of the upper half, so each lane holds
    // eight consecutive features -- 32 nb + 16 q + 8 lh + (0..7) -- and one
    // 16-byte store per lane writes 32 contiguous bytes of each of the 32
    // rows.  Output and residual go through buffer descriptors limited to the
    // tile's valid rows; the residual loads of one nb are all issued before
    // the first is used.
    const __amdgpu_buffer_rsrc_t rc = make_rsrc(p.c + T.m0 * p.ldc, T.rows * p.ldc * 2);
    // (A LayerNorm kernel without a residual reads it through an empty
    // descriptor: zeros.)
    const bool hr = RESID && p.r != nullptr;
    const __amdgpu_buffer_rsrc_t rr = make_rsrc(hr ? p.r + T.m0 * p.ldr : p.c, hr ? T.rows * p.ldr * 2 : 0);
    // Per-row byte offsets, computed here (opaque: not hoisted out of the tile
    // loop as 64 live registers); the nb / g part is an instruction offset.
    int ebase[C::MBW], rbase[C::MBW];
#pragma unroll
    for (int mb = 0; mb < C::MBW; ++mb) {
      const int col = T.n0 + 32 * C::NBW * wn;
      ebase[mb] = opaque(((arow + 32 * mb) * p.ldc + col + 8 * lh) * 2);
      rbase[mb] = RESID ? opaque(((arow + 32 * mb) * p.ldr + col + 4 * lh) * 2) : 0;
    }
    auto eoff = [&](int nb, int q, int mb) { return ebase[mb] + (32 * nb + 16 * q) * 2; };
    auto roff = [&](int nb, int g, int mb) { return rbase[mb] + (32 * nb + 8 * g) * 2; };
    // Stores of the eight-feature groups of fragment (nb, mb), o[g] holding
    // feature group g (the v_permlane32_swap pairing described above).
    auto store_frag = [&](const u32x2 (&o)[4], int nb, int mb) {
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const auto lo = __builtin_amdgcn_permlane32_swap(o[2 * q][0], o[2 * q + 1][0], false, false);
        const auto hi = __builtin_amdgcn_permlane32_swap(o[2 * q][1], o[2 * q + 1][1], false, false);
        const u32x4 w = {(unsigned)lo[0], (unsigned)hi[0], (unsigned)lo[1], (unsigned)hi[1]};
        buf_store_u4(rc, eoff(nb, q, mb), w);
      }
    };
    if constexpr (LNM != 0) {
      // LayerNorm epilogue.  Pass 1: v = fp16(acc + bias + r) -- the value a
      // separate LayerNorm launch would read -- and the row sums.  The fp16
      // values go back into the first eight registers of their accumulator
      // fragment as pairs, and every later use reads them through
      // v_fma_mix_f32 (fp16 operands taken as they are), which keeps the
      // epilogue's VALU work about half of an fp32 formulation's.  A lane
      // holds 64 features of its row (16 per fragment nb), the lane 32 apart
      // the other 64 of the wave's 128.
      static_assert(C::NBW == 4, "a wave holds 128 features of its rows");
      float s[C::MBW], mean[C::MBW], rstd[C::MBW];
#pragma unroll
      for (int mb = 0; mb < C::MBW; ++mb) s[mb] = 0.f;
      // 1.0 the compiler cannot see: fma(x, one, y) stays an fma (one
      // v_fma_mix_f32 when x is an fp16 value) instead of becoming x + y.
      float one = 1.f;
      asm volatile("" : "+v"(one));
#pragma unroll
      for (int nb = 0; nb < C::NBW; ++nb) {
#pragma unroll
        for (int mb = 0; mb < C::MBW; ++mb) asm volatile("" : "+a"(acc[nb][mb]));
        h4 res[4][C::MBW];
#pragma unroll
        for (int g = 0; g < 4; ++g)
#pragma unroll
          for (int mb = 0; mb < C::MBW; ++mb) res[g][mb] = buf_load_h4(rr, roff(nb, g, mb));
#pragma unroll
        for (int mb = 0; mb < C::MBW; ++mb) {
          h2 pk[8];
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            f2 t;
#pragma unroll
            for (int e = 0; e < 2; ++e) {
              // fma(x, 1, y) rounds x + y once: the sums of the plain epilogue
              const int i = 2 * j + e;
              t[e] = __builtin_fmaf(E::val(bias[nb][i / 4][i % 4]), one, acc[nb][mb][i]);
              t[e] = __builtin_fmaf(E::val(res[i / 4][mb][i % 4]), one, t[e]);
            }
            // Rounded to fp16 from the fp32 sum, as the plain epilogue does (the
            // barrier keeps the rounding out of the fma: one v_cvt_pk_f16_f32).
            asm volatile("" : "+v"(t));
            pk[j] = E::cvt2(t);
#pragma unroll
            for (int e = 0; e < 2; ++e) s[mb] = __builtin_fmaf(E::val(pk[j][e]), one, s[mb]);
          }
#pragma unroll
          for (int j = 0; j < 8; ++j) acc[nb][mb][j] = __builtin_bit_cast(float, pk[j]);
        }
#pragma unroll
        for (int mb = 0; mb < C::MBW; ++mb) asm volatile("" : "+a"(acc[nb][mb]));  // v back in AGPRs
      }
      // (The element is copied out first: __builtin_bit_cast of a vector
      // element lvalue reads element 0 of the vector in this compiler.)
      auto vh = [&](int nb, int mb, int i) {
        const float w = acc[nb][mb][i / 2];
        return E::val(__builtin_bit_cast(h2, w)[i % 2]);
      };
      // Pass 2: the wave's mean and sum of squared deviations per row.
      float q[C::MBW];
#pragma unroll
      for (int mb = 0; mb < C::MBW; ++mb) {
        mean[mb] = sum_lane_halves(s[mb]) * (1.f / 128);
        q[mb] = 0.f;
#pragma unroll
        for (int nb = 0; nb < C::NBW; ++nb)
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const float d = __builtin_fmaf(vh(nb, mb, i), one, -mean[mb]);
            q[mb] = __builtin_fmaf(d, d, q[mb]);
          }
        q[mb] = sum_lane_halves(q[mb]);
      }
      bool ok = true;
      if constexpr (LNM == 1) {
#pragma unroll
        for (int mb = 0; mb < C::MBW; ++mb) rstd[mb] = rsqrtf(q[mb] * (1.f / 128) + p.eps);
      } else {
        // Publish (mean, M2) of this wave's 128 features for each of its
        // rows, count the wave's commit on the row block, wait for all
        // N / BN x NW commits, and combine the N / 128 partials (Chan et al.:
        // M2 = sum M2_i + 128 sum (mean_i - mean)^2), P <= 8.
        const int P = p.N >> 7;
        const int pidx = (T.n0 >> 7) + wn;
#pragma unroll
        for (int mb = 0; mb < C::MBW; ++mb) {
          const int r = arow + 32 * mb;
          if (lh == 0 && r < T.rows)
            __hip_atomic_store(p.stats + (T.m0 + r) * P + pidx, __builtin_bit_cast(unsigned long long, f2{mean[mb], q[mb]}),
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __builtin_amdgcn_s_waitcnt(kWaitAll);
        QCounter* const c = p.cnt + (int)(T.m0 / C::BM);
        if (lane == 0) qcommit(c, p.ctx.epoch);
        const uint32_t target = p.ln_target;
        for (int it = 0;; ++it) {
          const unsigned long long v = __hip_atomic_load(&c->v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          if (qcount(v, p.ctx.epoch) >= target) break;
          if (q_aborted(p.ctx)) {
            ok = false;
            break;
          }
          if (it >= p.ctx.limit) {
            if (lane == 0) q_fail(p.ctx, kErrTimeout);
            ok = false;
            break;
          }
          __builtin_amdgcn_s_sleep(4);
        }
#pragma unroll
        for (int mb = 0; mb < C::MBW; ++mb) {
          const int r = arow + 32 * mb;
          f2 part[8];
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            part[i] = f2{0.f, 0.f};
            if (i < P && r < T.rows && ok)
              part[i] = __builtin_bit_cast(f2, __hip_atomic_load(p.stats + (T.m0 + r) * P + i, __ATOMIC_RELAXED,
                                                                 __HIP_MEMORY_SCOPE_AGENT));
          }
          float m = 0.f;
#pragma unroll
          for (int i = 0; i < 8; ++i) m += part[i][0];
          m /= (float)P;
          float m2 = 0.f;
#pragma unroll
          for (int i = 0; i < 8; ++i)
            if (i < P) {
              const float d = part[i][0] - m;
              m2 += __builtin_fmaf(128.f * d, d, part[i][1]);
            }
          mean[mb] = m;
          rstd[mb] = rsqrtf(m2 / (float)p.N + p.eps);
        }
      }
      // Pass 3: normalise, affine, fp16, store.  After a failed wait nothing
      // is stored.
      if (ok) {
#pragma unroll
        for (int nb = 0; nb < C::NBW; ++nb) {
#pragma unroll
          for (int mb = 0; mb < C::MBW; ++mb) asm volatile("" : "+a"(acc[nb][mb]));
#pragma unroll
          for (int mb = 0; mb < C::MBW; ++mb) {
            u32x2 o[4];
#pragma unroll
            for (int g = 0; g < 4; ++g) {
              f4 v;
#pragma unroll
              for (int e = 0; e < 4; ++e)
                v[e] = __builtin_fmaf(__builtin_fmaf(vh(nb, mb, 4 * g + e), one, -mean[mb]) * rstd[mb],
                                      E::val(gam[nb][g][e]), E::val(bet[nb][g][e]));
              o[g] = __builtin_bit_cast(u32x2, E::cvt4(v));
            }
            store_frag(o, nb, mb);
          }
        }
      }
#pragma unroll
      for (int nb = 0; nb < C::NBW; ++nb)
#pragma unroll
        for (int mb = 0; mb < C::MBW; ++mb) acc[nb][mb] = f16x{};  // ready for the next tile
    } else {
#pragma unroll
      for (int nb = 0; nb < C::NBW; ++nb) {
        // Pin the accumulators of block nb in place until here: the blocks are
        // read one after another rather than all hoisted into VGPRs at once.
#pragma unroll
        for (int mb = 0; mb < C::MBW; ++mb) asm volatile("" : "+a"(acc[nb][mb]));
        h4 res[4][C::MBW];
        if constexpr (RESID) {
#pragma unroll
          for (int g = 0; g < 4; ++g)
#pragma unroll
            for (int mb = 0; mb < C::MBW; ++mb) res[g][mb] = buf_load_h4(rr, roff(nb, g, mb));
        }
#pragma unroll
        for (int mb = 0; mb < C::MBW; ++mb) {
          u32x2 o[4];
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            f4 v;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              v[e] = apply_act(acc[nb][mb][4 * g + e] + E::val(bias[nb][g][e]), ACT);
              if constexpr (RESID) v[e] += E::val(res[g][mb][e]);
            }
            o[g] = __builtin_bit_cast(u32x2, E::cvt4(v));
          }
          store_frag(o, nb, mb);
        }
#pragma unroll
        for (int mb = 0; mb < C::MBW; ++mb) acc[nb][mb] = f16x{};  // ready for the next tile
      }
    }
    if (!more) break;
    wait_first(true);
    t = tnext;
    T = Nx;
  }
}

// One 64 x 64 tile of wt[Np][Kp] = w[K][N] transposed, zero where k >= K or
// n >= N (16-bit values, any element type).  Rows of w come in as 16-byte
// chunks (one 128-byte row segment per eight threads) into an LDS tile whose
// chunk c of row r sits at chunk position c ^ (r % 8).  ds_read_b64_tr_b16
// then hands lane j of a 16-lane group column j of the 4 x 16 block its lanes
// point at (lane m at row r0 + m/4, columns c0 + 4 (m % 4) .. +3): two reads
// give a lane eight consecutive k of one output row, stored as one 16-byte
// chunk.  The swizzle keeps both the chunk writes and the transposing reads
// free of bank conflicts.
__device__ __forceinline__ void transpose_tile64(const half_t* w, int K, int N, half_t* wt, int Kp, int k0, int n0,
                                                 GP_LDS char* tile) {
  const int t = threadIdx.x;
  const bool whole = N % 8 == 0 && (uintptr_t)w % 16 == 0 && k0 + 64 <= K && n0 + 64 <= N;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int c = t + 256 * h;  // row r = c / 8, 8-column chunk cg = c % 8
    const int r = c >> 3, cg = c & 7;
    h8 v;
    if (whole) {
      v = *(const h8*)(w + (int64_t)(k0 + r) * N + n0 + 8 * cg);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int k = k0 + r, n = n0 + 8 * cg + e;
        v[e] = (k < K && n < N) ? w[(int64_t)k * N + n] : (half_t)0.f;
      }
    }
    *(GP_LDS h8*)(tile + r * 128 + ((cg ^ (r & 7)) << 4)) = v;
  }
  __syncthreads();
  const int m = t & 15, grp = t >> 4;  // 16 groups of 16 lanes
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int nb = grp & 3, kg = (grp >> 2) + 4 * q;  // output rows n0 + 16 nb + m, k0 + 8 kg .. +7
    s4 part[2];
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const int r = 8 * kg + 4 * hh + (m >> 2), col = 16 * nb + 4 * (m & 3);
      part[hh] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (GP_LDS s4*)(tile + r * 128 + (((col >> 3) ^ (r & 7)) << 4) + (col & 7) * 2));
    }
    *(h8*)(wt + (int64_t)(n0 + 16 * nb + m) * Kp + k0 + 8 * kg) =
        __builtin_bit_cast(h8, __builtin_shufflevector(part[0], part[1], 0, 1, 2, 3, 4, 5, 6, 7));
  }
}

// The weight preparation of a whole chain in one launch: for every layer,
// wt[Np][Kp] = w[K][N] transposed and zero-padded (transpose_tile64), and
// bp[Np] = b zero-padded (zeros for a null b; skipped for a null bp).  Layer i
// owns blocks [blk0_i, blk0_{i+1}); its first block also writes the bias.
struct PrepLayer {
  const half_t* w;
  half_t* wt;
  const half_t* b;
  half_t* bp;
  int K, N, Kp, Np, blk0;
};
constexpr int kMaxPrep = 32;
struct PrepBatch {
  PrepLayer L[kMaxPrep];
  int n;
};

__global__ __launch_bounds__(256) void prep_kernel(PrepBatch pb) {
  __shared__ __attribute__((aligned(16))) char tile[64 * 128];
  int i = 0;
  while (i + 1 < pb.n && (int)blockIdx.x >= pb.L[i + 1].blk0) ++i;
  const PrepLayer& L = pb.L[i];
  const int local = (int)blockIdx.x - L.blk0;
  const int tn = L.Np / 64;
  const int n0 = (local % tn) * 64, k0 = (local / tn) * 64;
  transpose_tile64(L.w, L.K, L.N, L.wt, L.Kp, k0, n0, (GP_LDS char*)tile);
  if (local == 0 && L.bp)
    for (int j = threadIdx.x; j < L.Np; j += 256) L.bp[j] = (L.b && j < L.N) ? L.b[j] : (half_t)0.f;
}

// A one-output layer, out[m] = act(a[m][0:K] . w[0:K] + b), fp32 accumulate:
// a GEMV over rows, which a 128-wide GEMM tile would spend 128 columns of
// MFMA and output on.  Each half of a wave takes one row and reads it as
// 16-byte chunks (one 512-byte row per instruction at K = 256), then sums
// its 32 partial dot products with lane exchanges.
template <typename E>
__global__ __launch_bounds__(256) void gemv1_kernel(const half_t* a, int lda, int64_t M, int K, const half_t* w,
                                                    const half_t* b, int act, half_t* out) {
  const int lane = threadIdx.x & 63, hw = lane >> 5, l32 = lane & 31;
  const int64_t wv = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int64_t nw = (int64_t)gridDim.x * 4;
  const int nc = K / 8;
  const float bias = b ? E::val(b[0]) : 0.f;
  for (int64_t m0 = 2 * wv; m0 < M; m0 += 2 * nw) {
    const int64_t m = m0 + hw;
    float s = 0.f;
    if (m < M) {
      const half_t* row = a + m * lda;
      for (int c = l32; c < nc; c += 32) {
        const h8 x = *(const h8*)(row + 8 * c);
        const h8 v = *(const h8*)(w + 8 * c);
#pragma unroll
        for (int e = 0; e < 8; ++e) s = __builtin_fmaf(E::val(x[e]), E::val(v[e]), s);
      }
    }
#pragma unroll
    for (int o = 16; o > 0; o >>= 1) s += __shfl_xor(s, o, 32);
    if (l32 == 0 && m < M) out[m] = E::cvt1(apply_act(s + bias, act));
  }
}

template <class C, int ACT, bool RESID, bool BROW, int LNM = 0, typename E = F16>
static hipError_t launch(const Args& a, int num_cus, hipStream_t s) {
  const int64_t tiles = ((a.M + C::BM - 1) / C::BM) * (a.N / C::BN);
  // One persistent workgroup per CU; the LNM 2 kernels run at most kLnPasses
  // passes of one tile per workgroup, every pass of whole row blocks.
  if (LNM == 2 && (tiles > kLnPasses * num_cus || (tiles > num_cus && num_cus % (a.N / C::BN) != 0)))
    return hipErrorInvalidValue;
  const int64_t grid = tiles < num_cus ? tiles : num_cus;
  hipLaunchKernelGGL((gemm_kernel<C, ACT, RESID, BROW, LNM, E>), dim3((unsigned)grid), dim3(NT), 0, s, a);
  return hipGetLastError();
}

template <class C, bool BROW, typename E>
static hipError_t dispatch(const Args& g, int act, int ncu, hipStream_t s) {
  if (g.r) return act == ACT_NONE ? launch<C, ACT_NONE, true, BROW, 0, E>(g, ncu, s) : hipErrorInvalidValue;
  switch (act) {
    case ACT_NONE: return launch<C, ACT_NONE, false, BROW, 0, E>(g, ncu, s);
    case ACT_RELU: return launch<C, ACT_RELU, false, BROW, 0, E>(g, ncu, s);
    case ACT_GELU_TANH: return launch<C, ACT_GELU_TANH, false, BROW, 0, E>(g, ncu, s);
    case ACT_SIGMOID: return launch<C, ACT_SIGMOID, false, BROW, 0, E>(g, ncu, s);
    default: return hipErrorInvalidValue;
  }
}

// Every kernel of one element type.
template <typename E>
static hipError_t launch_typed(const GemmArgs& a, Args& g, bool brow, int num_cus, hipStream_t s) {
  if (a.ln) {
    if (a.N == 128 && (a.M + Narrow::BM - 1) / Narrow::BM < num_cus)
      return brow ? launch<Short, ACT_NONE, true, true, 1, E>(g, num_cus, s)
                  : launch<Short, ACT_NONE, true, false, 1, E>(g, num_cus, s);
    if (a.N == 128) return brow ? launch<Narrow, ACT_NONE, true, true, 1, E>(g, num_cus, s)
                                : launch<Narrow, ACT_NONE, true, false, 1, E>(g, num_cus, s);
    return brow ? launch<Wide, ACT_NONE, true, true, 2, E>(g, num_cus, s)
                : launch<Wide, ACT_NONE, true, false, 2, E>(g, num_cus, s);
  }
  if (a.N % Wide::BN == 0) return brow ? dispatch<Wide, true, E>(g, a.act, num_cus, s) : dispatch<Wide, false, E>(g, a.act, num_cus, s);
  return brow ? dispatch<Narrow, true, E>(g, a.act, num_cus, s) : dispatch<Narrow, false, E>(g, a.act, num_cus, s);
}

// The LNM 2 exchange area: the status word's line, kLnMaxBlocks counter
// lines (one per row block of a launch: a Wide tile row), then 8 bytes per
// row and wave of partial statistics.  The counters sit at the same place whatever the
// launch's shape: the statistics of one call must never land where a later
// call with more row blocks keeps a counter (a payload word there would
// defeat the epoch test and the wait would run out).
constexpr int64_t kLnMaxBlocks = 1024;
size_t ln_ws_bytes(int64_t M, int64_t N) {
  return sizeof(QCounter) * (size_t)(1 + kLnMaxBlocks) + (size_t)M * (size_t)(N / 128) * 8;
}

}  // namespace gemm

int64_t gemm_ln_max_rows(int64_t N, int num_cus) {
  if (N == 128) return int64_t(1) << 62;  // rows stay within a wave: any M
  if (N % gemm::Wide::BN || N > 1024) return 0;
  const int64_t tiles_n = N / gemm::Wide::BN;
  const int64_t one_pass = (num_cus / tiles_n) * gemm::Wide::BM;
  return num_cus % tiles_n == 0 ? gemm::kLnPasses * one_pass : one_pass;
}

size_t gemm_ln_ws_bytes(int64_t M, int64_t N) { return N == 128 ? 0 : gemm::ln_ws_bytes(M, N); }

hipError_t gemm_launch(const GemmArgs& a, int num_cus, hipStream_t s) {
  using namespace gemm;
  if (a.M <= 0) return hipSuccess;
  if (a.N % 128 != 0 || a.K % BK != 0) return hipErrorInvalidValue;
  const int ka = a.ka ? (int)a.ka : (int)a.K;
  if (ka < 1 || ka > a.K || ka % 8) return hipErrorInvalidValue;
  const int lda = a.lda ? (int)a.lda : ka, ldc = a.ldc ? (int)a.ldc : (int)a.N;
  const int ldr = a.ldr ? (int)a.ldr : (int)a.N;
  if (lda < ka || ldc < a.N || (a.r && ldr < a.N) || lda % 8 || ldc % 8 || ldr % 8) return hipErrorInvalidValue;
  const bool brow = a.w != nullptr;
  const int ldw = a.ldw ? (int)a.ldw : (int)a.N, kw = a.kw ? (int)a.kw : (int)a.K;
  if (brow && (ldw < a.N || ldw % 8 || kw < 1 || kw > a.K || (uintptr_t)a.w % 16 ||
               (int64_t)kw * ldw * 2 > (int64_t(1) << 31) - 1))
    return hipErrorInvalidValue;
  if (!brow && !a.wt) return hipErrorInvalidValue;
  Args g{(const half_t*)a.x, (const half_t*)a.wt, (const half_t*)a.w, ldw, kw, (const half_t*)a.b,
         (const half_t*)a.r, (half_t*)a.out, a.M, (int)a.N, (int)a.K, ka, lda, ldc, ldr,
         (const half_t*)a.gamma, (const half_t*)a.beta, a.eps, nullptr, nullptr, QueueCtx{}, 0};
  if (a.dtype != GP_DTYPE_F16 && a.dtype != GP_DTYPE_BF16) return hipErrorInvalidValue;
  if (a.ln) {
    // N = 128 (rows within a wave) or 256 .. 1024 in whole 256-feature tiles.
    if (a.act != ACT_NONE || a.N > 1024 || (a.N != 128 && a.N % Wide::BN) || ((uintptr_t)a.gamma | (uintptr_t)a.beta) % 8)
      return hipErrorInvalidValue;
    if (a.N != 128) {
      if (!a.ln_ws || !a.status || a.epoch == 0 || a.M > gemm_ln_max_rows(a.N, num_cus)) return hipErrorInvalidValue;
      if ((a.M + Wide::BM - 1) / Wide::BM > kLnMaxBlocks) return hipErrorInvalidValue;
      QCounter* const q = (QCounter*)a.ln_ws;
      g.cnt = q + 1;
      g.stats = (unsigned long long*)(q + 1 + kLnMaxBlocks);
      g.ctx = QueueCtx{a.epoch, a.status, a.spin_limit > 0 ? a.spin_limit : kQueueSpinLimit};
      const int64_t tiles_n = a.N / Wide::BN;
      if (a.ln_round < 0 || (a.ln_round + 1) * tiles_n * NW > 0x7fffffff) return hipErrorInvalidValue;
      g.ln_target = (uint32_t)((a.ln_round + 1) * tiles_n * NW);
    }
  }
  return a.dtype == GP_DTYPE_BF16 ? launch_typed<BF16>(a, g, brow, num_cus, s) : launch_typed<F16>(a, g, brow, num_cus, s);
}

hipError_t prep_launch(const PrepSpec* L, int n, hipStream_t s) {
  using namespace gemm;
  for (int i0 = 0; i0 < n; i0 += kMaxPrep) {
    PrepBatch pb{};
    int blocks = 0;
    pb.n = n - i0 < kMaxPrep ? n - i0 : kMaxPrep;
    for (int i = 0; i < pb.n; ++i) {
      const PrepSpec& q = L[i0 + i];
      if (q.Kp % 64 != 0 || q.Np % 64 != 0 || q.K > q.Kp || q.N > q.Np || q.K < 1 || q.N < 1 || !q.w || !q.wt ||
          (uintptr_t)q.wt % 16 != 0)
        return hipErrorInvalidValue;
      pb.L[i] = {(const half_t*)q.w, (half_t*)q.wt, (const half_t*)q.b, (half_t*)q.bp,
                 (int)q.K, (int)q.N, (int)q.Kp, (int)q.Np, blocks};
      blocks += (int)(q.Np / 64 * (q.Kp / 64));
    }
    hipLaunchKernelGGL(prep_kernel, dim3((unsigned)blocks), dim3(256), 0, s, pb);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

hipError_t gemv1_launch(int64_t M, int64_t K, const void* a, int64_t lda, const void* w, const void* b, int act,
                        void* out, int num_cus, hipStream_t s, int dtype) {
  if (M <= 0) return hipSuccess;
  if (K < 8 || K % 8 || lda < K || lda % 8 || !a || !w || !out) return hipErrorInvalidValue;
  const int64_t want = (M + 7) / 8;  // eight rows per block and pass
  const int64_t grid = want < (int64_t)num_cus * 8 ? want : (int64_t)num_cus * 8;
  if (dtype != GP_DTYPE_F16 && dtype != GP_DTYPE_BF16) return hipErrorInvalidValue;
  if (dtype == GP_DTYPE_BF16)
    hipLaunchKernelGGL(gemm::gemv1_kernel<BF16>, dim3((unsigned)grid), dim3(256), 0, s, (const half_t*)a,
                       (int)lda, M, (int)K, (const half_t*)w, (const half_t*)b, act, (half_t*)out);
  else
    hipLaunchKernelGGL(gemm::gemv1_kernel<F16>, dim3((unsigned)grid), dim3(256), 0, s, (const half_t*)a,
                       (int)lda, M, (int)K, (const half_t*)w, (const half_t*)b, act, (half_t*)out);
  return hipGetLastError();
}

hipError_t transpose_launch(const void* in, void* out, int64_t K, int64_t N, hipStream_t s, int64_t Kp,
                            int64_t Np) {
  if (Kp == 0) Kp = K;
  if (Np == 0) Np = N;
  if (Kp % 64 != 0 || Np % 64 != 0 || K > Kp || N > Np) return hipErrorInvalidValue;
  const PrepSpec one{in, out, nullptr, nullptr, K, N, Kp, Np};
  return prep_launch(&one, 1, s);
}

}  // namespace gp
