// Stage-level kernels: the library's stage functions run over whole matrices
// (the reference's bulk-sync building blocks, and its identity pipeline).
//
//  * linear_kernel      one pipe_gemm_* stage per workgroup over M rows
//                       (the bulk-sync GEMM of common/bulksync_gemm.cuh:13-110,
//                       fp32 accumulation instead of fp16);
//  * layer_norm_rows_kernel  LayerNorm over M rows (host_layer_norm,
//                       common/layer_norm_v2.cuh:129-147), one wave per row;
//  * add_kernel         pipe_add (host_add2, common/elemwise_add.cuh:42-54);
//  * concat_kernel      pipe_concat (host_concat2, common/concat.cuh:50-69);
//  * route_kernel       copy pipelines over the reference's queue topologies:
//                       1:1 (misc_tests/pipeval/pipe_val_ext.cu:65-149),
//                       one producer / two consumers, and split / merge.
// Stage workgroups are persistent: workgroup b of G handles tiles b, b+G, ...
#include <hip/hip_runtime.h>

#include <atomic>

#include "../../include/gpipes.h"
#include "gp_host.hpp"
#include "pipeline.hpp"
#include "stages.hpp"

namespace gp {

constexpr int MBLK = 128;  // rows per tile, as the reference's mblk

struct TileWalk {
  int64_t ntiles;
  int nt;  // tiles of this workgroup
};

__device__ __forceinline__ TileWalk tile_walk(int64_t M) {
  const int64_t ntiles = (M + MBLK - 1) / MBLK;
  const int64_t b = blockIdx.x;
  return {ntiles, b < ntiles ? (int)((ntiles - 1 - b) / gridDim.x + 1) : 0};
}

// Reader over this workgroup's tiles of a row-major [M][width] matrix.
__device__ __forceinline__ MemoryReader tiles_in(const void* base, int64_t M, int width) {
  const int64_t b = blockIdx.x, G = gridDim.x;
  return MemoryReader(base ? (half_t*)base + b * MBLK * width : nullptr, G * MBLK * width, width, MBLK, M - b * MBLK,
                      G * MBLK);
}
__device__ __forceinline__ MemoryWriter tiles_out(void* base, int width) {
  const int64_t b = blockIdx.x, G = gridDim.x;
  return MemoryWriter((half_t*)base + b * MBLK * width, G * MBLK * width, width);
}

// Memory reader that yields null views when its base is null (optional
// accumulator input of pipe_gemm).
struct OptionalReader : MemoryReader {
  using MemoryReader::MemoryReader;
  __device__ TensorView read_acquire() {
    TensorView v = MemoryReader::read_acquire();
    if (base == nullptr) v.data = nullptr;
    return v;
  }
};

// The whole-matrix linear reads its input from memory: three 64-row part
// buffers let the next tile's copies run under this tile's MFMAs.
constexpr int kLinearBufs = 3;

template <int K, int ACT, bool LN>
__global__ __launch_bounds__(kStageThreads) void linear_kernel(LinearArgs a) {
  const TileWalk tw = tile_walk(a.M);
  if (tw.nt == 0) return;
  MemoryReader ir = tiles_in(a.x, a.M, K);
  MemoryReader acc0 = tiles_in(a.acc, a.M, 128);
  OptionalReader ar(acc0.base, acc0.stride, acc0.tile_stride, acc0.tile_rows, acc0.rows_left0, acc0.row_step);
  MemoryWriter ow = tiles_out(a.out, 128);
  const TensorView w{(half_t*)a.w, 128, K}, b{(half_t*)a.b, 1, 1};
  if constexpr (LN) {
    const TensorView g{(half_t*)a.gamma, 1, 1}, be{(half_t*)a.beta, 1, 1};
    pipe_gemm_bias_layer_norm<MBLK, K, kLinearBufs>(w, b, g, be, a.eps, ir, ar, ow, tw.nt);
  } else {
    pipe_gemm_bias_act<MBLK, K, ACT, kLinearBufs>(w, b, ir, ar, ow, tw.nt);
  }
}

__global__ __launch_bounds__(kStageThreads) void add_kernel(const half_t* a, const half_t* b, half_t* c, int64_t M,
                                                            int n) {
  const TileWalk tw = tile_walk(M);
  if (tw.nt == 0) return;
  MemoryReader r0 = tiles_in(a, M, n), r1 = tiles_in(b, M, n);
  MemoryWriter ow = tiles_out(c, n);
  pipe_add_n(r0, r1, ow, tw.nt, n);
}

__global__ __launch_bounds__(kStageThreads) void concat_kernel(const half_t* a, const half_t* b, half_t* c, int64_t M,
                                                               int n0, int n1) {
  const TileWalk tw = tile_walk(M);
  if (tw.nt == 0) return;
  MemoryReader r0 = tiles_in(a, M, n0), r1 = tiles_in(b, M, n1);
  MemoryWriter ow = tiles_out(c, n0 + n1);
  pipe_concat_n(r0, r1, ow, tw.nt, n0, n1);
}

// ---------------------------------------------------------------------------
// Copy pipelines over the queue topologies of the reference's apps.  Every
// stage copies 128-row tiles; pipeline g of P moves tiles g, g+P, ...
//  * ROUTE_IDENT (2 stages): x -> q -> out
//    (misc_tests/pipeval/pipe_val_ext.cu:65-149).  Pipeline g moves one
//    contiguous chunk of ceil(T / P) tiles, read with read_striped_input
//    (common/pipes.cuh:21-25), the reference apps' input striping.
//  * ROUTE_BROADCAST (3 stages): x -> q (one producer, two consumers) -> out
//    and -> out2, the MpmcRingQueue<E, N, 1, 2> of
//    apps/bert_addln_ffn/pipelined/bert_addln_ffn_pl.cuh:55 and
//    apps/nerf_a/pipelined/nerf_a_pl.cuh:55.
//  * ROUTE_DRAIN (3 stages): the broadcast with its second consumer writing
//    to a NullWriter (common/pipes.cuh:104-108) -- the reference's
//    dummy_consumer (bert_addln_ffn_pl.cuh:178-187), which keeps a
//    two-consumer queue draining; out2 is not written.
//  * ROUTE_SPLIT (5 stages): x -> q0 -> 3 workers (SplitQueueReader, round
//    robin) -> q1 (SplitQueueWriter, round robin) -> one reader in sequence
//    order -> out, the split write of bert_addln_ffn_pl.cuh:121.
//  * ROUTE_HANDOFF (2 stages): generated tiles -> q -> per-tile checksums,
//    the queue benchmark of misc_tests/pipeperf/pipeperf.cu:125-215.
//  * ROUTE_RELOAD (2 stages): x -> q (one slot, 64-row entries) -> out.  The
//    consumer reads the same 16 KiB of slot every tile, which fits its CU's
//    L1: payload loads served by L1 would return the slot's previous round.
// ---------------------------------------------------------------------------
using RouteEntry = QueueEntry2D<MBLK, 128>;
using IdentQueue = RingQueue<RouteEntry, 2>;
using BcastQueue = RingQueue<RouteEntry, 2, 1, 2>;
constexpr int kSplitWorkers = 3;
using SplitQueue = RingQueue<RouteEntry, kSplitWorkers + 1>;
constexpr int kReloadRows = 64;
using ReloadQueue = RingQueue<QueueEntry2D<kReloadRows, 128>, 1>;

struct RouteQueues {
  union {
    IdentQueue ident;
    BcastQueue bcast;
    struct {
      SplitQueue q0, q1;
    } split;
    ReloadQueue reload;
  };
};

struct RouteArgs {
  const half_t* x;
  half_t* out;
  half_t* out2;
  int64_t M;
  PipeCtl* ctl;
  RouteQueues* queues;
  QueueCtx ctx;
  int max_pipes;
};

constexpr int route_stages(int route) {
  return route == GP_ROUTE_IDENT || route == GP_ROUTE_HANDOFF || route == GP_ROUTE_RELOAD
             ? 2
             : (route == GP_ROUTE_SPLIT ? 2 + kSplitWorkers : 3);
}

// Hand-off benchmark payload: word i of tile t (row-major, 64 words per
// 128-wide fp16 row) is (t * 0x9E3779B1) ^ (i * 0x85EBCA77).  Thread j
// handles 16-byte chunks j, j + 256, ... (chunk q holds words 4q .. 4q+3 and
// lies in row q / 16); only the tile's valid rows are written and summed.
constexpr int kHandoffChunks = MBLK * 128 * 2 / 16;
__device__ __forceinline__ void handoff_fill(const TensorView& v, int64_t t) {
  const unsigned a = (unsigned)t * 0x9E3779B1u;
  for (int q = threadIdx.x; q < v.rows * 16; q += kStageThreads) {
    u32x4 w;
#pragma unroll
    for (int e = 0; e < 4; ++e) w[e] = a ^ ((unsigned)(4 * q + e) * 0x85EBCA77u);
    *(u32x4*)((char*)v.data + (int64_t)q * 16) = w;
  }
}
// Sum mod 2^32 of the tile's valid words, returned to thread 0.
__device__ __forceinline__ unsigned handoff_sum(const TensorView& v) {
  __shared__ unsigned part[kStageThreads / kWave];
  unsigned s = 0;
  for (int q = threadIdx.x; q < v.rows * 16; q += kStageThreads) {
    const u32x4 w = __builtin_bit_cast(u32x4, view_load_h8<true>(v, (int64_t)q * 8));  // a queue payload
    s += (w[0] + w[1]) + (w[2] + w[3]);
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) s += (unsigned)__shfl_xor((int)s, m);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
  __syncthreads();
  unsigned tot = 0;
  if (threadIdx.x == 0)
    for (int w = 0; w < kStageThreads / kWave; ++w) tot += part[w];
  __syncthreads();  // `part` is reused by the next tile
  return tot;
}
static_assert(kHandoffChunks % kStageThreads == 0, "whole chunks per thread");

template <int ROUTE>
__global__ __launch_bounds__(kStageThreads) void route_kernel(RouteArgs a) {
  constexpr int S = route_stages(ROUTE);
  const Role r = assign_role(a.ctl, S, a.ctx, a.max_pipes);
  if (r.pipe < 0) return;
  const int64_t T = (a.M + MBLK - 1) / MBLK, P = r.npipes, g = r.pipe;
  const int nt = g < T ? (int)((T - 1 - g) / P + 1) : 0;
  RouteQueues* q = a.queues + g;
  const int64_t tile = (int64_t)MBLK * 128;
  auto input = [&]() { return MemoryReader((half_t*)a.x + g * tile, P * tile, 128, MBLK, a.M - g * MBLK, P * MBLK); };
  auto output = [&](half_t* base) { return MemoryWriter(base + g * tile, P * tile, 128); };
  if constexpr (ROUTE == GP_ROUTE_IDENT) {
    // contiguous chunks: pipeline g moves tiles [g C, g C + C) of C = ceil(T / P)
    const int64_t C = (T + P - 1) / P;
    const int nc = g * C < T ? (int)(T - g * C < C ? T - g * C : C) : 0;
    if (r.stage == 0) {
      MemoryReader ir = read_striped_input((half_t*)a.x, (int)g, (int)C, MBLK, 128, a.M);
      QueueWriter<IdentQueue> ow(&q->ident, &a.ctx);
      pipe_copy_n(ir, ow, nc, 128);
    } else {
      QueueReader<IdentQueue> ir(&q->ident, &a.ctx);
      MemoryWriter ow((half_t*)a.out + g * C * tile, tile, 128);
      pipe_copy_n(ir, ow, nc, 128);
    }
  } else if constexpr (ROUTE == GP_ROUTE_RELOAD) {
    // 64-row tiles g, g + P, ... of pipeline g
    const int64_t T2 = (a.M + kReloadRows - 1) / kReloadRows;
    const int n2 = g < T2 ? (int)((T2 - 1 - g) / P + 1) : 0;
    const int64_t t2 = (int64_t)kReloadRows * 128;
    if (r.stage == 0) {
      MemoryReader ir((half_t*)a.x + g * t2, P * t2, 128, kReloadRows, a.M - g * kReloadRows, P * kReloadRows);
      QueueWriter<ReloadQueue> ow(&q->reload, &a.ctx);
      pipe_copy_n(ir, ow, n2, 128);
    } else {
      QueueReader<ReloadQueue> ir(&q->reload, &a.ctx);
      MemoryWriter ow((half_t*)a.out + g * t2, P * t2, 128);
      pipe_copy_n(ir, ow, n2, 128);
    }
  } else if constexpr (ROUTE == GP_ROUTE_HANDOFF) {
    // misc_tests/pipeperf/pipeperf.cu:125-163: sender / receiver over one
    // two-slot queue per pipeline, with generated payloads instead of the
    // reference's per-thread 4-byte stores and loads.
    if (r.stage == 0) {
      QueueWriter<IdentQueue> ow(&q->ident, &a.ctx);
      for (int i = 0; i < nt; ++i) {
        const int64_t t = g + (int64_t)i * P;
        const int64_t left = a.M - t * MBLK;
        const TensorView c = ow.write_acquire((int)(left < MBLK ? left : MBLK));
        handoff_fill(c, t);
        ow.write_release();
      }
    } else {
      QueueReader<IdentQueue> ir(&q->ident, &a.ctx);
      for (int i = 0; i < nt; ++i) {
        const TensorView v = ir.read_acquire();
        const unsigned sum = handoff_sum(v);
        ir.read_release();
        // a tile whose wait ran out has no rows: its checksum is not written
        if (threadIdx.x == 0 && v.rows > 0) ((unsigned*)a.out)[g + (int64_t)i * P] = sum;
      }
    }
  } else if constexpr (ROUTE == GP_ROUTE_BROADCAST || ROUTE == GP_ROUTE_DRAIN) {
    if (r.stage == 0) {
      MemoryReader ir = input();
      QueueWriter<BcastQueue> ow(&q->bcast, &a.ctx);
      pipe_copy_n(ir, ow, nt, 128);
    } else if (ROUTE == GP_ROUTE_DRAIN && r.stage == 2) {
      QueueReader<BcastQueue> ir(&q->bcast, &a.ctx);
      NullWriter ow;
      pipe_copy_n(ir, ow, nt, 128);
    } else {
      QueueReader<BcastQueue> ir(&q->bcast, &a.ctx);
      MemoryWriter ow = output(r.stage == 1 ? a.out : a.out2);
      pipe_copy_n(ir, ow, nt, 128);
    }
  } else {
    if (r.stage == 0) {
      MemoryReader ir = input();
      QueueWriter<SplitQueue> ow(&q->split.q0, &a.ctx);
      pipe_copy_n(ir, ow, nt, 128);
    } else if (r.stage <= kSplitWorkers) {
      const int w = r.stage - 1;
      const int cnt = nt > w ? (nt - w + kSplitWorkers - 1) / kSplitWorkers : 0;
      SplitQueueReader<SplitQueue> ir(&q->split.q0, &a.ctx, w, kSplitWorkers);
      SplitQueueWriter<SplitQueue> ow(&q->split.q1, &a.ctx, w, kSplitWorkers);
      pipe_copy_n(ir, ow, cnt, 128);
    } else {
      QueueReader<SplitQueue> ir(&q->split.q1, &a.ctx);
      MemoryWriter ow = output(a.out);
      pipe_copy_n(ir, ow, nt, 128);
    }
  }
}

// ---------------------------------------------------------------------------
// Host launchers
// ---------------------------------------------------------------------------
static int persistent_grid(int64_t M, int num_cus, int per_cu) {
  const int64_t ntiles = (M + MBLK - 1) / MBLK;
  const int64_t g = (int64_t)num_cus * per_cu;
  return (int)(ntiles < g ? ntiles : g);
}

template <int K, int ACT, bool LN>
static hipError_t launch_linear(const LinearArgs& a, int num_cus, hipStream_t s) {
  constexpr int lds = gemm_stage_lds<MBLK, K, kLinearBufs>() + kGemmParamLds;
  auto kern = linear_kernel<K, ACT, LN>;
  // The LDS limit is set once per device (not per launch, so that a launch
  // under graph capture makes no other runtime call).
  static std::atomic<bool> lds_set[64];
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= 64) return hipErrorInvalidDevice;
  if (!lds_set[dev].load(std::memory_order_acquire)) {
    e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    if (e != hipSuccess) return e;
    lds_set[dev].store(true, std::memory_order_release);
  }
  hipLaunchKernelGGL(kern, dim3(persistent_grid(a.M, num_cus, 1)), dim3(kStageThreads), lds, s, a);
  return hipGetLastError();
}

template <int K>
static hipError_t linear_dispatch_k(const LinearArgs& a, int num_cus, hipStream_t s) {
  if (a.gamma) return launch_linear<K, ACT_NONE, true>(a, num_cus, s);
  switch (a.act) {
    case ACT_NONE: return launch_linear<K, ACT_NONE, false>(a, num_cus, s);
    case ACT_RELU: return launch_linear<K, ACT_RELU, false>(a, num_cus, s);
    case ACT_GELU_TANH: return launch_linear<K, ACT_GELU_TANH, false>(a, num_cus, s);
    case ACT_SIGMOID: return launch_linear<K, ACT_SIGMOID, false>(a, num_cus, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t linear_launch(const LinearArgs& a, int num_cus, hipStream_t s) {
  switch (a.K) {
    case 128: return linear_dispatch_k<128>(a, num_cus, s);
    case 256: return linear_dispatch_k<256>(a, num_cus, s);
    case 384: return linear_dispatch_k<384>(a, num_cus, s);
    default: return hipErrorInvalidValue;
  }
}

// Whole-matrix LayerNorm (host_layer_norm, common/layer_norm_v2.cuh:129-147)
// with the same two-pass arithmetic as pipe_layer_norm, laid out for
// bandwidth: a row is read by LPR lanes with 16 or 32 bytes each (LPR = D/8
// up to 64: four rows per wave instruction at D = 128, one at D >= 512), the
// sums over a row's lanes are DPP row rotations and v_permlane16/32_swap, and
// each wave issues the loads of U row groups before it reduces the first, so
// that several memory latencies overlap (the kernel is HBM-bound).
template <int LPR>
__device__ __forceinline__ float sum_lanes(float x) {
  static_assert(LPR == 16 || LPR == 32 || LPR == 64, "16, 32 or 64 lanes per row");
#define GP_DPP_F(v, ctrl) __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), ctrl, 0xF, 0xF, false))
  x += GP_DPP_F(x, 0x128);  // row_ror:8
  x += GP_DPP_F(x, 0x124);  // row_ror:4
  x += GP_DPP_F(x, 0x4E);   // quad_perm [2,3,0,1]
  x += GP_DPP_F(x, 0xB1);   // quad_perm [1,0,3,2]
#undef GP_DPP_F
  if constexpr (LPR >= 32) {
    const unsigned u = __builtin_bit_cast(unsigned, x);
    const auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    x = __builtin_bit_cast(float, (unsigned)a[0]) + __builtin_bit_cast(float, (unsigned)a[1]);
  }
  if constexpr (LPR == 64) x = sum_lane_halves(x);
  return x;
}

template <int D>
__global__ __launch_bounds__(kStageThreads) void layer_norm_rows_kernel(const half_t* x, const half_t* gamma,
                                                                        const half_t* beta, float eps, half_t* out,
                                                                        int64_t M) {
  constexpr int LPR = D / 8 < kWave ? D / 8 : kWave;  // lanes per row
  constexpr int EPL = D / LPR;                        // elements per lane: 8 or 16
  constexpr int RPW = kWave / LPR;                    // rows per wave instruction
  constexpr int U = EPL == 8 ? 4 : 1;                 // row groups in flight per wave
  typedef _Float16 hv __attribute__((ext_vector_type(EPL)));
  const int lane = threadIdx.x & 63;
  const int sub = lane / LPR, c = lane % LPR;
  float g[EPL], bb[EPL];
  {
    hv gv, bv;
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
      gv[e] = (half_t)1.f;
      bv[e] = (half_t)0.f;
    }
    if (gamma) gv = *(const hv*)(gamma + c * EPL);
    if (beta) bv = *(const hv*)(beta + c * EPL);
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
      g[e] = (float)gv[e];
      bb[e] = (float)bv[e];
    }
  }
  const int64_t waves = (int64_t)gridDim.x * (kStageThreads / kWave);
  const int64_t w0 = (int64_t)blockIdx.x * (kStageThreads / kWave) + (threadIdx.x >> 6);
  // wave w takes row groups w, w + waves, ...; a group is RPW consecutive rows
  for (int64_t grp = w0; grp * RPW < M; grp += U * waves) {
    hv v[U];
    int64_t row[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      row[u] = (grp + u * waves) * RPW + sub;
      if (row[u] < M) v[u] = *(const hv*)(x + row[u] * D + c * EPL);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float f[EPL], s = 0.f;
#pragma unroll
      for (int e = 0; e < EPL; ++e) {
        f[e] = (float)v[u][e];
        s += f[e];
      }
      const float mean = sum_lanes<LPR>(s) * (1.f / D);
      float q = 0.f;
#pragma unroll
      for (int e = 0; e < EPL; ++e) {
        f[e] -= mean;
        q = __builtin_fmaf(f[e], f[e], q);
      }
      const float rstd = rsqrtf(sum_lanes<LPR>(q) * (1.f / D) + eps);
      hv o;
#pragma unroll
      for (int e = 0; e < EPL; ++e) o[e] = (half_t)__builtin_fmaf(f[e] * rstd, g[e], bb[e]);
      if (row[u] < M) *(hv*)(out + row[u] * D + c * EPL) = o;
    }
  }
}

hipError_t layer_norm_launch(int64_t M, int64_t D, const void* x, const void* gamma, const void* beta, float eps,
                             void* out, int num_cus, hipStream_t s) {
  const int64_t rows_per_block = kStageThreads / kWave;
  const int64_t want = (M + rows_per_block - 1) / rows_per_block, cap = (int64_t)num_cus * 8;
  const dim3 grid((unsigned)(want < cap ? want : cap)), block(kStageThreads);
  const half_t *hx = (const half_t*)x, *hg = (const half_t*)gamma, *hb = (const half_t*)beta;
  half_t* ho = (half_t*)out;
  switch (D) {
    case 128: hipLaunchKernelGGL(layer_norm_rows_kernel<128>, grid, block, 0, s, hx, hg, hb, eps, ho, M); break;
    case 256: hipLaunchKernelGGL(layer_norm_rows_kernel<256>, grid, block, 0, s, hx, hg, hb, eps, ho, M); break;
    case 512: hipLaunchKernelGGL(layer_norm_rows_kernel<512>, grid, block, 0, s, hx, hg, hb, eps, ho, M); break;
    case 1024: hipLaunchKernelGGL(layer_norm_rows_kernel<1024>, grid, block, 0, s, hx, hg, hb, eps, ho, M); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// dst[m][j] = act(src[m][j]) for j < w, 0 for w <= j < wpad: moves a column
// block between matrices with zero padding (the concat inputs, padded inputs
// and narrow heads of the MLP chains).  Strides in elements.  V elements per
// thread: 8 (16-byte vectors) when every width, stride and base allows it.
// Without an activation the values are copied as raw 16-bit patterns, so the
// copy serves fp16 and bf16 alike.
template <int V>
__global__ __launch_bounds__(kStageThreads) void place_kernel(const half_t* src, int64_t lds, int w, half_t* dst,
                                                              int64_t ldd, int wpad, int act, int64_t M) {
  typedef _Float16 hv __attribute__((ext_vector_type(V)));
  const int vpr = wpad / V;  // vectors per row
  const int64_t total = M * vpr;
  for (int64_t i = (int64_t)blockIdx.x * kStageThreads + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * kStageThreads) {
    const int64_t m = i / vpr;
    const int j = (int)(i - m * vpr) * V;
    hv v;
    if (j + V <= w) {
      v = *(const hv*)(src + m * lds + j);
      if (act != ACT_NONE) {
#pragma unroll
        for (int e = 0; e < V; ++e) v[e] = (half_t)apply_act((float)v[e], act);
      }
    } else if (act == ACT_NONE) {  // a raw 16-bit copy: any element type
#pragma unroll
      for (int e = 0; e < V; ++e) v[e] = j + e < w ? src[m * lds + j + e] : (half_t)0.f;
    } else {
#pragma unroll
      for (int e = 0; e < V; ++e) v[e] = j + e < w ? (half_t)apply_act((float)src[m * lds + j + e], act) : (half_t)0.f;
    }
    *(hv*)(dst + m * ldd + j) = v;
  }
}

hipError_t place_launch(int64_t M, const void* src, int64_t lds, int64_t w, void* dst, int64_t ldd, int64_t wpad,
                        int act, int num_cus, hipStream_t s) {
  if (M <= 0 || wpad <= 0) return hipSuccess;
  const bool vec = wpad % 8 == 0 && ldd % 8 == 0 && ((uintptr_t)dst & 15) == 0 &&
                   (w == 0 || (w % 8 == 0 && lds % 8 == 0 && ((uintptr_t)src & 15) == 0));
  const int V = vec ? 8 : 1;
  const int64_t want = (M * (wpad / V) + kStageThreads - 1) / kStageThreads, cap = (int64_t)num_cus * 16;
  const dim3 grid((unsigned)(want < cap ? want : cap)), block(kStageThreads);
  if (vec)
    hipLaunchKernelGGL(place_kernel<8>, grid, block, 0, s, (const half_t*)src, lds, (int)w, (half_t*)dst, ldd,
                       (int)wpad, act, M);
  else
    hipLaunchKernelGGL(place_kernel<1>, grid, block, 0, s, (const half_t*)src, lds, (int)w, (half_t*)dst, ldd,
                       (int)wpad, act, M);
  return hipGetLastError();
}

hipError_t add_launch(int64_t M, int64_t N, const void* a, const void* b, void* c, int num_cus, hipStream_t s) {
  hipLaunchKernelGGL(add_kernel, dim3(persistent_grid(M, num_cus, 4)), dim3(kStageThreads), 0, s, (const half_t*)a,
                     (const half_t*)b, (half_t*)c, M, (int)N);
  return hipGetLastError();
}

hipError_t concat_launch(int64_t M, int64_t N0, int64_t N1, const void* a, const void* b, void* c, int num_cus,
                         hipStream_t s) {
  hipLaunchKernelGGL(concat_kernel, dim3(persistent_grid(M, num_cus, 4)), dim3(kStageThreads), 0, s,
                     (const half_t*)a, (const half_t*)b, (half_t*)c, M, (int)N0, (int)N1);
  return hipGetLastError();
}

template <int ROUTE>
static int route_launch(int64_t M, const void* x, void* out, void* out2, int max_pipes, int dev, int num_cus,
                        hipStream_t s) {
  if (int rc = refuse_capture(s)) return rc;
  constexpr int S = route_stages(ROUTE);
  auto kern = route_kernel<ROUTE>;
  int per_cu = 0;
  hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, kStageThreads, 0);
  if (e != hipSuccess) return fail_hip(e, "occupancy query");
  int grid = per_cu * num_cus;
  if (max_pipes > 0) {
    // Workgroups are spread round-robin over the XCDs and a pipeline needs
    // all its workgroups on one XCD: launch whole rounds of kXcdHint * S.
    const int64_t rounds = (max_pipes + kXcdHint - 1) / kXcdHint;
    if (rounds * kXcdHint * S < grid) grid = (int)(rounds * kXcdHint * S);
  }
  if (grid < S) return fail(GP_ERR_NO_DEVICE, "not enough co-resident workgroups for a pipeline");
  const size_t bytes = sizeof(PipeCtl) + (size_t)(grid / S) * sizeof(RouteQueues);
  void* base = nullptr;
  uint32_t epoch = 0;
  const uint32_t layout = ROUTE == GP_ROUTE_RELOAD ? kArenaLayoutRouteReload : kArenaLayoutRoute + (ROUTE == GP_ROUTE_SPLIT);
  int rc = arena_acquire(dev, s, bytes, layout, &base, &epoch);
  if (rc != GP_OK) return rc;
  RouteArgs a;
  a.x = (const half_t*)x;
  a.out = (half_t*)out;
  a.out2 = (half_t*)out2;
  a.M = M;
  a.ctl = (PipeCtl*)base;
  a.queues = (RouteQueues*)((char*)base + sizeof(PipeCtl));
  a.ctx = QueueCtx{epoch, &a.ctl->err.v, (int)wait_limit(kQueueSpinLimit)};
  status_note(dev, s, &a.ctl->err.v, epoch);
  a.max_pipes = max_pipes;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(kStageThreads), 0, s, a);
  e = hipGetLastError();
  if (e != hipSuccess) return fail_hip(e, "route_kernel launch");
  return GP_OK;
}

int pipe_route_run(int64_t M, const void* x, void* out, void* out2, int route, int max_pipes, int dev, int num_cus,
                   hipStream_t s) {
  switch (route) {
    case GP_ROUTE_IDENT: return route_launch<GP_ROUTE_IDENT>(M, x, out, out2, max_pipes, dev, num_cus, s);
    case GP_ROUTE_BROADCAST: return route_launch<GP_ROUTE_BROADCAST>(M, x, out, out2, max_pipes, dev, num_cus, s);
    case GP_ROUTE_SPLIT: return route_launch<GP_ROUTE_SPLIT>(M, x, out, out2, max_pipes, dev, num_cus, s);
    case GP_ROUTE_DRAIN: return route_launch<GP_ROUTE_DRAIN>(M, x, out, out2, max_pipes, dev, num_cus, s);
    case GP_ROUTE_HANDOFF: return route_launch<GP_ROUTE_HANDOFF>(M, x, out, out2, max_pipes, dev, num_cus, s);
    case GP_ROUTE_RELOAD: return route_launch<GP_ROUTE_RELOAD>(M, x, out, out2, max_pipes, dev, num_cus, s);
    default: return fail(GP_ERR_INVALID_ARG, "unknown route %d", route);
  }
}

}  // namespace gp
