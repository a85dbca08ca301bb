// Stage-chained MeshGraphNet MLP: one workgroup per stage, stages linked by
// L2-resident ring queues -- the reference's pipelined form.
//
// Reference: apps/mgn_fullmlp/pipelined/mgn_fullmlp_pl.cuh:23-273 and
// apps/mgn_linears/pipelined/mgn_linears_pl.cuh:22-212.  The reference's
// pipeline is one block per layer plus LayerNorm workers:
//   X -> [Linear K->128 + ReLU] -q12-> [Linear + ReLU] -q23-> [Linear] -lnq-> 5 x [LayerNorm] -> out
// (mlp0_sm0 :83-101, mlp1_sm0 :146-160, mlp2_sm0 :162-181, ln_sm :183-203).
// That shape is kept as the split layout.  Layer 1 carries K/128 times the
// work of layers 2 and 3 (60% of the FLOPs at K = 384) and sets its pace
// (its K-split fix is disabled, :103-144).
//
// The default layout is built for MI355X:
//   X rows [0, 64)   -> [Linear K->128 + ReLU] -.
//                                               |-q12-> [Linear + ReLU, Linear (+ LN)] -> out
//   X rows [64, 128) -> [Linear K->128 + ReLU] -'
// * Two layer-1 workers per pipeline each take one 64-row half of every
//   128-row tile and write that half of the q12 entry (a row-split queue
//   writer: two producers per entry), so no partial sums pass through fp16
//   queues and layer 1's share of the work is split evenly.
// * Layers 2 and 3 (+ LayerNorm) run in one workgroup: layer 2's 128 x 128
//   result goes through LDS to layer 3 instead of through a queue.  A queue
//   hand-off costs a stage more per tile than a 128-wide layer's MFMAs do
//   (store completion, commit, the consumer's poll and its copy from L2).
// * Every stage fits in 80 KiB of LDS and 256 registers per wave, so two
//   stage workgroups share each CU: at one wave per SIMD a stage's epilogue
//   (LayerNorm, conversion, stores) and its waits leave the matrix core idle,
//   and the other workgroup's waves fill those cycles.
// * q12 is the only queue, and its lines are the only intermediate data
//   kept in L2.
// X tiles are copied with the non-temporal policy (stream-once input), so they
// do not evict the queues' lines from L2, and the output leaves in whole
// 256-byte rows with the non-temporal policy.
//
// MI355X: stage roles come from the XCD-aware assignment (pipeline.hpp), so
// every queue's producer and consumer share an L2; the grid is sized to the
// occupancy limit so that all workgroups are resident, as spin-waiting stages
// require (pipeline.hpp); pipelines take
// tiles g, g+P, ... of any M, with the partial last tile carried by the
// queue's row count.  Stage bodies are the library's stage functions.
#include <hip/hip_runtime.h>

#include "../../include/gpipes.h"
#include "gp_host.hpp"
#include "pipeline.hpp"
#include "stages.hpp"

namespace gp {
namespace mgnpl {

constexpr int MBLK = 128;
constexpr int D = 128;
constexpr int NLN = 5;  // LayerNorm workers per pipeline in the split layout (mgn_fullmlp_pl.cuh:28)
constexpr int kHalf = MBLK / 2;  // rows of a layer-1 worker's tile in the default layout

using QEntry = QueueEntry2D<MBLK, D>;

// Default layout: q12 with the two layer-1 workers as producers of every
// entry (row halves).  One slot: the consumer hands it back as soon as the
// tile is in its LDS, so the producers write the next tile while it computes.
// A slot that is rewritten within a tile's time stays in L2; with two slots
// each line waited two tiles, long enough for the X stream to evict about
// half of them dirty (WRITE_SIZE 406 MB per call against 276 MB, the output
// being 268 MB), and the call was 1-2% slower.
using HalfQueue = RingQueue<QEntry, 1, 2, 1>;
struct Queues {
  HalfQueue q12;
};

// Split layout: q12, q23 (qlen = 2, mgn_fullmlp_pl.cuh:32) and lnq
// (ln_qlen = n_ln_cols + 1, :33).
using Queue = RingQueue<QEntry, 2>;
using LnQueue = RingQueue<QEntry, NLN + 1>;
struct SplitQueues {
  Queue q12;
  Queue q23;
  LnQueue lnq;
};

// Split layout: the layer-1 block reads X through three 64-row part buffers
// (the copies of the next tile run under the MFMAs of the current one);
// layers 2 and 3 keep two 128-row tile buffers (a tile already in the queue
// is copied under the MFMAs of the one before it).
constexpr int kL1Bufs = 3;
constexpr int kQBufs = 4;

template <typename QS>
struct Args {
  MgnArgs m;
  PipeCtl* ctl;
  QS* queues;
  QueueCtx ctx;
};

// Default layout: stages 0, 1 = layer-1 workers (row halves), stage 2 = layers 2 + 3.
constexpr int kStages = 3;

template <int K, bool LN>
__global__ __launch_bounds__(kStageThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void mgn_pipelined_kernel(
    Args<Queues> a) {
  const Role r = assign_role(a.ctl, kStages, a.ctx);
  if (r.pipe < 0) return;
  const MgnArgs& m = a.m;
  Queues* qs = a.queues + r.pipe;
  const int64_t T = (m.M + MBLK - 1) / MBLK, NP = r.npipes, g = r.pipe;
  const int nt = g < T ? (int)((T - 1 - g) / NP + 1) : 0;
  NullReader ar;

  if (r.stage < 2) {
    // worker w: rows [64 w, 64 w + 64) of each of the pipeline's tiles
    // g, g + NP, ..., written to the same rows of the tile's q12 entry
    const int w = r.stage;
    const int64_t r0 = g * MBLK + w * kHalf;
    MemoryReader ir((half_t*)m.x + r0 * K, NP * MBLK * K, K, kHalf, m.M - r0, NP * MBLK);
    RowSplitQueueWriter<HalfQueue> ow(&qs->q12, &a.ctx, w, 2, m.M - g * MBLK, NP * MBLK);
    pipe_gemm_bias_relu<kHalf, K, 1>({(half_t*)m.w1, D, K}, {(half_t*)m.b1, 1, 1}, ir, ar, ow, nt);
  } else {
    // layers 2 and 3 (+ LayerNorm), layer 2's tile in LDS
    QueueReader<HalfQueue> ir(&qs->q12, &a.ctx);
    MemoryWriter ow((half_t*)m.out + g * MBLK * D, NP * MBLK * D, D);
    pipe_gemm_bias_relu_chain<MBLK, D, LN>({(half_t*)m.w2, D, D}, {(half_t*)m.b2, 1, 1}, {(half_t*)m.w3, D, D},
                                           {(half_t*)m.b3, 1, 1}, {(half_t*)m.gamma, 1, 1},
                                           {(half_t*)m.beta, 1, 1}, m.eps, ir, ar, ow, nt);
  }
}

// The reference's split layout: one layer-1 block, layer 2, layer 3, NLN
// LayerNorm workers.
constexpr int kSplitStages = 3 + NLN;

template <int K>
__global__ __launch_bounds__(kStageThreads) void mgn_split_kernel(Args<SplitQueues> a) {
  const Role r = assign_role(a.ctl, kSplitStages, a.ctx);
  if (r.pipe < 0) return;
  const MgnArgs& m = a.m;
  SplitQueues* qs = a.queues + r.pipe;
  const int64_t T = (m.M + MBLK - 1) / MBLK, NP = r.npipes, g = r.pipe;
  const int nt = g < T ? (int)((T - 1 - g) / NP + 1) : 0;
  NullReader ar;

  if (r.stage == 0) {
    MemoryReader ir((half_t*)m.x + g * MBLK * K, NP * MBLK * K, K, MBLK, m.M - g * MBLK, NP * MBLK);
    QueueWriter<Queue> ow(&qs->q12, &a.ctx);
    pipe_gemm_bias_relu<MBLK, K, kL1Bufs>({(half_t*)m.w1, D, K}, {(half_t*)m.b1, 1, 1}, ir, ar, ow, nt);
  } else if (r.stage == 1) {
    QueueReader<Queue> ir(&qs->q12, &a.ctx);
    QueueWriter<Queue> ow(&qs->q23, &a.ctx);
    pipe_gemm_bias_relu<MBLK, D, kQBufs>({(half_t*)m.w2, D, D}, {(half_t*)m.b2, 1, 1}, ir, ar, ow, nt);
  } else if (r.stage == 2) {
    QueueReader<Queue> ir(&qs->q23, &a.ctx);
    QueueWriter<LnQueue> ow(&qs->lnq, &a.ctx);
    pipe_gemm_bias<MBLK, D, kQBufs>({(half_t*)m.w3, D, D}, {(half_t*)m.b3, 1, 1}, ir, ar, ow, nt);
  } else {
    // LayerNorm worker w takes queue sequence numbers w, w + NLN, ...
    const int w = r.stage - 3;
    const int cnt = nt > w ? (nt - w + NLN - 1) / NLN : 0;
    SplitQueueReader<LnQueue> ir(&qs->lnq, &a.ctx, w, NLN);
    MemoryWriter ow((half_t*)m.out + (g + (int64_t)w * NP) * MBLK * D, (int64_t)NLN * NP * MBLK * D, D);
    pipe_layer_norm<MBLK, D>({(half_t*)m.gamma, 1, 1}, {(half_t*)m.beta, 1, 1}, ir, ow, cnt, m.eps);
  }
}

// Launch a pipelined kernel on a grid of `per CU` x CUs workgroups with its
// queues at the start of the stream's arena.
template <typename QS, typename KERN>
static int launch(KERN kern, int S, int lds, uint32_t layout, const MgnArgs& m, int dev, int num_cus, hipStream_t s) {
  if (int rc = refuse_capture(s)) return rc;
  hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
  if (e != hipSuccess) return fail_hip(e, "hipFuncSetAttribute");
  int per_cu = 0;
  e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, kStageThreads, lds);
  if (e != hipSuccess) return fail_hip(e, "occupancy query");
  const int grid = per_cu * num_cus;
  if (grid < S) return fail(GP_ERR_NO_DEVICE, "not enough co-resident workgroups for one pipeline");
  const size_t bytes = sizeof(PipeCtl) + (size_t)(grid / S) * sizeof(QS);
  void* base = nullptr;
  uint32_t epoch = 0;
  int rc = arena_acquire(dev, s, bytes, layout, &base, &epoch);
  if (rc != GP_OK) return rc;
  Args<QS> a;
  a.m = m;
  a.ctl = (PipeCtl*)base;
  a.queues = (QS*)((char*)base + sizeof(PipeCtl));
  a.ctx = QueueCtx{epoch, &a.ctl->err.v, (int)wait_limit(kQueueSpinLimit)};
  status_note(dev, s, &a.ctl->err.v, epoch);
  hipLaunchKernelGGL(kern, dim3(grid), dim3(kStageThreads), lds, s, a);
  e = hipGetLastError();
  if (e != hipSuccess) return fail_hip(e, "mgn_pipelined launch");
  return GP_OK;
}

template <int K>
static int run_k(const MgnArgs& m, bool split, int dev, int ncu, hipStream_t s) {
  if (split) {
    constexpr int l1 = gemm_stage_lds<MBLK, K, kL1Bufs>(), l23 = gemm_stage_lds<MBLK, D, kQBufs>();
    constexpr int lds = (l1 > l23 ? l1 : l23) + kGemmParamLds;
    return launch<SplitQueues>(mgn_split_kernel<K>, kSplitStages, lds, kArenaLayoutMgnSplit, m, dev, ncu, s);
  }
  constexpr int l1 = gemm_stage_lds<kHalf, K, 1>() + gemm_param_lds<kHalf>();
  constexpr int l23 = gemm_stage_lds<MBLK, D>() + gemm_chain_lds<MBLK>() + kGemmParamLds;
  constexpr int lds = l1 > l23 ? l1 : l23;
  static_assert(2 * lds <= 160 * 1024, "two stage workgroups per CU");
  if (m.gamma != nullptr)
    return launch<Queues>(mgn_pipelined_kernel<K, true>, kStages, lds, kArenaLayoutMgn, m, dev, ncu, s);
  return launch<Queues>(mgn_pipelined_kernel<K, false>, kStages, lds, kArenaLayoutMgn, m, dev, ncu, s);
}

}  // namespace mgnpl

int mgn_pipelined_run(const MgnArgs& a, bool split_ln, int dev, int num_cus, hipStream_t stream) {
  if (split_ln && a.gamma == nullptr) return fail(GP_ERR_INVALID_ARG, "the split-LayerNorm layout needs gamma/beta");
  switch (a.K) {
    case 384: return mgnpl::run_k<384>(a, split_ln, dev, num_cus, stream);
    case 256: return mgnpl::run_k<256>(a, split_ln, dev, num_cus, stream);
    case 128: return mgnpl::run_k<128>(a, split_ln, dev, num_cus, stream);
    default: return fail(GP_ERR_SHAPE, "K must be 128, 256 or 384");
  }
}

}  // namespace gp
