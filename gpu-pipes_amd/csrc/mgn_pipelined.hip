// Stage-chained MeshGraphNet MLP: one workgroup per stage, stages linked by
// L2-resident ring queues -- the reference's pipelined form.
//
// Reference: apps/mgn_fullmlp/pipelined/mgn_fullmlp_pl.cuh:23-273 and
// apps/mgn_linears/pipelined/mgn_linears_pl.cuh:22-212.  Per pipeline:
//   X -> 3 x [Linear K->128 + ReLU] -q12-> [Linear + ReLU] -q23-> [Linear (+ LN)] -> out
// Layer 1 carries K/128 times the work of layers 2 and 3 (60% of the FLOPs at
// K = 384), which sets the reference's pipeline pace (one block per stage,
// mgn_fullmlp_pl.cuh:83-101; its K-split fix is disabled, :103-144).  Here two
// layer-1 workers (for K > 128) take the pipeline's tiles round robin and
// write q12 through a split queue writer, so no partial sums pass through fp16
// queues.  A stage's time per tile is mostly fixed cost (queue hand-offs, the
// tile copy, store completion), so more workers per pipeline mean fewer
// pipelines: at K = 384 two workers measured 0.41 ms, one 0.54 ms and three
// 0.53 ms per call.  The split layout keeps the reference's shape, one
// layer-1 block and five LayerNorm workers:
//   X -> [Linear K->128 + ReLU] -q12-> [Linear] -q23-> [Linear] -lnq-> 5 x [LayerNorm] -> out
// (mlp0_sm0 :83-101, mlp1_sm0 :146-160, mlp2_sm0 :162-181, ln_sm :183-203).
// X tiles are copied with the non-temporal policy (stream-once input), so they
// do not evict the queues' lines from L2.
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

using QEntry = QueueEntry2D<MBLK, D>;
using Queue = RingQueue<QEntry, 2>;              // q23 (qlen = 2, mgn_fullmlp_pl.cuh:32); q12 with one writer
// q12, written round robin by the layer-1 workers.  Two slots: a deeper q12
// was no faster and kept more queue lines in L2, so more of them were written
// back to HBM (WRITE_SIZE 575 MiB per call with four slots, 440 with two).
using Queue1 = RingQueue<QEntry, 2>;
using LnQueue = RingQueue<QEntry, NLN + 1>;      // lnq (ln_qlen = n_ln_cols + 1, :33)

struct Queues {
  Queue1 q12;
  Queue q23;
  LnQueue lnq;
};

// Layer-1 workers read X through three 64-row part buffers, so the copies of
// the next tile (from HBM) run under the MFMAs of the current one.
constexpr int kL1Bufs = 3;
// Layers 2 and 3 keep two 128-row tile buffers: a tile that is already in
// the queue is copied under the MFMAs of the one before it.
constexpr int kQBufs = 4;

// Layer-1 workers per pipeline: 2 for K > 128 (1 in the reference's split layout).
template <int K, bool SPLIT>
constexpr int layer1_workers() {
  return SPLIT ? 1 : (K > 128 ? 2 : 1);
}

struct Args {
  MgnArgs m;
  PipeCtl* ctl;
  Queues* queues;
  QueueCtx ctx;
};

template <int K, bool LN, bool SPLIT>
__global__ __launch_bounds__(kStageThreads) void mgn_pipelined_kernel(Args a) {
  constexpr int W1 = layer1_workers<K, SPLIT>();
  constexpr int S = W1 + (SPLIT ? 2 + NLN : 2);
  const Role r = assign_role(a.ctl, S, a.ctx);
  if (r.pipe < 0) return;
  const MgnArgs& m = a.m;
  Queues* qs = a.queues + r.pipe;
  const int64_t T = (m.M + MBLK - 1) / MBLK, NP = r.npipes, g = r.pipe;
  const int nt = g < T ? (int)((T - 1 - g) / NP + 1) : 0;
  half_t* out = (half_t*)m.out;
  const TensorView gamma{(half_t*)m.gamma, 1, 1}, beta{(half_t*)m.beta, 1, 1};
  NullReader ar;

  if (r.stage < W1) {
    // layer-1 worker w takes the pipeline's tiles w, w + W1, ... (global tiles
    // g + (w + i W1) NP) and writes them to q12 in sequence order
    const int w = r.stage;
    const int cnt = nt > w ? (nt - w + W1 - 1) / W1 : 0;
    const int64_t first = g + (int64_t)w * NP;
    MemoryReader ir((half_t*)m.x + first * MBLK * K, W1 * NP * MBLK * K, K, MBLK, m.M - first * MBLK,
                    W1 * NP * MBLK);
    SplitQueueWriter<Queue1> ow(&qs->q12, &a.ctx, w, W1);
    pipe_gemm_bias_relu<MBLK, K, kL1Bufs>({(half_t*)m.w1, D, K}, {(half_t*)m.b1, 1, 1}, ir, ar, ow, cnt);
  } else if (r.stage == W1) {
    QueueReader<Queue1> ir(&qs->q12, &a.ctx);
    QueueWriter<Queue> ow(&qs->q23, &a.ctx);
    pipe_gemm_bias_relu<MBLK, D, kQBufs>({(half_t*)m.w2, D, D}, {(half_t*)m.b2, 1, 1}, ir, ar, ow, nt);
  } else if (r.stage == W1 + 1) {
    QueueReader<Queue> ir(&qs->q23, &a.ctx);
    const TensorView w3{(half_t*)m.w3, D, D}, b3{(half_t*)m.b3, 1, 1};
    if constexpr (SPLIT) {
      QueueWriter<LnQueue> ow(&qs->lnq, &a.ctx);
      pipe_gemm_bias<MBLK, D, kQBufs>(w3, b3, ir, ar, ow, nt);
    } else {
      MemoryWriter ow(out + g * MBLK * D, NP * MBLK * D, D);
      if constexpr (LN) pipe_gemm_bias_layer_norm<MBLK, D, kQBufs>(w3, b3, gamma, beta, m.eps, ir, ar, ow, nt);
      else pipe_gemm_bias<MBLK, D, kQBufs>(w3, b3, ir, ar, ow, nt);
    }
  } else if constexpr (SPLIT) {
    // LayerNorm worker w takes queue sequence numbers w, w + NLN, ...
    const int w = r.stage - W1 - 2;
    const int cnt = nt > w ? (nt - w + NLN - 1) / NLN : 0;
    SplitQueueReader<LnQueue> ir(&qs->lnq, &a.ctx, w, NLN);
    MemoryWriter ow(out + (g + (int64_t)w * NP) * MBLK * D, (int64_t)NLN * NP * MBLK * D, D);
    pipe_layer_norm<MBLK, D>(gamma, beta, ir, ow, cnt, m.eps);
  }
}

template <int K, bool LN, bool SPLIT>
static int run(const MgnArgs& m, int dev, int num_cus, hipStream_t s) {
  if (int rc = refuse_capture(s)) return rc;
  constexpr int S = layer1_workers<K, SPLIT>() + (SPLIT ? 2 + NLN : 2);
  constexpr int l1 = gemm_stage_lds<MBLK, K, kL1Bufs>(), l23 = gemm_stage_lds<MBLK, D, kQBufs>();
  constexpr int lds = (l1 > l23 ? l1 : l23) + kGemmParamLds;
  auto kern = mgn_pipelined_kernel<K, LN, SPLIT>;
  hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
  if (e != hipSuccess) return fail_hip(e, "hipFuncSetAttribute");
  int per_cu = 0;
  e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, kStageThreads, lds);
  if (e != hipSuccess) return fail_hip(e, "occupancy query");
  const int grid = per_cu * num_cus;
  if (grid < S) return fail(GP_ERR_NO_DEVICE, "not enough co-resident workgroups for one pipeline");
  const size_t bytes = sizeof(PipeCtl) + (size_t)(grid / S) * sizeof(Queues);
  void* base = nullptr;
  uint32_t epoch = 0;
  int rc = arena_acquire(dev, s, bytes, kArenaLayoutMgn, &base, &epoch);
  if (rc != GP_OK) return rc;
  Args a;
  a.m = m;
  a.ctl = (PipeCtl*)base;
  a.queues = (Queues*)((char*)base + sizeof(PipeCtl));
  a.ctx = QueueCtx{epoch, &a.ctl->err.v, (int)wait_limit(kQueueSpinLimit)};
  status_note(dev, s, &a.ctl->err.v, epoch);
  hipLaunchKernelGGL(kern, dim3(grid), dim3(kStageThreads), lds, s, a);
  e = hipGetLastError();
  if (e != hipSuccess) return fail_hip(e, "mgn_pipelined launch");
  return GP_OK;
}

template <int K>
static int run_k(const MgnArgs& m, bool split, int dev, int ncu, hipStream_t s) {
  const bool ln = m.gamma != nullptr;
  if (split) return run<K, true, true>(m, dev, ncu, s);
  return ln ? run<K, true, false>(m, dev, ncu, s) : run<K, false, false>(m, dev, ncu, s);
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
