// Queue-chained NerfA trunk (the nerf_a app): one workgroup per stage, stages
// linked by L2-resident ring queues.
//
// Reference: apps/nerf_a/pipelined/nerf_a_pl.cuh:23-227 and the model
// apps/nerf_a/torch/model.py:5-38 (hidden 256, skip after the fifth layer):
//
//   x -[L1]-> q0 -[L2]-> q1 -[L3]-> q2 -[L4]-> q3 -[L5]-> q4 -[concat x]-> qc -[L6]-> q6 -[L7]-> q7 -[L8]-> out
//
// every Li being Linear + ReLU.  A stage workgroup computes 128 outputs, so
// each 256-wide layer is two workgroups that read the same input entry (two
// consumers) and write the two 128-column halves of the output entry (two
// producers).  The concat stage (concat0, nerf_a_pl.cuh:138-152) joins a queue
// tile with an input tile: pipe_concat fed from a queue.  Its 384-wide entry
// holds [h5 | x] in its first 256 + Kx columns; layer 6 reads it as a K = 384
// tile whose columns past 256 + Kx load as zeros.  Layer 1 reads x the same
// way, as a K = 128 tile of Kx valid columns.
//
// Not reproduced (a defect of the reference): its first layer uses a
// K = 256 block shape on the 64-wide input (nerf_a_pl.cuh:108); here each
// layer takes its real input width.
//
// 64-row tiles (the reference's mblk, nerf_a_pl.cuh:29) keep a stage's LDS at
// 52 KiB, so three stage workgroups share a CU.  Roles come from the XCD-aware
// assignment (pipeline.hpp).  Any M.
#include <hip/hip_runtime.h>

#include "../../include/gpipes.h"
#include "gp_host.hpp"
#include "pipeline.hpp"
#include "stages.hpp"

namespace gp {
namespace nerfa {

constexpr int MBLK = 64;
constexpr int W = 256;   // hidden width
constexpr int WC = 384;  // concat entry width: 256 + Kx <= 384

using E256 = QueueEntry2D<MBLK, W>;
using E384 = QueueEntry2D<MBLK, WC>;
using QH = RingQueue<E256, 2, 2, 2>;   // a layer's two halves -> the next layer's two halves
using QH1 = RingQueue<E256, 2, 2, 1>;  // layer 5's halves -> the concat stage
using QC = RingQueue<E384, 2, 1, 2>;   // concat -> layer 6's halves

struct Queues {
  QH q0, q1, q2, q3;
  QH1 q4;
  QC qc;
  QH q6, q7;
};

// Stages: layers 1-5 (two each), concat, layers 6-8 (two each).
constexpr int S = 2 * 5 + 1 + 2 * 3;

struct Args {
  NerfAArgs m;
  PipeCtl* ctl;
  Queues* queues;
  QueueCtx ctx;
};

// Linear + ReLU, output columns [128 j, 128 j + 128) of layer `li` (0-based).
template <int K, typename IR, typename OW>
__device__ __forceinline__ void half_layer(const NerfAArgs& m, int li, int j, int kvalid, IR& ir, OW& ow, int nt) {
  NullReader nr;
  const TensorView w{(half_t*)m.w[li] + 128 * j, W, kvalid};
  const TensorView b{m.b[li] ? (half_t*)m.b[li] + 128 * j : nullptr, 1, 1};
  // fragment prefetch depth 2: keeps the stage within three workgroups per CU
  pipe_gemm_bias_relu<MBLK, K, 0, 2>(w, b, ir, nr, ow, nt);
}

__global__ __launch_bounds__(kStageThreads) void nerf_a_pipelined_kernel(Args a) {
  const Role r = assign_role(a.ctl, S, a.ctx);
  if (r.pipe < 0) return;
  const NerfAArgs& m = a.m;
  Queues* qs = a.queues + r.pipe;
  const int64_t T = (m.M + MBLK - 1) / MBLK, NP = r.npipes, g = r.pipe;
  const int nt = g < T ? (int)((T - 1 - g) / NP + 1) : 0;
  const int Kx = (int)m.Kx;
  auto x_tiles = [&]() {
    return MemoryReader((half_t*)m.x + g * MBLK * Kx, NP * MBLK * Kx, Kx, MBLK, m.M - g * MBLK, NP * MBLK);
  };
  const int st = r.stage;
  const int j = st & 1;  // the output half of a layer stage

  if (st < 2) {  // layer 1: x (Kx columns) -> q0   (preskip0, nerf_a_pl.cuh:97-110)
    MemoryReader ir = x_tiles();
    QueueWriter<QH> ow(&qs->q0, &a.ctx, 128 * j);
    half_layer<128>(m, 0, j, Kx, ir, ow, nt);
  } else if (st < 8) {  // layers 2-4: q_{l-1} -> q_l   (preskip1-3, :122-132)
    QH* qin = st < 4 ? &qs->q0 : (st < 6 ? &qs->q1 : &qs->q2);
    QH* qout = st < 4 ? &qs->q1 : (st < 6 ? &qs->q2 : &qs->q3);
    QueueReader<QH> ir(qin, &a.ctx);
    QueueWriter<QH> ow(qout, &a.ctx, 128 * j);
    half_layer<W>(m, st / 2, j, W, ir, ow, nt);
  } else if (st < 10) {  // layer 5: q3 -> q4   (preskip4, :134-136)
    QueueReader<QH> ir(&qs->q3, &a.ctx);
    QueueWriter<QH1> ow(&qs->q4, &a.ctx, 128 * j);
    half_layer<W>(m, 4, j, W, ir, ow, nt);
  } else if (st == 10) {  // [h5 | x] -> qc   (concat0, :138-152)
    QueueReader<QH1> ir0(&qs->q4, &a.ctx);
    MemoryReader ir1 = x_tiles();
    QueueWriter<QC> ow(&qs->qc, &a.ctx);
    pipe_concat_n(ir0, ir1, ow, nt, W, Kx);
  } else if (st < 13) {  // layer 6: qc (256 + Kx columns) -> q6   (postskip0, :154-163)
    const int jj = (st - 11) & 1;
    QueueReader<QC> ir(&qs->qc, &a.ctx);
    QueueWriter<QH> ow(&qs->q6, &a.ctx, 128 * jj);
    half_layer<WC>(m, 5, jj, W + Kx, ir, ow, nt);
  } else if (st < 15) {  // layer 7: q6 -> q7   (postskip1, :165-167)
    const int jj = (st - 13) & 1;
    QueueReader<QH> ir(&qs->q6, &a.ctx);
    QueueWriter<QH> ow(&qs->q7, &a.ctx, 128 * jj);
    half_layer<W>(m, 6, jj, W, ir, ow, nt);
  } else {  // layer 8: q7 -> out columns [128 jj, 128 jj + 128)   (postskip2, :169-179)
    const int jj = (st - 15) & 1;
    QueueReader<QH> ir(&qs->q7, &a.ctx);
    MemoryWriter ow((half_t*)m.out + g * MBLK * W + 128 * jj, NP * MBLK * W, W);
    half_layer<W>(m, 7, jj, W, ir, ow, nt);
  }
}

}  // namespace nerfa

int nerf_a_pipelined_run(const NerfAArgs& m, int dev, int num_cus, hipStream_t s) {
  using namespace nerfa;
  if (int rc = refuse_capture(s)) return rc;
  if (m.Kx < 8 || m.Kx > 128 || m.Kx % 8)
    return fail(GP_ERR_SHAPE, "the pipelined layout takes Kx a multiple of 8 in [8, 128] (got %lld)",
                (long long)m.Kx);
  constexpr int lds = gemm_stage_lds<MBLK, WC>() + gemm_param_lds<MBLK>();
  auto kern = nerf_a_pipelined_kernel;
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
  int rc = arena_acquire(dev, s, bytes, kArenaLayoutNerfA, &base, &epoch);
  if (rc != GP_OK) return rc;
  Args a;
  a.m = m;
  a.ctl = (PipeCtl*)base;
  a.queues = (Queues*)((char*)base + sizeof(PipeCtl));
  a.ctx = QueueCtx{epoch, &a.ctl->err.v, (int)wait_limit(kQueueSpinLimit)};
  status_note(dev, s, &a.ctl->err.v, epoch);
  hipLaunchKernelGGL(kern, dim3(grid), dim3(kStageThreads), lds, s, a);
  e = hipGetLastError();
  if (e != hipSuccess) return fail_hip(e, "nerf_a pipelined launch");
  return GP_OK;
}

}  // namespace gp
