// Queue-chained BERT FFN block (the bert_ffn app): one workgroup per stage,
// stages linked by L2-resident ring queues.
//
// Reference: apps/bert_ffn/pipelined/bert_ffn_pl.cuh:79-162 and the model
// apps/bert_ffn/torch/model.py:3-14,
//   out = LayerNorm(act(x W1 + b1) W2 + b2 + x) * gamma + beta,
// at the app's shape (H = 128, FF = 512).  Per pipeline of 128-row tiles:
//
//   x --[W1 cols 0..127 + b1, act]---.
//     --[W1 cols 128..255 ...]      |-> q1 (512 wide) -> 2 x [W2 + b2 + x, LayerNorm] -> out
//     --[... 4 column slices]      -'
//
// * The reference's linear0 computes the 512-wide layer in one block
//   (:80-89); a stage workgroup here computes 128 outputs, so four workers
//   each write a 128-column block of every q1 entry (MpmcRingQueue with four
//   producers, as q3 of the bert_addln layout).
// * The reference's linear1 adds x as an accumulator tile (:91-101) and its
//   LayerNorm workers (:103-118) read linear1's queue; here the residual tile
//   enters the same way (the GEMM stage's accumulator reader) and the
//   LayerNorm runs in the W2 stage's epilogue, so no queue carries the
//   pre-LayerNorm rows.  The W2 stage (K = 512, all of W2 in registers) has
//   four times a W1 slice's work: two W2 workers take q1's entries round
//   robin (split queue reader), each writing its tiles to memory.
//
// Roles come from the XCD-aware assignment (pipeline.hpp): every queue's
// producers and consumers share an L2.  Any M: the partial last tile is
// carried by the queue's row counts.
#include <hip/hip_runtime.h>

#include "../../include/gpipes.h"
#include "gp_host.hpp"
#include "pipeline.hpp"
#include "stages.hpp"

namespace gp {
namespace bffn {

constexpr int MBLK = 128;
constexpr int H = 128;
constexpr int FF = 512;
constexpr int NF1 = FF / 128;  // column slices of the FF-wide layer
constexpr int NW2 = 2;         // W2 + LayerNorm workers

using E512 = QueueEntry2D<MBLK, FF>;
using Q1 = RingQueue<E512, NW2 + 1, NF1, 1>;  // the W1 slices -> the W2 workers

struct Queues {
  Q1 q1;
};

// Stages of a pipeline: W1 x NF1, W2 x NW2.
constexpr int S = NF1 + NW2;

struct Args {
  BertFfnArgs m;
  PipeCtl* ctl;
  Queues* queues;
  QueueCtx ctx;
};

__device__ __forceinline__ TensorView vec(const void* p) { return {(half_t*)p, 1, 1}; }

template <int ACT>
__global__ __launch_bounds__(kStageThreads) void bert_ffn_pipelined_kernel(Args a) {
  const Role r = assign_role(a.ctl, S, a.ctx);
  if (r.pipe < 0) return;
  const BertFfnArgs& m = a.m;
  Queues* qs = a.queues + r.pipe;
  const int64_t T = (m.M + MBLK - 1) / MBLK, NP = r.npipes, g = r.pipe;
  const int nt = g < T ? (int)((T - 1 - g) / NP + 1) : 0;
  NullReader nr;
  const int st = r.stage;

  if (st < NF1) {  // act(x W1 + b1), output columns [128 st, 128 st + 128)   (linear0, bert_ffn_pl.cuh:80-89)
    MemoryReader ir((half_t*)m.x + g * MBLK * H, NP * MBLK * H, H, MBLK, m.M - g * MBLK, NP * MBLK);
    QueueWriter<Q1> ow(&qs->q1, &a.ctx, 128 * st);
    // four 64-row part buffers: the next tile's copies run under this tile's MFMAs
    pipe_gemm_bias_act<MBLK, H, ACT, 4>({(half_t*)m.w1 + 128 * st, FF, H},
                                         vec(m.b1 ? (const half_t*)m.b1 + 128 * st : nullptr), ir, nr, ow, nt);
    return;
  }
  // LayerNorm(q1 W2 + b2 + x), worker w of NW2 takes the pipeline's tiles w,
  // w + NW2, ...   (linear1 :91-101 with ln_sm :103-118)
  const int w = st - NF1;
  const int cnt = nt > w ? (nt - w + NW2 - 1) / NW2 : 0;
  const int64_t first = g + (int64_t)w * NP;  // this worker's first tile
  SplitQueueReader<Q1> ir(&qs->q1, &a.ctx, w, NW2);
  MemoryReader xr((half_t*)m.x + first * MBLK * H, NW2 * NP * MBLK * H, H, MBLK, m.M - first * MBLK,
                  NW2 * NP * MBLK);
  MemoryWriter ow((half_t*)m.out + first * MBLK * H, (int64_t)NW2 * NP * MBLK * H, H);
  pipe_gemm_bias_layer_norm<MBLK, FF>({(half_t*)m.w2, H, FF}, vec(m.b2), vec(m.gamma), vec(m.beta), m.eps, ir, xr,
                                      ow, cnt);
}

template <int ACT>
static int run(const BertFfnArgs& m, int dev, int num_cus, hipStream_t s) {
  if (int rc = refuse_capture(s)) return rc;
  static_assert(gemm_stage_lds<MBLK, H, 4>() <= gemm_stage_lds<MBLK, FF>(), "W1's part buffers fit the W2 stage's LDS");
  constexpr int lds = gemm_stage_lds<MBLK, FF>() + gemm_param_lds<MBLK>();
  auto kern = bert_ffn_pipelined_kernel<ACT>;
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
  int rc = arena_acquire(dev, s, bytes, kArenaLayoutBertFfn, &base, &epoch);
  if (rc != GP_OK) return rc;
  Args a;
  a.m = m;
  a.ctl = (PipeCtl*)base;
  a.queues = (Queues*)((char*)base + sizeof(PipeCtl));
  a.ctx = QueueCtx{epoch, &a.ctl->err.v, (int)wait_limit(kQueueSpinLimit)};
  status_note(dev, s, &a.ctl->err.v, epoch);
  hipLaunchKernelGGL(kern, dim3(grid), dim3(kStageThreads), lds, s, a);
  e = hipGetLastError();
  if (e != hipSuccess) return fail_hip(e, "bert_ffn pipelined launch");
  return GP_OK;
}

}  // namespace bffn

int bert_ffn_pipelined_run(const BertFfnArgs& a, int dev, int num_cus, hipStream_t stream) {
  if (a.H != bffn::H || a.FF != bffn::FF)
    return fail(GP_ERR_SHAPE, "the pipelined layout is built for the app's shape H = 128, FF = 512 (got %lld, %lld)",
                (long long)a.H, (long long)a.FF);
  switch (a.act) {
    case GP_ACT_RELU: return bffn::run<ACT_RELU>(a, dev, num_cus, stream);
    case GP_ACT_GELU_TANH: return bffn::run<ACT_GELU_TANH>(a, dev, num_cus, stream);
    default: return fail(GP_ERR_INVALID_ARG, "the pipelined layout supports ReLU and GELU(tanh) only");
  }
}

}  // namespace gp
