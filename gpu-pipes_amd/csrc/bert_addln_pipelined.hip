// Queue-chained add + LayerNorm + FFN block (the bert_addln_ffn app): one
// workgroup per stage, stages linked by L2-resident ring queues.
//
// Reference: apps/bert_addln_ffn/pipelined/bert_addln_ffn_pl.cuh:24-235 and the
// model apps/bert_addln_ffn/torch/model.py:3-20,
//   h0 = ln0(attn W0 + b0 + x),   out = ln2(W2 act(W1 h0 + b1) + b2 + h0),
// at the app's shape (H = 128, FF = 512).  Per pipeline of 128-row tiles:
//
//   attn -[W0+b0]-> q0 -[add x]-> q1 -[ln0]-> q2 --[W1 cols 0..127 + act]--.
//                                              |   [W1 cols 128..255]      |-> q3 -[W2+b2]-> q4 -[add q2]-> q5 -[ln2]-> out
//                                              |   [... 4 column slices]  -'                       ^
//                                              '------------------------------------------------------'
//
// * add0 (bert_addln_ffn_pl.cuh:103-111) adds a queue tile and an input tile,
//   add1 (:150-158) two queue tiles: pipe_add fed from queues.
// * q2 has five consumers (the four W1 column slices and add1), q3 four
//   producers that each write a 128-column block of a 512-wide entry -- the
//   MpmcRingQueue<E, N, NP, NC> roles of the reference (:54-57), here with the
//   FF-wide layer split by columns because a stage workgroup computes 128
//   outputs.  The reference computes it in one 512-wide block.
// * The W2 stage keeps all of W2 (K = 512) in registers.
// * Not reproduced (defects of the reference): its dispatcher never
//   reaches ln0 (:227 subtracts where it should add), ln2 reads q3 instead of
//   the queue of add1 (:167), and its extension passes be0 for be2 (_ext.cu:71).
//   Here ln0 runs on add0's output, ln2 on add1's, each with its own affine.
//
// Roles come from the XCD-aware assignment (pipeline.hpp): every queue's
// producers and consumers share an L2.  Any M: the partial last tile is
// carried by the queues' row counts.
#include <hip/hip_runtime.h>

#include "../../include/gpipes.h"
#include "gp_host.hpp"
#include "pipeline.hpp"
#include "stages.hpp"

namespace gp {
namespace addln {

constexpr int MBLK = 128;
constexpr int H = 128;
constexpr int FF = 512;
constexpr int NF1 = FF / 128;  // column slices of the FF-wide layer
constexpr int NL0 = 1;         // LayerNorm workers (split queue readers) of ln0
constexpr int NL2 = 1;         // and of ln2

using E128 = QueueEntry2D<MBLK, H>;
using E512 = QueueEntry2D<MBLK, FF>;
using Q0 = RingQueue<E128, 2>;                // W0 stage -> add0
using Q1 = RingQueue<E128, NL0 + 1>;          // add0 -> ln0 workers
using Q2 = RingQueue<E128, 8, 1, NF1 + 1>;    // ln0 -> the W1 slices and add1 (deep: add1 reads late)
using Q3 = RingQueue<E512, 2, NF1, 1>;        // the W1 slices -> W2 stage
using Q4 = RingQueue<E128, 2>;                // W2 stage -> add1
using Q5 = RingQueue<E128, NL2 + 1>;          // add1 -> ln2 workers

struct Queues {
  Q0 q0;
  Q1 q1;
  Q2 q2;
  Q3 q3;
  Q4 q4;
  Q5 q5;
};

// Stages of a pipeline: W0, add0, ln0 x NL0, W1 x NF1, W2, add1, ln2 x NL2.
constexpr int S = 4 + NL0 + NF1 + NL2;

struct Args {
  BertAddlnArgs m;
  PipeCtl* ctl;
  Queues* queues;
  QueueCtx ctx;
};

__device__ __forceinline__ TensorView vec(const void* p) { return {(half_t*)p, 1, 1}; }

template <int ACT>
__global__ __launch_bounds__(kStageThreads) void bert_addln_pipelined_kernel(Args a) {
  const Role r = assign_role(a.ctl, S, a.ctx);
  if (r.pipe < 0) return;
  const BertAddlnArgs& m = a.m;
  Queues* qs = a.queues + r.pipe;
  const int64_t T = (m.M + MBLK - 1) / MBLK, NP = r.npipes, g = r.pipe;
  const int nt = g < T ? (int)((T - 1 - g) / NP + 1) : 0;
  // This pipeline's tiles g, g + NP, ... of a row-major [M][H] input.
  auto tiles_of = [&](const void* base) {
    return MemoryReader((half_t*)base + g * MBLK * H, NP * MBLK * H, H, MBLK, m.M - g * MBLK, NP * MBLK);
  };
  NullReader nr;
  int st = r.stage;

  if (st == 0) {  // y0 = attn W0 + b0   (lin_attn_out, bert_addln_ffn_pl.cuh:92-101)
    MemoryReader ir = tiles_of(m.attn);
    QueueWriter<Q0> ow(&qs->q0, &a.ctx);
    // four 64-row part buffers (within the W2 stage's LDS): the next tile's
    // copies run under this tile's MFMAs
    pipe_gemm_bias<MBLK, H, 4>({(half_t*)m.w0, H, H}, vec(m.b0), ir, nr, ow, nt);
    return;
  }
  if (st == 1) {  // y0 + x   (add0, :103-111)
    QueueReader<Q0> ir0(&qs->q0, &a.ctx);
    MemoryReader ir1 = tiles_of(m.x);
    QueueWriter<Q1> ow(&qs->q1, &a.ctx);
    pipe_add<MBLK, H>(ir0, ir1, ow, nt);
    return;
  }
  st -= 2;
  if (st < NL0) {  // h0 = ln0(y0 + x), worker st of NL0   (ln0, :113-125)
    const int cnt = nt > st ? (nt - st + NL0 - 1) / NL0 : 0;
    SplitQueueReader<Q1> ir(&qs->q1, &a.ctx, st, NL0);
    SplitQueueWriter<Q2> ow(&qs->q2, &a.ctx, st, NL0);
    pipe_layer_norm<MBLK, H>(vec(m.ga0), vec(m.be0), ir, ow, cnt, m.eps);
    return;
  }
  st -= NL0;
  if (st < NF1) {  // act(h0 W1 + b1), output columns [128 st, 128 st + 128)   (y1w1_relu, :128-137)
    QueueReader<Q2> ir(&qs->q2, &a.ctx);
    QueueWriter<Q3> ow(&qs->q3, &a.ctx, 128 * st);
    // two tile buffers: a tile already in the queue is copied under the MFMAs
    pipe_gemm_bias_act<MBLK, H, ACT, 4>({(half_t*)m.w1 + 128 * st, FF, H},
                                         vec(m.b1 ? (const half_t*)m.b1 + 128 * st : nullptr), ir, nr, ow, nt);
    return;
  }
  st -= NF1;
  if (st == 0) {  // a W2 + b2, K = 512   (y2w2, :139-148)
    QueueReader<Q3> ir(&qs->q3, &a.ctx);
    QueueWriter<Q4> ow(&qs->q4, &a.ctx);
    pipe_gemm_bias<MBLK, FF>({(half_t*)m.w2, H, FF}, vec(m.b2), ir, nr, ow, nt);
    return;
  }
  if (st == 1) {  // ffn(h0) + h0   (add1, :150-158)
    QueueReader<Q4> ir0(&qs->q4, &a.ctx);
    QueueReader<Q2> ir1(&qs->q2, &a.ctx);
    QueueWriter<Q5> ow(&qs->q5, &a.ctx);
    pipe_add<MBLK, H>(ir0, ir1, ow, nt);
    return;
  }
  st -= 2;
  if (st < NL2) {  // out = ln2(...), worker st of NL2 writes tiles st, st + NL2, ...   (ln2, :161-176)
    const int cnt = nt > st ? (nt - st + NL2 - 1) / NL2 : 0;
    SplitQueueReader<Q5> ir(&qs->q5, &a.ctx, st, NL2);
    MemoryWriter ow((half_t*)m.out + (g + (int64_t)st * NP) * MBLK * H, (int64_t)NL2 * NP * MBLK * H, H);
    pipe_layer_norm<MBLK, H>(vec(m.ga2), vec(m.be2), ir, ow, cnt, m.eps);
  }
}

template <int ACT>
static int run(const BertAddlnArgs& m, int dev, int num_cus, hipStream_t s) {
  if (int rc = refuse_capture(s)) return rc;
  static_assert(gemm_stage_lds<MBLK, H, 4>() <= gemm_stage_lds<MBLK, FF>(), "W0's part buffers fit the W2 stage's LDS");
  constexpr int lds = gemm_stage_lds<MBLK, FF>() + gemm_param_lds<MBLK>();
  auto kern = bert_addln_pipelined_kernel<ACT>;
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
  int rc = arena_acquire(dev, s, bytes, kArenaLayoutBertAddln, &base, &epoch);
  if (rc != GP_OK) return rc;
  Args a;
  a.m = m;
  a.ctl = (PipeCtl*)base;
  a.queues = (Queues*)((char*)base + sizeof(PipeCtl));
  a.ctx = QueueCtx{epoch, &a.ctl->err.v, (int)wait_limit(kQueueSpinLimit)};
  status_note(dev, s, &a.ctl->err.v, epoch);
  hipLaunchKernelGGL(kern, dim3(grid), dim3(kStageThreads), lds, s, a);
  e = hipGetLastError();
  if (e != hipSuccess) return fail_hip(e, "bert_addln pipelined launch");
  return GP_OK;
}

}  // namespace addln

int bert_addln_pipelined_run(const BertAddlnArgs& a, int dev, int num_cus, hipStream_t stream) {
  if (a.H != addln::H || a.FF != addln::FF)
    return fail(GP_ERR_SHAPE, "the pipelined layout is built for the app's shape H = 128, FF = 512 (got %lld, %lld)",
                (long long)a.H, (long long)a.FF);
  switch (a.act) {
    case GP_ACT_RELU: return addln::run<ACT_RELU>(a, dev, num_cus, stream);
    case GP_ACT_GELU_TANH: return addln::run<ACT_GELU_TANH>(a, dev, num_cus, stream);
    default: return fail(GP_ERR_INVALID_ARG, "the pipelined layout supports ReLU and GELU(tanh) only");
  }
}

}  // namespace gp
