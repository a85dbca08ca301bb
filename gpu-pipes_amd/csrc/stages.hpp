// Pipeline stage functions for gfx950 (workgroup-collective device functions).
//
// Reference stages: common/pipe_gemm_bias_relu.cuh:85-192,
// common/pipe_gemm_bias.cuh:85-191, common/pipe_gemm.cuh:78-183 (GEMM with an
// accumulator tile from an AccumReader), common/pipe_gemm_bias_layer_norm.cuh:
// 100-249 (GEMM + bias then LayerNorm in the same block), common/
// pipe_layer_norm.cuh:13-60 + common/layer_norm_v2.cuh:16-73 (LayerNorm),
// common/pipe_add.cuh:13-40 and common/pipe_concat.cuh:48-74.  Each stage
// keeps the reference's calling convention -- (weights, bias, input reader,
// accumulator reader, output writer, num_iters) -- and loops acquire /
// compute / release over its tiles.
//
// MI355X implementation: a stage runs in a workgroup of 256 threads (four
// wave64s).  GEMM stages keep the whole weight matrix resident in registers
// for all tiles (the reference re-streams it through shared memory for every
// tile, pipe_gemm_bias_relu.cuh:119-124): wave w owns output features
// [32w, 32w+32) and holds W[:, 32w:32w+32]^T as MFMA A fragments; input
// tiles are copied into LDS with buffer_load ... lds (XOR-swizzled rows, rows
// past the tile's valid count zero-filled) and multiplied with
// v_mfma_f32_32x32x16_f16, accumulating in fp32 (the reference accumulates in
// fp16, pipe_gemm_bias_relu.cuh:43).  The bias is the accumulator's initial
// value, the activation / LayerNorm are applied in the epilogue.
//
// Dynamic LDS: every stage uses the kernel's dynamic shared memory from
// offset 0; stage_lds_bytes<...>() gives the requirement.
#pragma once

#include <type_traits>

#include "gp_device.hpp"
#include "pipes.hpp"

namespace gp {

enum Act : int { ACT_NONE = 0, ACT_RELU = 1, ACT_GELU_TANH = 2, ACT_SIGMOID = 3 };

// GELU with the tanh approximation, 0.5 v (1 + tanh(u)), u = sqrt(2/pi)(v + 0.044715 v^3),
// evaluated through the identity 0.5 (1 + tanh(u)) = 1 / (1 + e^(-2u)):
//   v / (1 + 2^(v (c0 + c1 v^2))),  c0 = -2 sqrt(2/pi) log2(e),  c1 = 0.044715 c0,
// five VALU operations and two transcendentals (v_exp_f32, v_rcp_f32).  For
// v -> -inf the power overflows to +inf and the result is -0; for v -> +inf it
// is v.  Relative error is a few ulp of fp32.
__device__ __forceinline__ float gelu_tanh(float v) {
  constexpr float c0 = -2.f * 0.7978845608028654f * 1.4426950408889634f;
  constexpr float c1 = 0.044715f * c0;
  const float z = v * __builtin_fmaf(c1, v * v, c0);
  return v * __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(z));
}

// Logistic sigmoid 1 / (1 + e^(-v)) with e^(-v) = 2^(-v log2(e)): one
// multiply, v_exp_f32, one add and v_rcp_f32.  For v -> -inf the power
// overflows to +inf and the result is 0; for v -> +inf it is 1.  Relative
// error is a few ulp of fp32, far below the fp16 rounding of the output.
__device__ __forceinline__ float sigmoid(float v) {
  return __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(v * -1.4426950408889634f));
}

__device__ __forceinline__ float apply_act(float v, int act) {
  if (act == ACT_RELU) return v > 0.f ? v : 0.f;
  if (act == ACT_GELU_TANH) return gelu_tanh(v);
  if (act == ACT_SIGMOID) return sigmoid(v);
  return v;
}

__device__ __forceinline__ GP_LDS char* dyn_lds() {
  extern __shared__ __attribute__((aligned(1024))) char gp_dyn_smem[];
  return (GP_LDS char*)gp_dyn_smem;
}

constexpr int kStageThreads = 256;

// LDS bytes of a GEMM stage with an MBLK x K input tile and N = 128 outputs.
// NB > 0: the input is staged through NB buffers of 64 rows (at least
// MBLK / 64 of them), so the next tile's copies overlap this tile's MFMAs.
template <int MBLK, int K, int NB = 0>
constexpr int gemm_stage_lds() {
  constexpr int rows = (NB > MBLK / 64 ? NB : MBLK / 64) * 64;
  constexpr int tile = (NB > 0 ? rows : MBLK) * K * 2;
  return tile > 64 * 256 ? tile : 64 * 256;  // at least one 64-row pass of weight staging
}
// bias/gamma/beta + the LayerNorm partials of MBLK rows
template <int MBLK>
constexpr int gemm_param_lds() {
  return 3 * 128 * 4 + MBLK * 4 * 8;
}
constexpr int kGemmParamLds = gemm_param_lds<128>();
// Extra LDS of a stage that chains a second 128 -> 128 layer: the first
// layer's MBLK x 128 fp16 output tile and the second layer's bias.
template <int MBLK>
constexpr int gemm_chain_lds() {
  return MBLK * 128 * 2 + 128 * 4;
}

// Copy rows [0, MBLK) x K halves of a tile view into LDS.  LDS row r holds
// 16-byte chunk c at chunk position (c & ~15) | ((c ^ r) & 15), so the 16
// rows read by one ds_read_b128 phase hit 16 different bank groups.  Rows at
// or past v.rows lie outside the buffer descriptor and arrive as zeros, and so
// do columns at or past kv (a multiple of 8): a narrower input (a 64-wide
// NeRF encoding, a 320-wide concatenation) runs as a K-wide tile whose extra
// columns are zero, never the next row's data.
// NT: copy with the non-temporal cache policy -- for an input streamed from
// memory once, so that it does not evict the L2 lines of the ring queues;
// otherwise the tile is a queue payload, copied with the agent-scope policy
// (kQueueLoadAux: read from L2, never from a stale L1 line).
template <int MBLK, int K, bool NT = false>
__device__ __forceinline__ void load_tile_swz(const TensorView& v, GP_LDS char* dst, int kv = K) {
  static_assert(K % 128 == 0, "K must be a multiple of 128");
  constexpr int CPR = K / 8;
  constexpr int NI = MBLK * K * 2 / 1024;
  static_assert(NI % 4 == 0, "tile must split over four waves");
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int rows = v.rows < MBLK ? (v.rows > 0 ? v.rows : 0) : MBLK;
  const __amdgpu_buffer_rsrc_t rsrc = make_rsrc(v.data, rows * v.stride * 2);
#pragma unroll
  for (int ii = 0; ii < NI / 4; ++ii) {
    const int i = ii * 4 + wave;
    const int q = i * kWave + lane;
    const int r = q / CPR;
    const int c = (q - r * CPR) ^ (r & 15);
    const int off = c * 8 < kv ? r * v.stride * 2 + c * 16 : (int)0x7FFFFFF0;
    if constexpr (NT)
      dma16_buf_nt(rsrc, off, dst + i * 1024);
    else
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, dst + i * 1024, 16, off, 0, 0, kQueueLoadAux);
  }
}

// Load a weight matrix W [K][128] (row stride w.stride elements) into MFMA A
// fragments: wf[s] of wave w, lane l holds W[16s + 8(l/32) + e][32w + l%32].
// W is copied into the LDS scratch (SCR bytes) in its own row-major shape --
// whole 1 KiB copies, the staged-rows layout of gp_device.hpp -- as many
// 64-row groups at a time as fit, and the fragments, columns of W, are read
// with the transposing ds_read_b64_tr_b16.  Rows at or past w.rows (the valid
// K of a padded layer) lie outside the copies' buffer descriptor and arrive
// as zeros.
template <int K, int SCR>
__device__ __forceinline__ void load_weight_frags(const TensorView& w, GP_LDS char* scratch, h8 (&wf)[K / 16]) {
  constexpr int RP0 = SCR / 256 / 64 * 64;
  constexpr int RP = RP0 < K ? RP0 : K;  // rows per pass
  static_assert(RP >= 64, "the scratch must hold 64 weight rows");
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int lh = lane >> 5;
  const int sb = w.stride * 2;
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(w.data, w.rows * sb);
  const int voff = wrow_voff(lane, sb);
  const int fb = 32 * wave + 16 * ((lane >> 4) & 1);
#pragma unroll
  for (int p0 = 0; p0 < K; p0 += RP) {
    const int rows = K - p0 < RP ? K - p0 : RP;
    if (p0 > 0) __syncthreads();  // the previous pass's rows are read
    for (int j = wave; j < rows / 4; j += kStageThreads / kWave) dma16_buf_so(rs, voff, (p0 + 4 * j) * sb, scratch + j * 1024);
    wait_vmcnt<0>();
    __syncthreads();
#pragma unroll
    for (int s = p0 / 16; s < (p0 + rows) / 16; ++s) {
      const GP_LDS char* blk = scratch + (16 * s + 8 * lh - p0) * 256;
      wf[s] = wrows_col8(blk, blk + 4 * 256, fb, lane & 15);
    }
  }
  __syncthreads();
}

// Parameter vectors (fp16 in memory, stride 0 or 1) -> fp32 LDS array.
// n parameters into LDS as fp32; a null view reads as `absent` (0 for a bias
// or beta, 1 for gamma).
__device__ __forceinline__ void load_param(const TensorView& p, GP_LDS float* dst, int n, float absent = 0.f) {
  for (int i = threadIdx.x; i < n; i += kStageThreads) dst[i] = p.data ? (float)p.data[p.stride ? i : 0] : absent;
}

// The k-loop of a tile part: RBP 32-row blocks share the A operand (weight
// fragments wf[0..KS)); B fragments come from LDS through ld(rp, s), read PF
// k-steps ahead.  The scheduling barriers pin the issue order (PF * RBP
// reads, then per k-step RBP MFMAs followed by the reads of step s + PF), so
// LDS reads stay in flight behind the MFMAs; left to itself the scheduler
// reads each step's fragments just before their MFMAs and waits for them.
template <int KS, int RBP, int PF, typename LD>
__device__ __forceinline__ void stage_mfma_loop(const h8* wf, LD ld, f16x* acc) {
  static_assert(PF >= 1 && PF <= KS, "prefetch depth");
  h8 q[PF][RBP];
#pragma unroll
  for (int p = 0; p < PF; ++p)
#pragma unroll
    for (int rp = 0; rp < RBP; ++rp) q[p][rp] = ld(rp, p);
  __builtin_amdgcn_sched_group_barrier(0x100, PF * RBP, 0);
#pragma unroll
  for (int s = 0; s < KS; ++s) {
#pragma unroll
    for (int rp = 0; rp < RBP; ++rp) acc[rp] = mfma32(wf[s], q[s % PF][rp], acc[rp]);
    __builtin_amdgcn_sched_group_barrier(0x008, RBP, 0);
    if (s + PF < KS) {
#pragma unroll
      for (int rp = 0; rp < RBP; ++rp) q[s % PF][rp] = ld(rp, s + PF);
      __builtin_amdgcn_sched_group_barrier(0x100, RBP, 0);
    }
  }
}

// A 32-row block's accumulators (lane (lr, lh) of wave w holds features
// 32 w + 4 lh + 8 g + (0..3), g = 0..3, of row lr) as two 16-byte words of
// fp16 after the activation: v_permlane32_swap trades groups g = 2q+1 of the
// lower wave half for groups g = 2q of the upper half, so word q holds the
// eight consecutive features 32 w + 16 q + 8 lh + (0..7) of the lane's row.
__device__ __forceinline__ void fp16_row_words(const f16x& a, int act, u32x4 (&w)[2]) {
  u32x2 o[4];
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    f4 v;
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = apply_act(a[4 * g + e], act);
    o[g] = __builtin_bit_cast(u32x2, __builtin_convertvector(v, h4));
  }
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const auto lo = __builtin_amdgcn_permlane32_swap(o[2 * q][0], o[2 * q + 1][0], false, false);
    const auto hi = __builtin_amdgcn_permlane32_swap(o[2 * q][1], o[2 * q + 1][1], false, false);
    w[q] = u32x4{(unsigned)lo[0], (unsigned)hi[0], (unsigned)lo[1], (unsigned)hi[1]};
  }
}

// Whether a writer's output may be stored non-temporally in whole lines
// (W::kStreamOut; false when a writer does not say).
template <typename W, typename = void>
struct stream_out : std::false_type {};
template <typename W>
struct stream_out<W, std::void_t<decltype(W::kStreamOut)>> : std::bool_constant<W::kStreamOut> {};

// One GEMM stage over num_iters tiles: out = act(in . W + b [+ acc]) or
// LayerNorm(in . W + b).
//
// NB > 0 with an input read from memory (whose next tile is always there):
// the tile is copied in 64-row parts through NB part buffers (at least
// MBLK / 64), and the copies of tile i+1 are issued while tile i is
// multiplied -- parts whose buffers are free at once before the MFMAs, the
// others as each part of tile i is done.  The input of a memory-fed first
// stage streams from HBM, so this takes its copy latency off the pipeline's
// pace.  Queue inputs (and NB = 0) take one tile at a time: acquire, copy,
// release, multiply.  With NB >= 2 MBLK / 64 a queue-fed stage keeps two
// tile buffers: while it waits for the current tile's copy it also looks
// (without waiting) at the next tile's counter, and if that tile is ready it
// is copied into the other buffer under this tile's MFMAs and epilogue.  A
// stage never waits for a next tile before its current one is out.  LPF is
// the depth (k-steps) of the LDS fragment prefetch of the MFMA loop; 0 picks
// 2 for four row blocks per part, else 4.
//
// CH: a second 128 -> 128 layer follows in the same workgroup (weight2,
// bias2).  The first layer's output act(in . W + b) goes, rounded to fp16 as
// a queue entry would hold it, into an LDS tile laid out as a 128-wide input
// tile, and the second layer reads its B operands from there; the epilogue
// (LayerNorm, or the plain store) applies to the second layer's result.  Two
// layers then cost one queue hand-off instead of two.
template <int MBLK, int K, int ACT, bool LN, int NB, int LPF, typename IR, typename AR, typename OW, bool CH = false>
__device__ void gemm_stage_impl(TensorView weight, TensorView bias, TensorView gamma, TensorView beta, float eps,
                                IR& ir, AR& ar, OW& ow, int num_iters, TensorView weight2 = {},
                                TensorView bias2 = {}) {
  constexpr int N = 128;
  constexpr int RB = MBLK / 32;
  static_assert(MBLK % 32 == 0 && MBLK <= 128, "MBLK must be 32, 64, 96 or 128");
  constexpr bool PF = NB > 0 && !IR::kFromQueue;
  constexpr bool QPF = IR::kFromQueue && NB >= 2 * (MBLK / 64);  // queue input, two tile buffers
  static_assert(NB == 0 || MBLK % 64 == 0, "prefetching works in 64-row parts");
  constexpr int H = PF ? MBLK / 64 : 1;                      // parts per tile
  constexpr int NBUF = PF ? (NB > H ? NB : H) : (QPF ? 2 : 1);  // part buffers
  constexpr int PROWS = PF ? 64 : MBLK;                      // rows per part
  constexpr int PB = PROWS * K * 2;                 // bytes per part buffer
  constexpr int RBP = PROWS / 32;                   // 32-row blocks per part
  static_assert(!CH || !PF, "a chained stage takes whole tiles");
  static_assert(!AR::kFromQueue, "accumulator tiles are read from memory");
  constexpr int ACT_OUT = CH ? ACT_NONE : ACT;      // activation of the stored result
  GP_LDS char* xs = dyn_lds();
  GP_LDS char* const chb = xs + gemm_stage_lds<MBLK, K, NB>();  // CH: the first layer's output tile
  GP_LDS float* const prm2 = (GP_LDS float*)(chb + MBLK * N * 2);  // CH: the second layer's bias
  GP_LDS float* prm = (GP_LDS float*)(xs + gemm_stage_lds<MBLK, K, NB>() + (CH ? gemm_chain_lds<MBLK>() : 0));
  // The weight view's row count is the layer's real K: input columns past it
  // are zero-filled (their weight rows are zero too).
  const int kv = weight.rows < K ? weight.rows : K;
  GP_LDS f2* lnpart = (GP_LDS f2*)(prm + 3 * N);  // [MBLK][4]

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int lr = lane & 31, lh = lane >> 5;
  const int fq = 32 * wave + 4 * lh;  // accumulator group g covers features fq + 8g + (0..3)

  h8 wf[K / 16];
  load_weight_frags<K, gemm_stage_lds<MBLK, K, NB>()>(weight, xs, wf);
  h8 wf2[CH ? N / 16 : 1];
  if constexpr (CH) load_weight_frags<N, gemm_stage_lds<MBLK, K, NB>()>(weight2, xs, wf2);
  // The weight fragments live in AGPRs (MFMA A operands are read from there
  // directly), which leaves the VGPRs to the accumulators and the epilogue.
#pragma unroll
  for (int i = 0; i < K / 16; ++i) asm volatile("" : "+a"(wf[i]));
  if constexpr (CH) {
#pragma unroll
    for (int i = 0; i < N / 16; ++i) asm volatile("" : "+a"(wf2[i]));
    load_param(bias2, prm2, N);
  }
  load_param(bias, prm, N);
  if (LN) {
    load_param(gamma, prm + N, N, 1.f);
    load_param(beta, prm + 2 * N, N);
  }
  __syncthreads();
  // This lane's 16 features' bias (and LayerNorm gamma, beta) are kept in
  // registers for all tiles -- except in 64-row stages, which are built to
  // run three workgroups per CU, and in chained stages, which hold two
  // weight matrices and run two workgroups per CU: they have no registers to
  // spare and read them from LDS for every tile.
  constexpr bool RP = MBLK >= 128 && !CH;
  float bias_r[RP ? 16 : 1], gm_r[RP && LN ? 16 : 1], bt_r[RP && LN ? 16 : 1], b2_r[RP && CH ? 16 : 1];
  if constexpr (RP) {
#pragma unroll
    for (int g = 0; g < 4; ++g)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        bias_r[4 * g + e] = prm[fq + 8 * g + e];
        if constexpr (LN) {
          gm_r[4 * g + e] = prm[N + fq + 8 * g + e];
          bt_r[4 * g + e] = prm[2 * N + fq + 8 * g + e];
        }
        if constexpr (CH) b2_r[4 * g + e] = prm2[fq + 8 * g + e];
      }
  }
  // parameter j (0 bias, 1 gamma, 2 beta, 3 the second layer's bias) of
  // this lane's feature i (0..15)
  auto param = [&](int j, int i) -> float {
    if constexpr (RP) {
      if (j == 3) return b2_r[CH ? i : 0];
      return j == 0 ? bias_r[i] : (j == 1 ? gm_r[LN ? i : 0] : bt_r[LN ? i : 0]);
    } else {
      return j == 3 ? prm2[fq + 8 * (i / 4) + i % 4] : prm[j * N + fq + 8 * (i / 4) + i % 4];
    }
  };
  // Part h of a tile view: rows [PROWS h, PROWS h + PROWS) into buffer `buf`.
  auto copy_part = [&](const TensorView& v, int h, int buf) {
    const int r0 = PROWS * h;
    const TensorView pv{v.rows > r0 ? v.data + (int64_t)r0 * v.stride : v.data, v.stride, v.rows - r0};
    load_tile_swz<PROWS, K, !IR::kFromQueue>(pv, xs + buf * PB, kv);
  };

  const int xa = lh ^ (lr & 15);
  TensorView cur{};
  int pb = 0;        // buffer of part 0 of the current tile (PF); tile buffer (QPF)
  bool pre = false;  // QPF: the current tile was copied during the previous one
  __shared__ int qflag[2];
  if constexpr (PF) {
    if (num_iters > 0) {
      cur = ir.read_acquire();
      ir.read_release();
#pragma unroll
      for (int h = 0; h < H; ++h) copy_part(cur, h, h);
    }
  }
  for (int it = 0; it < num_iters; ++it) {
    const bool more = it + 1 < num_iters;
    TensorView nxt{};
    bool qnext = false;  // QPF: the next tile is being copied
    const int npb = (pb + H) % NBUF;
    if constexpr (PF) {
      __builtin_amdgcn_s_waitcnt(kWaitAll);
      __syncthreads();  // every part of the tile is in LDS
      if (more) {
        nxt = ir.read_acquire();
        ir.read_release();
#pragma unroll
        for (int h = 0; h < NBUF - H && h < H; ++h) copy_part(nxt, h, (npb + h) % NBUF);
      }
    } else if constexpr (QPF) {
      if (!pre) {
        cur = ir.read_acquire();
        copy_part(cur, 0, pb);
      }
      if (threadIdx.x == 0) {
        // both loads are in flight with the tile copy
        const bool pk = more && ir.peek_next();
        const int rw = pre ? ir.rows() : 0;
        qflag[0] = pk;
        qflag[1] = rw;
      }
      __builtin_amdgcn_s_waitcnt(kWaitAll);
      __syncthreads();
      if (pre) cur = ir.view(qflag[1]);
      qnext = qflag[0] != 0;
      ir.read_release_landed();  // the tile is in LDS: hand the input slot back at once
      if (qnext) {
        // the peeked tile is now the reader's current one; copy all MBLK rows
        // (rows past its count are never stored)
        copy_part(ir.view(MBLK), 0, pb ^ 1);
      }
    } else {
      cur = ir.read_acquire();
      copy_part(cur, 0, 0);
      __builtin_amdgcn_s_waitcnt(kWaitAll);
      __syncthreads();
      ir.read_release_landed();  // the tile is in LDS: hand the input slot back at once
    }

    // accumulators start at bias (+ the accumulator tile, pipe_gemm.cuh:128-146)
    f16x acc[RB];
    const TensorView at = ar.read_acquire();
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[rb][i] = param(0, i);
      if (at.data != nullptr) {
        const int r = 32 * rb + lr;
        if (r < at.rows) {
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const h4 a4 = *(const h4*)(at.data + (int64_t)r * at.stride + fq + 8 * g);
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[rb][4 * g + e] += (float)a4[e];
          }
        }
      }
    }
    ar.read_release();

#pragma unroll
    for (int h = 0; h < H; ++h) {
      const GP_LDS char* xp = xs + ((pb + h) % NBUF) * PB + lr * (K * 2);
      stage_mfma_loop<K / 16, RBP, LPF ? LPF : (RBP >= 4 ? 2 : 4)>(wf, [&](int rp, int s) {
        const int off = ((2 * s) & ~15) * 16 + (((2 * s) ^ xa) & 15) * 16;
        return *(const GP_LDS h8*)(xp + rp * (32 * K * 2) + off);
      }, acc + RBP * h);
      if constexpr (PF) {
        // part h's buffer is free once every wave is past its MFMAs: part
        // h + NBUF - H of the next tile goes there
        const int hn = h + NBUF - H;
        if (hn < H && more) {
          __syncthreads();
          copy_part(nxt, hn, (pb + h) % NBUF);
        }
      }
    }

    if constexpr (CH) {
      // The first layer's output into the chain tile: chunk c of row r at
      // chunk position (c ^ r) & 15, the layout load_tile_swz gives a
      // 128-wide tile.  The tile is free: the last reads of the previous
      // tile's second layer came before that tile's epilogue barriers.
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        const int r = 32 * rb + lr;
        u32x4 w[2];
        fp16_row_words(acc[rb], ACT, w);
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          const int c = 4 * wave + 2 * q + lh;
          *(GP_LDS u32x4*)(chb + r * (N * 2) + ((c ^ (r & 15)) << 4)) = w[q];
        }
      }
      __syncthreads();
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[rb][i] = param(3, i);
      const GP_LDS char* xp = chb + lr * (N * 2);
      stage_mfma_loop<N / 16, RB, (RB >= 4 ? 2 : 4)>(wf2, [&](int rp, int s) {
        const int off = (((2 * s) ^ xa) & 15) * 16;
        return *(const GP_LDS h8*)(xp + rp * (32 * N * 2) + off);
      }, acc);
    }

    if constexpr (LN) {
      // per-wave (mean, M2) over 32 features, combined over the four waves
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        float s0 = 0.f;
#pragma unroll
        for (int v = 0; v < 16; ++v) s0 += acc[rb][v];
        s0 = sum_lane_halves(s0);
        const float m0 = s0 * (1.f / 32.f);
        float q0 = 0.f;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const float d = acc[rb][v] - m0;
          q0 = __builtin_fmaf(d, d, q0);
        }
        q0 = sum_lane_halves(q0);
        if (lh == 0) lnpart[(32 * rb + lr) * 4 + wave] = f2{m0, q0};
      }
      __syncthreads();
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        const GP_LDS f2* pr = lnpart + (32 * rb + lr) * 4;
        const f2 p0 = pr[0], p1 = pr[1], p2 = pr[2], p3 = pr[3];
        const float mu = 0.25f * ((p0[0] + p1[0]) + (p2[0] + p3[0]));
        const float d0 = p0[0] - mu, d1 = p1[0] - mu, d2 = p2[0] - mu, d3 = p3[0] - mu;
        const float m2 = (p0[1] + p1[1]) + (p2[1] + p3[1]) + 32.f * (d0 * d0 + d1 * d1 + d2 * d2 + d3 * d3);
        const float rstd = rsqrtf(m2 * (1.f / N) + eps);
        const float nmr = -mu * rstd;
#pragma unroll
        for (int i = 0; i < 16; ++i)
          acc[rb][i] = __builtin_fmaf(__builtin_fmaf(acc[rb][i], rstd, nmr), param(1, i), param(2, i));
      }
    }

    // Stores: each lane writes the eight consecutive features of each word
    // of fp16_row_words with one 16-byte store.
    //
    // A LayerNorm or chained stage writing memory (stream_out) stages the
    // tile in its input tile buffer instead -- free since the LayerNorm or
    // chain barrier, which follows every wave's MFMAs on that buffer -- and
    // each wave then stores four whole 256-byte rows per instruction with
    // the non-temporal policy.  16-byte
    // chunk c of row r sits at chunk position c ^ (r % 16), so the 32 rows a
    // wave writes at one chunk and the 16 chunks of a row it reads both
    // spread over the banks.  Whole-line non-temporal stores keep the output
    // out of L2, whose lines the queues need; 32-byte pieces would be
    // written back as partial lines.
    constexpr bool STAGED = ((LN && QPF) || (CH && !PF)) && stream_out<OW>::value && MBLK * N * 2 <= PB;
    const TensorView ot = ow.write_acquire(cur.rows);
    GP_LDS char* const st = xs + pb * PB;
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      const int r = 32 * rb + lr;
      u32x4 w[2];
      fp16_row_words(acc[rb], LN ? ACT_NONE : ACT_OUT, w);
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        if constexpr (STAGED) {
          const int c = 4 * wave + 2 * q + lh;
          *(GP_LDS u32x4*)(st + r * (N * 2) + ((c ^ (r & 15)) << 4)) = w[q];
        } else {
          if (r < ot.rows) *(u32x4*)(ot.data + (int64_t)r * ot.stride + 32 * wave + 16 * q + 8 * lh) = w[q];
        }
      }
    }
    if constexpr (STAGED) {
      __syncthreads();
      const int j = lane & 15;
#pragma unroll
      for (int i = 0; i < MBLK / 16; ++i) {
        const int row = (MBLK / 4) * wave + 4 * i + (lane >> 4);
        const u32x4 v = *(const GP_LDS u32x4*)(st + row * (N * 2) + ((j ^ (row & 15)) << 4));
        if (row < ot.rows) __builtin_nontemporal_store(v, (u32x4*)(ot.data + (int64_t)row * ot.stride + 8 * j));
      }
    }
    ow.write_release();
    // LDS tile / LN partials are reused by the next iteration; a queue
    // writer's release already ends with a barrier after every wave's stores.
    // A staged tile needs none either: its barrier follows every wave's reads
    // of the LN partials and the queue flags, and the next copy into the
    // staging buffer comes after the next iteration's first barrier (the one
    // after the tile wait when the next tile was prefetched into the other
    // buffer, else the one in read_acquire).
    if constexpr (!OW::kReleaseBarrier && !STAGED) __syncthreads();
    if constexpr (PF) {
      pb = npb;
      cur = nxt;
    } else if constexpr (QPF) {
      pre = qnext;
      if (pre) pb ^= 1;
    }
  }
}

// pipe_gemm_bias_relu.cuh:85-192: out = relu(in . W + b).
template <int MBLK, int K, int NB = 0, int LPF = 0, typename IR, typename AR, typename OW>
__device__ void pipe_gemm_bias_relu(TensorView weight, TensorView bias, IR& ir, AR& ar, OW& ow, int num_iters) {
  gemm_stage_impl<MBLK, K, ACT_RELU, false, NB, LPF>(weight, bias, {}, {}, 0.f, ir, ar, ow, num_iters);
}

// pipe_gemm_bias.cuh:85-191: out = in . W + b.
template <int MBLK, int K, int NB = 0, int LPF = 0, typename IR, typename AR, typename OW>
__device__ void pipe_gemm_bias(TensorView weight, TensorView bias, IR& ir, AR& ar, OW& ow, int num_iters) {
  gemm_stage_impl<MBLK, K, ACT_NONE, false, NB, LPF>(weight, bias, {}, {}, 0.f, ir, ar, ow, num_iters);
}

// pipe_gemm.cuh:78-183: out = in . W (+ accumulator tile from ar).
template <int MBLK, int K, int NB = 0, int LPF = 0, typename IR, typename AR, typename OW>
__device__ void pipe_gemm(TensorView weight, IR& ir, AR& ar, OW& ow, int num_iters) {
  gemm_stage_impl<MBLK, K, ACT_NONE, false, NB, LPF>(weight, {}, {}, {}, 0.f, ir, ar, ow, num_iters);
}

// Generic activation epilogue (GELU / sigmoid heads of the later apps).
template <int MBLK, int K, int ACT, int NB = 0, int LPF = 0, typename IR, typename AR, typename OW>
__device__ void pipe_gemm_bias_act(TensorView weight, TensorView bias, IR& ir, AR& ar, OW& ow, int num_iters) {
  gemm_stage_impl<MBLK, K, ACT, false, NB, LPF>(weight, bias, {}, {}, 0.f, ir, ar, ow, num_iters);
}

// pipe_gemm_bias_layer_norm.cuh:100-249: out = LayerNorm(in . W + b) * gamma + beta.
template <int MBLK, int K, int NB = 0, int LPF = 0, typename IR, typename AR, typename OW>
__device__ void pipe_gemm_bias_layer_norm(TensorView weight, TensorView bias, TensorView gamma, TensorView beta,
                                          float eps, IR& ir, AR& ar, OW& ow, int num_iters) {
  gemm_stage_impl<MBLK, K, ACT_NONE, true, NB, LPF>(weight, bias, gamma, beta, eps, ir, ar, ow, num_iters);
}

// pipe_gemm_bias_relu followed by pipe_gemm_bias_layer_norm (LN) or
// pipe_gemm_bias in one workgroup: out = LayerNorm(relu(in . W + b) . W2 + b2)
// * gamma + beta, or relu(in . W + b) . W2 + b2.  The 128-wide intermediate
// tile passes through LDS (rounded to fp16, as a queue entry holds it), not a
// queue.  Whole input tiles (a queue input with NB >= 2 MBLK / 64 copies the
// next tile under this one).
template <int MBLK, int K, bool LN, int NB = 0, typename IR, typename AR, typename OW>
__device__ void pipe_gemm_bias_relu_chain(TensorView weight, TensorView bias, TensorView weight2, TensorView bias2,
                                          TensorView gamma, TensorView beta, float eps, IR& ir, AR& ar, OW& ow,
                                          int num_iters) {
  gemm_stage_impl<MBLK, K, ACT_RELU, LN, NB, 0, IR, AR, OW, true>(weight, bias, gamma, beta, eps, ir, ar, ow,
                                                                  num_iters, weight2, bias2);
}

// ---------------------------------------------------------------------------
// pipe_layer_norm.cuh:13-60 with layer_norm_v2.cuh:16-73: LayerNorm over D
// features of each row, fp32 math, fp16 I/O, two-pass variance.  Sixteen
// lanes share a row (D/16 features each, 16-byte vectors), so one wave
// covers four rows per step; the reductions are 16-lane butterflies.
// ---------------------------------------------------------------------------
template <int MBLK, int D, typename IR, typename OW>
__device__ void pipe_layer_norm(TensorView gamma, TensorView beta, IR& ir, OW& ow, int num_iters, float eps) {
  static_assert(D % 128 == 0 && D <= 1024, "D must be a multiple of 128, at most 1024");
  constexpr int NV = D / 128;  // 16-byte vectors per lane per row
  const int tid = threadIdx.x;
  const int g16 = tid & 15;    // lane within the row group
  const int rsub = tid >> 4;   // row within a 16-row pass
  float gm[NV][8], bt[NV][8];
#pragma unroll
  for (int j = 0; j < NV; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int f = 128 * j + 8 * g16 + e;
      gm[j][e] = gamma.data ? (float)gamma.data[gamma.stride ? f : 0] : 1.f;
      bt[j][e] = beta.data ? (float)beta.data[beta.stride ? f : 0] : 0.f;
    }
  for (int it = 0; it < num_iters; ++it) {
    const TensorView in = ir.read_acquire();
    const TensorView ot = ow.write_acquire(in.rows);
    const int nrows = in.rows < ot.rows ? in.rows : ot.rows;  // a NullWriter takes no rows
    for (int r0 = 0; r0 < MBLK; r0 += kStageThreads / 16) {
      const int r = r0 + rsub;
      const bool valid = r < nrows;
      float x[NV][8];
      float s = 0.f;
#pragma unroll
      for (int j = 0; j < NV; ++j) {
        h8 v = {};
        if (valid) v = view_load_h8<IR::kFromQueue>(in, (int64_t)r * in.stride + 128 * j + 8 * g16);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          x[j][e] = (float)v[e];
          s += x[j][e];
        }
      }
#pragma unroll
      for (int m = 8; m >= 1; m >>= 1) s += __shfl_xor(s, m, 16);
      const float mean = s * (1.f / D);
      float q = 0.f;
#pragma unroll
      for (int j = 0; j < NV; ++j)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float d = x[j][e] - mean;
          q = __builtin_fmaf(d, d, q);
        }
#pragma unroll
      for (int m = 8; m >= 1; m >>= 1) q += __shfl_xor(q, m, 16);
      const float rstd = rsqrtf(q * (1.f / D) + eps);
      if (valid) {
#pragma unroll
        for (int j = 0; j < NV; ++j) {
          h8 o;
#pragma unroll
          for (int e = 0; e < 8; ++e) o[e] = (half_t)((x[j][e] - mean) * rstd * gm[j][e] + bt[j][e]);
          *(h8*)(ot.data + (int64_t)r * ot.stride + 128 * j + 8 * g16) = o;
        }
      }
    }
    ir.read_release();
    ow.write_release();
  }
}

// ---------------------------------------------------------------------------
// pipe_add.cuh:13-40 (elemwise_add.cuh:5-21): c = a + b, n halves per row.
// fp16 addition of two fp16 values is the correctly rounded real sum, i.e.
// identical to adding in fp32 and rounding once.
// ---------------------------------------------------------------------------
template <typename IR0, typename IR1, typename OW>
__device__ void pipe_add_n(IR0& ir0, IR1& ir1, OW& ow, int num_iters, int n) {
  const int vpr = n / 8;  // 16-byte vectors per row
  for (int it = 0; it < num_iters; ++it) {
    const TensorView a = ir0.read_acquire();
    const TensorView b = ir1.read_acquire();
    const int rows = a.rows < b.rows ? a.rows : b.rows;
    const TensorView c = ow.write_acquire(rows);
    const int n = rows < c.rows ? rows : c.rows;  // a NullWriter takes no rows
    for (int i = threadIdx.x; i < n * vpr; i += kStageThreads) {
      const int r = i / vpr, v = i - r * vpr;
      const h8 x = view_load_h8<IR0::kFromQueue>(a, (int64_t)r * a.stride + 8 * v);
      const h8 y = view_load_h8<IR1::kFromQueue>(b, (int64_t)r * b.stride + 8 * v);
      *(h8*)(c.data + (int64_t)r * c.stride + 8 * v) = x + y;
    }
    ir0.read_release();
    ir1.read_release();
    ow.write_release();
  }
}

template <int MBLK, int N, typename IR0, typename IR1, typename OW>
__device__ void pipe_add(IR0& ir0, IR1& ir1, OW& ow, int num_iters) {
  static_assert(N % 8 == 0, "N must be a multiple of 8");
  pipe_add_n(ir0, ir1, ow, num_iters, N);
}

// ---------------------------------------------------------------------------
// pipe_concat.cuh:48-74 (concat2_internal :6-39): c[r] = [a[r] | b[r]] with
// 16-byte copies; n0 and n1 halves must be multiples of 8 (pipe_concat.cuh:13-14).
// ---------------------------------------------------------------------------
template <typename IR0, typename IR1, typename OW>
__device__ void pipe_concat_n(IR0& ir0, IR1& ir1, OW& ow, int num_iters, int n0, int n1) {
  const int v0 = n0 / 8, vo = (n0 + n1) / 8;
  for (int it = 0; it < num_iters; ++it) {
    const TensorView a = ir0.read_acquire();
    const TensorView b = ir1.read_acquire();
    const int rows = a.rows < b.rows ? a.rows : b.rows;
    const TensorView c = ow.write_acquire(rows);
    const int n = rows < c.rows ? rows : c.rows;  // a NullWriter takes no rows
    for (int i = threadIdx.x; i < n * vo; i += kStageThreads) {
      const int r = i / vo, v = i - r * vo;
      const h8 x = v < v0 ? view_load_h8<IR0::kFromQueue>(a, (int64_t)r * a.stride + 8 * v)
                          : view_load_h8<IR1::kFromQueue>(b, (int64_t)r * b.stride + 8 * (v - v0));
      *(h8*)(c.data + (int64_t)r * c.stride + 8 * v) = x;
    }
    ir0.read_release();
    ir1.read_release();
    ow.write_release();
  }
}

template <int MBLK, int N0, int N1, typename IR0, typename IR1, typename OW>
__device__ void pipe_concat(IR0& ir0, IR1& ir1, OW& ow, int num_iters) {
  static_assert(N0 % 8 == 0 && N1 % 8 == 0, "N0 * 2 and N1 * 2 must be multiples of 16 bytes");
  pipe_concat_n(ir0, ir1, ow, num_iters, N0, N1);
}

// Copy stage (the sender / receiver of the reference's identity pipeline,
// misc_tests/pipeval/pipe_val_ext.cu:65-108): out tile = in tile, n halves per row.
template <typename IR, typename OW>
__device__ void pipe_copy_n(IR& ir, OW& ow, int num_iters, int n) {
  const int vpr = n / 8;
  for (int it = 0; it < num_iters; ++it) {
    const TensorView a = ir.read_acquire();
    const TensorView c = ow.write_acquire(a.rows);
    const int n = a.rows < c.rows ? a.rows : c.rows;  // a NullWriter takes no rows
    for (int i = threadIdx.x; i < n * vpr; i += kStageThreads) {
      const int r = i / vpr, v = i - r * vpr;
      *(h8*)(c.data + (int64_t)r * c.stride + 8 * v) = view_load_h8<IR::kFromQueue>(a, (int64_t)r * a.stride + 8 * v);
    }
    ir.read_release();
    ow.write_release();
  }
}

}  // namespace gp
