// The DLRM bottom MLP (K0 -> 512 -> 256 -> 128) as one persistent gfx950
// kernel: the three layers of a 256-row tile run back to back without their
// activations leaving the CU.
//
// Semantics: apps/dlrm_botmlp/torch/model.py (DlrmMlp of common/mlps.py:23-34
// with widths [K0, 512, 256, 128], ReLU after every layer).  The reference
// runs it as one pipelined kernel of three GEMM stage blocks linked by queues
// (apps/dlrm_botmlp/pipelined/dlrm_botmlp_pl.cuh:79-173); here the stages of
// one tile are a single wave's instruction stream instead.
//
// Design.
//  * A workgroup of eight waves (two per SIMD) owns a tile of 256 rows; wave
//    w owns rows 32w .. 32w+31 and computes every feature of every layer for
//    them as C^T = W^T X^T with v_mfma_f32_32x32x16: the A operand is a
//    32-feature x 16-k block of the weights (a "fragment", 64 lanes x 16
//    bytes), the B operand a 16-k x 32-row block of the layer input.
//  * The 512-wide first layer never exists as a whole: its 32-feature block j
//    (16 accumulator registers) is converted to fp16 and is, in exactly the
//    accumulator lane layout, the B operand of the second layer's k-blocks
//    2j and 2j+1 (the weight packing folds in the permutation, sigma below).
//    So a wave holds the second layer's 256 accumulators' worth of state (128
//    registers), one first-layer block and its two B operands at a time.
//  * The first layer's weights (16 or 32 KiB) stay in LDS for the whole
//    kernel.  The second and third layers' (320 KiB) stream from L2 every
//    tile: the host packs them once per call into the order the kernel
//    consumes them, 16 fragments to a 16 KiB slot -- slot j holds the second
//    layer's k-blocks 2j, 2j+1 for all eight feature blocks (the 16 MFMAs that
//    consume first-layer block j), slots 16-19 the third layer.  Waves 0-3
//    copy slots L2 -> LDS with buffer_load ... lds into a ring of six; a slot
//    is acquired by waiting for this wave's own copies of it and one barrier,
//    and its ring place is refilled with the slot five ahead once its first
//    MFMAs are issued.
//  * The tile's input rows come through an LDS tile (K0 <= 32 columns),
//    copied by waves 4-7 one tile ahead, so their HBM latency never holds up
//    a wait for a ring slot (vmcnt counts a wave's own memory operations, in
//    issue order).
//  * Biases enter through the MFMA: the first product of every accumulator is
//    the bias fragment (bias in k = 0) times a B operand that is 1 at k = 0,
//    so the hidden epilogues are only the fp16 conversion and the ReLU.
//  * The 128 outputs of a row are stored as 16-byte buffer stores bounded to
//    the tile's valid rows.
#include <hip/hip_runtime.h>

#include <type_traits>
#include <utility>

#include "../../include/gpipes.h"
#include "gp_device.hpp"
#include "gp_host.hpp"
#include "gp_kernels.hpp"
#include "stages.hpp"

namespace gp {
namespace dlrm {

constexpr int NW = 8;                // waves per workgroup, two per SIMD
constexpr int NT = NW * kWave;
constexpr int ROWS = 32 * NW;        // rows per tile
constexpr int FRAG = 1024;           // one A operand: 64 lanes x 16 bytes
constexpr int FPS = 16;              // fragments per slot
constexpr int SLOT = FPS * FRAG;     // bytes per ring slot
constexpr int NS = 6;                // ring slots
constexpr int RW = 4;                // waves 0 .. RW-1 copy the ring, the others the input rows
constexpr int CPW = FPS / RW;        // 1 KiB ring copies per copying wave per slot
constexpr int H1 = 512, H2 = 256, H3 = 128;
constexpr int FB1 = H1 / 32, FB2 = H2 / 32, FB3 = H3 / 32;  // feature blocks per layer
constexpr int KB3 = H2 / 16;                                // k-blocks of the third layer
constexpr int kMaxK0 = 32;
constexpr int S_W3 = FB1;                      // slots 0-15: second layer; 16-19: third
constexpr int ST = S_W3 + KB3 * FB3 / FPS;     // slots per tile
constexpr int W1_BYTES = FB1 * (kMaxK0 / 16) * FRAG;  // first-layer fragments, [fb][kb]
constexpr int XBUF = ROWS * kMaxK0 * 2;               // one tile of input rows
constexpr int XCPW = XBUF / FRAG / (NW - RW);         // input copies per input wave
constexpr int kOutStores = FB3 * 2;                   // output stores per wave and tile
// Bias tables: per feature block fb a 64-entry A-operand column, bias[32 fb +
// lane] for lanes < 32 and 0 for the upper half (k = 8..15).
constexpr int BF_1 = 0, BF_2 = 64 * FB1, BF_3 = BF_2 + 64 * FB2, B_TOTAL = BF_3 + 64 * FB3;
// LDS: ring, first-layer weights, input tile, bias tables.
constexpr int L_W1 = NS * SLOT, L_X = L_W1 + W1_BYTES, L_B = L_X + XBUF, LDS_BYTES = L_B + B_TOTAL * 2;
static_assert(LDS_BYTES <= 160 * 1024, "LDS");
static_assert(XCPW <= CPW * (NS - 2), "input copies in flight");
// Packed weights (one workspace block): first-layer fragments, the slot
// stream, the bias tables.
constexpr size_t P_STREAM = W1_BYTES;
constexpr size_t P_BIAS = P_STREAM + (size_t)ST * SLOT;
constexpr size_t P_TOTAL = P_BIAS + (size_t)B_TOTAL * 2;

struct Args {
  const half_t* x;     // [M][K0]
  const char* pack;    // P_TOTAL bytes (dlrm_pack_kernel)
  half_t* out;         // [M][128]
  int64_t M;
  int K0;
  int relu1, relu2;    // ReLU after the first / second layer (else identity)
  int act3;            // activation of the third layer (ACT_*)
};

// B-operand k-order of a k-block fed from registers: position p holds input
// feature 16 kb + sigma(p) (the accumulator layout of the layer before).
__host__ __device__ constexpr int sigma(int p) { return p < 4 ? p : p < 8 ? p + 4 : p < 12 ? p - 4 : p; }

template <int... I, class F>
__device__ __forceinline__ void static_for(std::integer_sequence<int, I...>, F&& f) {
  (f(std::integral_constant<int, I>{}), ...);
}

// fp16 (bf16) pair of an accumulator block with an optional ReLU: lo holds
// elements 0-7, hi 8-15.  In bf16 the ReLU is a signed 16-bit integer max on
// the rounded bits (a bf16 value with its sign bit set becomes +0).
template <typename E>
__device__ __forceinline__ void to_operands(const f16x& a, bool relu, h8& lo, h8& hi) {
  if constexpr (std::is_same_v<E, F16>) {
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      lo[r] = (half_t)a[r];
      hi[r] = (half_t)a[8 + r];
    }
    if (relu) {
      lo = __builtin_elementwise_max(lo, h8{});
      hi = __builtin_elementwise_max(hi, h8{});
    }
  } else {
    lo = __builtin_shufflevector(E::cvt4(f4{a[0], a[1], a[2], a[3]}), E::cvt4(f4{a[4], a[5], a[6], a[7]}), 0, 1, 2, 3,
                                 4, 5, 6, 7);
    hi = __builtin_shufflevector(E::cvt4(f4{a[8], a[9], a[10], a[11]}), E::cvt4(f4{a[12], a[13], a[14], a[15]}), 0, 1,
                                 2, 3, 4, 5, 6, 7);
    if (relu) {
      lo = __builtin_bit_cast(h8, __builtin_elementwise_max(__builtin_bit_cast(s8, lo), s8{}));
      hi = __builtin_bit_cast(h8, __builtin_elementwise_max(__builtin_bit_cast(s8, hi), s8{}));
    }
  }
}

// E: F16 or BF16.  NKB1: k-blocks of the first layer (K0 <= 16 NKB1).
template <typename E, int NKB1>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(2, 2))) void dlrm_bot_kernel(Args p) {
  __shared__ __attribute__((aligned(1024))) char smem[LDS_BYTES];
  GP_LDS char* const ring = (GP_LDS char*)smem;
  GP_LDS const char* const w1 = (GP_LDS const char*)smem + L_W1;
  GP_LDS half_t* const bfrag = (GP_LDS half_t*)(smem + L_B);

  const int tid = threadIdx.x;
  const int lane0 = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool ring_wave = wave < RW;
  const int G = gridDim.x;
  // Tile and slot counts fit in 32 bits: the host limits M to 2^31 - 1.
  const int ntiles = (int)((p.M + ROWS - 1) / ROWS);
  const int my = (ntiles - (int)blockIdx.x + G - 1) / G;  // tiles blockIdx.x + k G, k < my

  // Resident for the whole kernel: the first layer's fragments and the bias
  // tables.
  for (int i = tid; i < NKB1 * FB1 * FRAG / 16; i += NT) {
    // fragment (fb, kb) sits at (2 fb + kb) FRAG in the packed block and at
    // (NKB1 fb + kb) FRAG in LDS
    const int f = i / kWave, l = i % kWave;
    const int src = ((f / NKB1) * 2 + f % NKB1) * FRAG + 16 * l;
    *(GP_LDS h8*)(smem + L_W1 + f * FRAG + 16 * l) = *(const h8*)(p.pack + src);
  }
  for (int i = tid; i < B_TOTAL / 8; i += NT) ((GP_LDS h8*)bfrag)[i] = ((const h8*)(p.pack + P_BIAS))[i];
  __syncthreads();

  auto tile_r0 = [&](int k) { return ((int64_t)blockIdx.x + (int64_t)k * G) * ROWS; };

  // ---------------------------------------------------------- input tiles
  // Waves RW .. NW-1 copy tile k's input rows into the input buffer, chunk
  // c = (NW - RW) i + (wave - RW) being copy i.  Past the last tile the range
  // is 0: the copies read nothing and zero a dead buffer, so an input wave
  // always has the same copies in flight.
  auto copy_input = [&](int k) {
    if (ring_wave) return;
    const int64_t row0 = tile_r0(k);
    const int64_t left = k < my ? p.M - row0 : 0;
    const int rows = left <= 0 ? 0 : left < ROWS ? (int)left : ROWS;
    // The range is rounded up to whole 16-byte copies; the bytes past the last
    // valid row lie in the same 16-byte block and land only in rows that are
    // never stored.
    const __amdgpu_buffer_rsrc_t r = make_rsrc(p.x + row0 * p.K0, (rows * p.K0 * 2 + 15) & ~15);
#pragma unroll
    for (int i = 0; i < XCPW; ++i) {
      const int c = (NW - RW) * i + (wave - RW);
      dma16_buf_so(r, 16 * lane0, c * FRAG, (GP_LDS char*)smem + L_X + c * FRAG);
    }
  };

  // ---------------------------------------------------------------- ring
  // Global slot q = k ST + l (tile k, local slot l) lives in ring slot
  // q % NS.  `cur` is the ring slot of the last acquired slot; (iss_k, iss_l)
  // the next slot to copy, which goes to ring slot (cur + NS - 1) % NS.
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(p.pack + P_STREAM, ST * SLOT);
  int cur = NS - 1, iss_k = 0, iss_l = 0;
  // Copy the next slot into ring slot `rs` (ring waves; chunk c = RW i + wave
  // is copy i).  Past the last slot the range is 0: the copies read nothing
  // and zero a dead slot, and every acquire finds the same copies in flight.
  auto issue = [&](int rs) {
    const __amdgpu_buffer_rsrc_t r = iss_k < my ? rw : make_rsrc(p.pack, 0);
    const int base = iss_l * SLOT;
    GP_LDS char* const dst = ring + rs * SLOT;
    if (ring_wave) {
#pragma unroll
      for (int i = 0; i < CPW; ++i) {
        const int c = RW * i + wave;
        dma16_buf_so(r, 16 * lane0, base + c * FRAG, dst + c * FRAG);
      }
    }
    const bool wrap = ++iss_l == ST;
    iss_l = wrap ? 0 : iss_l;
    iss_k += wrap ? 1 : 0;
  };
  copy_input(0);
  for (int i = 0; i < NS - 1; ++i) issue(i);
  // Acquire the next slot in stream order: a ring wave waits for its own
  // copies of it (the CPW (NS - 2) copies issued after them may still be in
  // flight, and OUT_STORES output stores of the previous tile issued after
  // those), then one barrier.  An input wave has fewer operations in flight
  // than that, so the wait is a no-op for it.  The copy that refills the ring
  // slot of the previous one (dead from the barrier on) is issued by refill(),
  // after the first MFMAs of the new slot; every acquire is followed by
  // exactly one refill() before the next acquire.
  auto acquire = [&](auto out_stores) {
    wait_vmcnt<CPW * (NS - 2) + decltype(out_stores)::value>();
    lds_barrier();
    cur = cur == NS - 1 ? 0 : cur + 1;
  };
  auto refill = [&] { issue(cur == 0 ? NS - 1 : cur - 1); };

  f16x acc[FB2];  // second-layer accumulators; the first FB3 are reused by the third layer
  f16x acc1;      // the first-layer block in flight
  h8 act[KB3];    // second-layer outputs as third-layer B operands
  h8 xin[NKB1];   // the input rows as first-layer B operands
  // A fragments, double-buffered: group g + 1 of a slot is read while group
  // g's MFMAs issue, and a slot's last group issues after the next slot's
  // barrier, so neither the LDS latency nor the barrier leaves the wave
  // without MFMAs to issue.
  h8 fa[2][4];
  // B operand that is 1 at k = 0 and 0 elsewhere: lanes 0-31 hold k = 0..7.
  h8 ones = {};
  ones[0] = __builtin_bit_cast(half_t, lane0 < 32 ? E::kOne : (unsigned short)0);

  using S0 = std::integral_constant<int, 0>;
  using SO = std::integral_constant<int, kOutStores>;
  using B0 = std::integral_constant<int, 0>;
  using B1 = std::integral_constant<int, 1>;

  for (int k = 0; k < my; ++k) {
    const int64_t r0 = tile_r0(k);
    const int vrows = p.M - r0 < ROWS ? (int)(p.M - r0) : ROWS;
    auto cur_slot = [&] { return (GP_LDS const char*)(ring + cur * SLOT); };
    // Read group g (fragments 4g .. 4g+3) of the current slot into fa[BUF].
    auto fetch = [&](int g, auto bufc) {
      constexpr int BUF = decltype(bufc)::value;
      GP_LDS const char* const s = cur_slot() + 4 * g * FRAG + 16 * lane0;
#pragma unroll
      for (int i = 0; i < 4; ++i) fa[BUF][i] = *(GP_LDS const h8*)(s + i * FRAG);
    };
    // Acquire the next slot and read its group 0 into fa[0].
    auto advance = [&] {
      acquire(S0{});
      fetch(0, B0{});
    };
    // acc[fb] = bias (x) ones for the FB feature blocks of a layer.
    auto bias_init = [&](auto FBc, int off) {
      constexpr int FB = decltype(FBc)::value;
#pragma unroll
      for (int fb = 0; fb < FB; ++fb) {
        h8 a = {};
        a[0] = bfrag[off + 64 * fb + lane0];
        acc[fb] = E::mma(a, ones, f16x{});
      }
    };
    // First-layer block j: bias, then the input k-blocks, weights from LDS.
    auto layer1 = [&](int j) {
      h8 a = {};
      a[0] = bfrag[BF_1 + 64 * j + lane0];
      f16x c = E::mma(a, ones, f16x{});
#pragma unroll
      for (int kb = 0; kb < NKB1; ++kb) {
        const h8 w = *(GP_LDS const h8*)(w1 + ((j * NKB1 + kb) * FRAG + 16 * lane0));
        c = E::mma(w, xin[kb], c);
      }
      return c;
    };

    // The tile's first slot.  The input waves wait for this tile's input
    // copies (the previous tile's output stores, issued after them, may still
    // be in flight); the acquire's barrier then publishes the input tile.
    if (k == 0) {
      if (!ring_wave) wait_vmcnt<0>();
      advance();
    } else {
      if (!ring_wave) wait_vmcnt<kOutStores>();
      acquire(SO{});
      fetch(0, B0{});
    }
    // This wave's rows of the input tile, K0 columns each, as NKB1 k-blocks
    // (zero past K0).
    {
      GP_LDS const char* const b = (GP_LDS const char*)smem + L_X;
      const int lane = opaque(lane0), lr = lane & 31, lh = lane >> 5;
      const int K = opaque(p.K0);
      const int e0 = (32 * wave + lr) * K + 8 * lh;
#pragma unroll
      for (int kb = 0; kb < NKB1; ++kb) {
        const int n = min(max(K - 16 * kb - 8 * lh, 0), 8);  // valid columns of this lane's 8
        h8 v;
        if ((p.K0 & 7) == 0) {
          v = *(GP_LDS const h8*)(b + (e0 + 16 * kb) * 2);
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e) v[e] = *(GP_LDS const half_t*)(b + (e0 + 16 * kb + e) * 2);
        }
        u32x4 w = __builtin_bit_cast(u32x4, v);
#pragma unroll
        for (int i = 0; i < 4; ++i) w[i] &= n >= 2 * i + 2 ? 0xffffffffu : n == 2 * i + 1 ? 0xffffu : 0u;
        xin[kb] = __builtin_bit_cast(h8, w);
      }
    }
    bias_init(std::integral_constant<int, FB2>{}, BF_2);
    acc1 = layer1(0);

    // Slots 0-15: first-layer block j feeds the second layer's k-blocks 2j
    // (group 0: feature blocks 0-3, group 1: 4-7) and 2j + 1 (groups 2, 3);
    // block j + 1 is computed meanwhile.
#pragma nounroll
    for (int j = 0; j < FB1; ++j) {
      h8 a0, a1;
      to_operands<E>(acc1, p.relu1 != 0, a0, a1);
      // (block FB1 - 1 is recomputed once at the end: branch-free)
      acc1 = layer1(j + 1 < FB1 ? j + 1 : j);
      fetch(1, B1{});
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[i] = E::mma(fa[0][i], a0, acc[i]);
      refill();
      // Every wave has read this tile's input rows (a barrier has passed
      // since): the next tile's go into the buffer now.
      if (j == 1) copy_input(k + 1);
      __builtin_amdgcn_sched_barrier(0);
      fetch(2, B0{});
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[4 + i] = E::mma(fa[1][i], a0, acc[4 + i]);
      __builtin_amdgcn_sched_barrier(0);
      fetch(3, B1{});
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[i] = E::mma(fa[0][i], a1, acc[i]);
      __builtin_amdgcn_sched_barrier(0);
      // The next slot (the first third-layer slot after j = 15); group 3's
      // fragments are in registers, so its MFMAs issue after the barrier.
      advance();
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[4 + i] = E::mma(fa[1][i], a1, acc[4 + i]);
    }
    // Second-layer epilogue, then the third layer: slot S_W3 + s holds
    // k-blocks 4s .. 4s+3 (group g: k-block 4s + g) for the four feature
    // blocks.
#pragma unroll
    for (int fb = 0; fb < FB2; ++fb) to_operands<E>(acc[fb], p.relu2 != 0, act[2 * fb], act[2 * fb + 1]);
    bias_init(std::integral_constant<int, FB3>{}, BF_3);
    static_for(std::make_integer_sequence<int, KB3 * FB3 / FPS>{}, [&](auto sc) {
      constexpr int s = decltype(sc)::value;
      fetch(1, B1{});
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[i] = E::mma(fa[0][i], act[4 * s], acc[i]);
      refill();
      __builtin_amdgcn_sched_barrier(0);
      fetch(2, B0{});
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[i] = E::mma(fa[1][i], act[4 * s + 1], acc[i]);
      __builtin_amdgcn_sched_barrier(0);
      fetch(3, B1{});
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[i] = E::mma(fa[0][i], act[4 * s + 2], acc[i]);
      __builtin_amdgcn_sched_barrier(0);
      // the next tile's first slot is acquired after this tile's stores
      if constexpr (s + 1 < KB3 * FB3 / FPS) advance();
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[i] = E::mma(fa[1][i], act[4 * s + 3], acc[i]);
    });

    // Output: out[row][f] = act3(acc) for f = 32 fb + 8 g + 4 lh + e.
    // v_permlane32_swap trades groups g = 2q+1 of the lower half-wave for
    // groups g = 2q of the upper one, so each lane holds eight consecutive
    // features 32 fb + 16 q + 8 lh + (0..7) and one 16-byte store per lane
    // writes 32 bytes of each of 32 rows.
    {
      const __amdgpu_buffer_rsrc_t ro = make_rsrc(p.out + r0 * H3, vrows * H3 * 2);
      const int lane = opaque(lane0), lr = lane & 31, lh = lane >> 5;
      const int row = 32 * wave + lr;
#pragma unroll
      for (int fb = 0; fb < FB3; ++fb) {
        u32x2 o[4];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          f4 v;
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = apply_act(acc[fb][4 * g + e], p.act3);
          o[g] = __builtin_bit_cast(u32x2, E::cvt4(v));
        }
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          const auto lo = __builtin_amdgcn_permlane32_swap(o[2 * q][0], o[2 * q + 1][0], false, false);
          const auto hi = __builtin_amdgcn_permlane32_swap(o[2 * q][1], o[2 * q + 1][1], false, false);
          const u32x4 w = {(unsigned)lo[0], (unsigned)hi[0], (unsigned)lo[1], (unsigned)hi[1]};
          buf_store_u4(ro, (row * H3 + 32 * fb + 16 * q + 8 * lh) * 2, w);
        }
      }
    }
  }
  // The ring and input copies issued past the last tile (empty ranges that
  // still write zeros into dead LDS slots) land before the waves exit.
  wait_vmcnt<0>();
}

// ------------------------------------------------------------------ packing
struct PackArgs {
  const half_t* w1;  // [K0][512] (nn.Linear.weight.t())
  const half_t* b1;  // [512] or null
  const half_t* w2;  // [512][256]
  const half_t* b2;
  const half_t* w3;  // [256][128]
  const half_t* b3;
  int K0;
  char* pack;
};

// One thread per 16-byte lane chunk of a fragment (first layer, then the
// slot stream), then one per bias-table entry.
__global__ __launch_bounds__(256) void dlrm_pack_kernel(PackArgs a) {
  constexpr int N_W1 = W1_BYTES / 16, N_ST = ST * SLOT / 16;
  const int gid = blockIdx.x * blockDim.x + threadIdx.x;
  if (gid < N_W1 + N_ST) {
    const bool first = gid < N_W1;
    const int c = first ? gid : gid - N_W1;
    const int f = c / kWave, lane = c % kWave, h = lane >> 5;
    int kb, fb, n;
    const half_t* w;
    if (first) {  // fragment (fb, kb) at 2 fb + kb; inputs in natural order
      fb = f / 2;
      kb = f % 2;
      w = a.w1;
      n = H1;
    } else if (f < S_W3 * FPS) {  // slot j: k-blocks 2j, 2j+1 x feature blocks 0-7
      kb = f / FB2;
      fb = f % FB2;
      w = a.w2;
      n = H2;
    } else {  // slots 16-19: k-blocks 4s .. 4s+3 x feature blocks 0-3
      const int fi = f - S_W3 * FPS;
      kb = fi / FB3;
      fb = fi % FB3;
      w = a.w3;
      n = H3;
    }
    const int out = 32 * fb + (lane & 31);
    h8 v;
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int pp = 8 * h + q;
      const int kin = first ? 16 * kb + pp : 16 * kb + sigma(pp);
      v[q] = (!first || kin < a.K0) ? w[(int64_t)kin * n + out] : (half_t)0.f;
    }
    *(h8*)(a.pack + (first ? 0 : P_STREAM) + (size_t)c * 16) = v;
    return;
  }
  const int t = gid - N_W1 - N_ST;
  if (t >= B_TOTAL) return;
  const int off = t < BF_2 ? BF_1 : t < BF_3 ? BF_2 : BF_3;
  const half_t* b = t < BF_2 ? a.b1 : t < BF_3 ? a.b2 : a.b3;
  const int fb = (t - off) / 64, ln = (t - off) % 64;
  ((half_t*)(a.pack + P_BIAS))[t] = (b && ln < 32) ? b[32 * fb + ln] : (half_t)0.f;
}

// ------------------------------------------------------------------ tail
// The last two layers of the DLRM top MLP (apps/dlrm_topmlp: ... -> K -> 256
// -> 1, the click head) as one persistent kernel: K -> 256 on MFMA with the
// 256 accumulators of a wave's 32 rows in registers, then the one-output
// layer as a dot product in the epilogue.  The reference chains these as
// stage blocks linked by queues (apps/dlrm_topmlp/pipelined/
// dlrm_topmlp_pl.cuh:185-224); here the 256-wide activations never leave the
// CU and the click head needs no launch of its own.
//
//  * Eight waves (two per SIMD) own a 256-row tile, wave w its rows 32w ..
//    32w+31.  The weights stream from L2 as in the bottom MLP: slot j holds
//    k-blocks 2j, 2j+1 for the eight feature blocks (ST = K / 32 slots a
//    tile), here in a ring of TS = 4 slots, every wave copying two of a
//    slot's sixteen fragments.
//  * The layer input comes from HBM straight into registers: the B operand of
//    k-block kb for lane (row lr, half lh) is the 16 bytes x[row][16 kb + 8 lh
//    ..], so each wave loads its own rows, two 16-byte loads per slot, into TS
//    register sets (set = slot % TS; ST is a multiple of TS, so a slot's set
//    does not depend on its tile).
//  * While slot i is computed a wave issues the input loads of slot i + TS - 1
//    and then its ring copies (OPS memory operations), the same order the
//    prologue uses for slots 0 .. TS-2.  vmcnt counts them in issue order, so
//    acquiring slot i waits until at most the (TS - 2) OPS operations issued
//    after slot i's copies are in flight, which also covers slot i's input
//    loads (issued just before its copies).
//  * Epilogue: out[row] = act(sum_f relu?(fp16(acc_f)) w5[f] + b5) -- the
//    hidden values rounded to the element type as a separate layer would
//    store them -- each lane summing its 128 features, v_permlane32_swap
//    adding the other half-wave's.
namespace tail {

constexpr int TS = 4;                 // ring slots = input register sets
constexpr int TCPW = FPS / NW;        // ring copies per wave per slot
constexpr int OPS = 2 + TCPW;         // memory operations per wave per slot
constexpr int kWait = (TS - 2) * OPS;
static_assert(FPS % NW == 0, "copies per wave");
// LDS: ring, bias table (8 feature blocks), head weights (fp32).
constexpr int L_B = TS * SLOT, L_W = L_B + 64 * FB2 * 2, LDS_BYTES = L_W + H2 * 4;
static_assert(LDS_BYTES <= 160 * 1024, "LDS");

// Packed block: ST slots, the bias table, then w5 [256] and b5 as fp32.
constexpr size_t p_bias(int ST) { return (size_t)ST * SLOT; }
constexpr size_t p_head(int ST) { return p_bias(ST) + 64 * FB2 * 2; }
constexpr size_t p_total(int ST) { return p_head(ST) + (H2 + 4) * 4; }

struct TailArgs {
  const half_t* x;   // [M][K]
  const char* pack;  // p_total(K / 32) bytes (dlrm_tail_pack_kernel)
  half_t* out;       // [M] (one output per row)
  int64_t M;
  int relu;          // ReLU after the K -> 256 layer (else identity)
  int act_out;       // activation of the click head (ACT_*)
};

__device__ __forceinline__ h8 buf_load_h8(__amdgpu_buffer_rsrc_t rsrc, int off) {
  return __builtin_bit_cast(h8, __builtin_amdgcn_raw_buffer_load_b128(rsrc, off, 0, 0));
}

template <typename E, int ST>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(2, 2))) void dlrm_tail_kernel(TailArgs p) {
  static_assert(ST % TS == 0, "a slot's input register set must not depend on its tile");
  constexpr int K = 32 * ST;
  __shared__ __attribute__((aligned(1024))) char smem[LDS_BYTES];
  GP_LDS char* const ring = (GP_LDS char*)smem;
  GP_LDS half_t* const bfrag = (GP_LDS half_t*)(smem + L_B);
  GP_LDS float* const w5 = (GP_LDS float*)(smem + L_W);

  const int tid = threadIdx.x;
  const int lane0 = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int G = gridDim.x;
  const int ntiles = (int)((p.M + ROWS - 1) / ROWS);
  const int my = (ntiles - (int)blockIdx.x + G - 1) / G;  // tiles blockIdx.x + k G, k < my

  for (int i = tid; i < 64 * FB2 / 8; i += NT) ((GP_LDS h8*)bfrag)[i] = ((const h8*)(p.pack + p_bias(ST)))[i];
  for (int i = tid; i < H2; i += NT) w5[i] = ((const float*)(p.pack + p_head(ST)))[i];
  const float b5 = ((const float*)(p.pack + p_head(ST)))[H2];
  __syncthreads();

  auto tile_r0 = [&](int k) { return ((int64_t)blockIdx.x + (int64_t)k * G) * ROWS; };
  const int lh = lane0 >> 5;
  const int trow = 32 * wave + (lane0 & 31);  // this lane's row within a tile

  // Input loads of global slot g (this workgroup's tile g / ST, k-blocks
  // 2 (g % ST) and +1) into register set R.  Past the last tile the range is
  // 0: the loads read zeros and every wave keeps the same count in flight.
  h8 xin[TS][2];
  auto load_input = [&](int g, auto rc) {
    constexpr int R = decltype(rc)::value;
    const int kk = g / ST, ls = g % ST;
    const int64_t row0 = tile_r0(kk);
    const int64_t left = kk < my ? p.M - row0 : 0;
    const int rows = left <= 0 ? 0 : left < ROWS ? (int)left : ROWS;
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(p.x + row0 * K, rows * K * 2);
    const int off = (trow * K + 32 * ls + 8 * lh) * 2;
    xin[R][0] = buf_load_h8(rs, off);
    xin[R][1] = buf_load_h8(rs, off + 32);
  };

  // Ring of TS slots: global slot q lives in ring slot q % TS; copying slot q
  // is every wave's TCPW fragments of it.  Past the last tile the range is 0.
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(p.pack, ST * SLOT);
  auto issue = [&](int q) {
    const int kk = q / ST, ls = q % ST;
    const __amdgpu_buffer_rsrc_t r = kk < my ? rw : make_rsrc(p.pack, 0);
    GP_LDS char* const dst = ring + (q % TS) * SLOT;
#pragma unroll
    for (int i = 0; i < TCPW; ++i) {
      const int c = NW * i + wave;
      dma16_buf_so(r, 16 * lane0, ls * SLOT + c * FRAG, dst + c * FRAG);
    }
  };
  // Prologue: slots 0 .. TS-2, inputs then copies, as a slot's iteration
  // issues them.
  static_for(std::make_integer_sequence<int, TS - 1>{}, [&](auto uc) {
    load_input(decltype(uc)::value, uc);
    issue(decltype(uc)::value);
  });

  f16x acc[FB2];
  // A fragments, double-buffered as in the bottom MLP: group g + 1 is read
  // while group g's MFMAs issue, and a slot's last group issues after the
  // next slot's barrier.
  h8 fa[2][4];
  h8 ones = {};
  ones[0] = __builtin_bit_cast(half_t, lane0 < 32 ? E::kOne : (unsigned short)0);
  using B0 = std::integral_constant<int, 0>;
  using B1 = std::integral_constant<int, 1>;
  // Read group g of ring slot RS into fa[BUF].
  auto fetch = [&](auto rsc, int g, auto bufc) {
    constexpr int RS = decltype(rsc)::value, BUF = decltype(bufc)::value;
    GP_LDS const char* const s = (GP_LDS const char*)(ring + RS * SLOT) + 16 * lane0;
#pragma unroll
    for (int i = 0; i < 4; ++i) fa[BUF][i] = *(GP_LDS const h8*)(s + (4 * g + i) * FRAG);
  };
  // Acquire the next slot in stream order (all but the kWait operations
  // issued after its copies have landed -- its input loads among them -- then
  // a barrier) and read its group 0.
  auto acquire = [&](auto rsc) {
    wait_vmcnt<kWait>();
    lds_barrier();
    fetch(rsc, 0, B0{});
  };

  for (int k = 0; k < my; ++k) {
    const int64_t r0 = tile_r0(k);
    const int vrows = p.M - r0 < ROWS ? (int)(p.M - r0) : ROWS;
#pragma unroll
    for (int fb = 0; fb < FB2; ++fb) {
      h8 a = {};
      a[0] = bfrag[64 * fb + lane0];
      acc[fb] = E::mma(a, ones, f16x{});
    }
    // the tile's first slot (ring slot 0: ST is a multiple of TS)
    acquire(std::integral_constant<int, 0>{});
#pragma nounroll
    for (int grp = 0; grp < ST / TS; ++grp) {
      const int i0 = k * ST + grp * TS;  // global slot of the group's first slot
      const bool last_grp = grp + 1 == ST / TS;
      static_for(std::make_integer_sequence<int, TS>{}, [&](auto uc) {
        constexpr int u = decltype(uc)::value;
        using RS = std::integral_constant<int, u>;
        // slot i0 + u is acquired (ring slot u) and its group 0 is in fa[0]
        fetch(RS{}, 1, B1{});
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i] = E::mma(fa[0][i], xin[u][0], acc[i]);
        // slot i0 + u + TS - 1 goes into the ring slot and register set of
        // slot i0 + u - 1, both dead since the barrier
        load_input(i0 + u + TS - 1, std::integral_constant<int, (u + TS - 1) % TS>{});
        issue(i0 + u + TS - 1);
        __builtin_amdgcn_sched_barrier(0);
        fetch(RS{}, 2, B0{});
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[4 + i] = E::mma(fa[1][i], xin[u][0], acc[4 + i]);
        __builtin_amdgcn_sched_barrier(0);
        fetch(RS{}, 3, B1{});
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i] = E::mma(fa[0][i], xin[u][1], acc[i]);
        __builtin_amdgcn_sched_barrier(0);
        // the next slot of this tile (the next tile's first is acquired after
        // this tile's output store)
        if (u + 1 < TS || !last_grp) acquire(std::integral_constant<int, (u + 1) % TS>{});
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[4 + i] = E::mma(fa[1][i], xin[u][1], acc[4 + i]);
      });
    }
    // Click head.  Lane (row, half lh) holds features 32 fb + 8 g + 4 lh + e
    // in element 4 g + e of block fb.
    float sum = 0.f;
#pragma unroll
    for (int fb = 0; fb < FB2; ++fb) {
      h8 lo, hi;
      to_operands<E>(acc[fb], p.relu != 0, lo, hi);
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const f4 w = *(GP_LDS const f4*)(w5 + 32 * fb + 8 * g + 4 * lh);
#pragma unroll
        for (int e = 0; e < 4; ++e) sum = __builtin_fmaf(E::val(g < 2 ? lo[4 * g + e] : hi[4 * g - 8 + e]), w[e], sum);
      }
    }
    sum = sum_lane_halves(sum);
    const unsigned short o = __builtin_bit_cast(unsigned short, E::cvt1(apply_act(sum + b5, p.act_out)));
    // lanes of the upper half store past the range (dropped): one store
    // instruction per wave and tile, whatever the row count
    const __amdgpu_buffer_rsrc_t ro = make_rsrc(p.out + r0, vrows * 2);
    __builtin_amdgcn_raw_buffer_store_b16(o, ro, lh == 0 ? 2 * trow : 2 * ROWS, 0, 0);
  }
  // The copies and loads issued past the last tile land before the waves exit.
  wait_vmcnt<0>();
}

struct TailPackArgs {
  const half_t* w4;  // [K][256]
  const half_t* b4;  // [256] or null
  const half_t* w5;  // [256] (the [256, 1] weight)
  const half_t* b5;  // [1] or null
  int ST;
  char* pack;
};

// One thread per 16-byte lane chunk of the slot stream, then one per bias
// entry, then one per head weight (and b5).
template <typename E>
__global__ __launch_bounds__(256) void dlrm_tail_pack_kernel(TailPackArgs a) {
  const int gid = blockIdx.x * blockDim.x + threadIdx.x;
  const int nst = a.ST * SLOT / 16;
  if (gid < nst) {
    const int f = gid / kWave, lane = gid % kWave, h = lane >> 5;
    const int kb = f / FB2, fb = f % FB2;  // slot j: k-blocks 2j, 2j+1 x feature blocks 0-7
    const int out = 32 * fb + (lane & 31);
    h8 v;
#pragma unroll
    for (int q = 0; q < 8; ++q) v[q] = a.w4[(int64_t)(16 * kb + 8 * h + q) * H2 + out];
    *(h8*)(a.pack + (size_t)gid * 16) = v;
    return;
  }
  const int t = gid - nst;
  if (t < 64 * FB2) {
    const int fb = t / 64, ln = t % 64;
    ((half_t*)(a.pack + p_bias(a.ST)))[t] = (a.b4 && ln < 32) ? a.b4[32 * fb + ln] : (half_t)0.f;
    return;
  }
  const int hI = t - 64 * FB2;
  float* const head = (float*)(a.pack + p_head(a.ST));
  if (hI < H2) head[hI] = E::val(a.w5[hI]);
  else if (hI == H2) head[H2] = a.b5 ? E::val(a.b5[0]) : 0.f;
}

}  // namespace tail
}  // namespace dlrm

size_t dlrm_tail_workspace(int64_t K) { return dlrm::tail::p_total((int)(K / 32)); }

hipError_t dlrm_tail_launch(int64_t M, int64_t K, const void* x, const void* w4, const void* b4, int act4,
                            const void* w5, const void* b5, int act5, void* out, void* ws, int num_cus,
                            hipStream_t s, int dtype, bool pack) {
  using namespace dlrm;
  using namespace dlrm::tail;
  if (dtype != GP_DTYPE_F16 && dtype != GP_DTYPE_BF16) return hipErrorInvalidValue;
  if (M <= 0) return hipSuccess;
  if (M > (int64_t(1) << 31) - 1 || !dlrm_tail_supported(K, act4, act5)) return hipErrorInvalidValue;
  if (((uintptr_t)x & 15) || ((uintptr_t)ws & 15) || ((uintptr_t)out & 1)) return hipErrorInvalidValue;
  const int ST = (int)(K / 32);
  TailPackArgs pa{(const half_t*)w4, (const half_t*)b4, (const half_t*)w5, (const half_t*)b5, ST, (char*)ws};
  const int nthreads = ST * SLOT / 16 + 64 * FB2 + H2 + 1;
  if (pack) {
    if (dtype == GP_DTYPE_BF16)
      hipLaunchKernelGGL(dlrm_tail_pack_kernel<BF16>, dim3((nthreads + 255) / 256), dim3(256), 0, s, pa);
    else
      hipLaunchKernelGGL(dlrm_tail_pack_kernel<F16>, dim3((nthreads + 255) / 256), dim3(256), 0, s, pa);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  const TailArgs a{(const half_t*)x, (const char*)ws, (half_t*)out, M, act4 == GP_ACT_RELU, act5};
  const int64_t tiles = (M + ROWS - 1) / ROWS;
  const dim3 grid((unsigned)(tiles < num_cus ? tiles : num_cus));
#define GP_TAIL(T, S) hipLaunchKernelGGL((dlrm_tail_kernel<T, S>), grid, dim3(NT), 0, s, a)
  if (dtype == GP_DTYPE_BF16) {
    if (ST == 8) GP_TAIL(BF16, 8);
    else if (ST == 16) GP_TAIL(BF16, 16);
    else GP_TAIL(BF16, 32);
  } else {
    if (ST == 8) GP_TAIL(F16, 8);
    else if (ST == 16) GP_TAIL(F16, 16);
    else GP_TAIL(F16, 32);
  }
#undef GP_TAIL
  return hipGetLastError();
}

size_t dlrm_bot_workspace() { return dlrm::P_TOTAL; }

hipError_t dlrm_bot_launch(int64_t M, int K0, const void* x, const void* const* w, const void* const* b,
                           const int* acts, void* out, void* ws, int num_cus, hipStream_t s, int dtype) {
  using namespace dlrm;
  if (dtype != GP_DTYPE_F16 && dtype != GP_DTYPE_BF16) return hipErrorInvalidValue;
  if (M <= 0) return hipSuccess;
  if (M > (int64_t(1) << 31) - 1 || !dlrm_bot_supported(K0, acts)) return hipErrorInvalidValue;
  if (((uintptr_t)x & 15) || ((uintptr_t)out & 15) || ((uintptr_t)ws & 15)) return hipErrorInvalidValue;
  PackArgs pa{(const half_t*)w[0], (const half_t*)b[0], (const half_t*)w[1], (const half_t*)b[1],
              (const half_t*)w[2], (const half_t*)b[2], K0, (char*)ws};
  const int nthreads = W1_BYTES / 16 + ST * SLOT / 16 + B_TOTAL;
  hipLaunchKernelGGL(dlrm_pack_kernel, dim3((nthreads + 255) / 256), dim3(256), 0, s, pa);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const Args a{(const half_t*)x, (const char*)ws, (half_t*)out, M, K0,
               acts[0] == GP_ACT_RELU, acts[1] == GP_ACT_RELU, acts[2]};
  const int64_t tiles = (M + ROWS - 1) / ROWS;
  const dim3 grid((unsigned)(tiles < num_cus ? tiles : num_cus));
  const bool two = K0 > 16;
  if (dtype == GP_DTYPE_BF16) {
    if (two)
      hipLaunchKernelGGL((dlrm_bot_kernel<BF16, 2>), grid, dim3(NT), 0, s, a);
    else
      hipLaunchKernelGGL((dlrm_bot_kernel<BF16, 1>), grid, dim3(NT), 0, s, a);
  } else {
    if (two)
      hipLaunchKernelGGL((dlrm_bot_kernel<F16, 2>), grid, dim3(NT), 0, s, a);
    else
      hipLaunchKernelGGL((dlrm_bot_kernel<F16, 1>), grid, dim3(NT), 0, s, a);
  }
  return hipGetLastError();
}

}  // namespace gp
