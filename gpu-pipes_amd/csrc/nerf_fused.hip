// The NeRF MLP as one persistent gfx950 kernel: all twelve layers of a
// 256-row tile run back to back without their activations leaving the CU.
//
// Semantics: apps/nerf_full/torch/model.py:5-66 (hidden 256, skip after the
// fifth layer, density head, bottleneck, colour branch).  The reference runs
// it as one pipelined kernel of fourteen GEMM / concat stage blocks linked by
// queues (apps/nerf_full/pipelined/nerf_full_pl.cuh:122-274); here the stages
// of one tile are a single wave's instruction stream instead.
//
// Design.
//  * A workgroup of eight waves (two per SIMD) owns a tile of 256 rows; wave
//    w owns rows 32w .. 32w+31 and computes every output feature of every
//    layer for them, as C^T = W^T X^T with
//    v_mfma_f32_32x32x16_f16: the MFMA A operand is a 32-feature x 16-k block
//    of the weights (a "fragment"), the B operand a 16-k x 32-row block of the
//    layer input.
//  * Activations stay in registers.  A 256-feature layer's accumulators take
//    128 registers; converted to fp16 they take 64, in exactly the
//    register layout of the next layer's B operands, because the accumulator
//    lane layout (4 features x 4 groups of one row) is a permutation of the B
//    operand layout (8 consecutive k of one row).  The permutation is folded
//    into the weight packing: B position p = 8h + q of k-block kb holds input
//    feature 16 kb + sigma(p), sigma swapping the middle two groups of four.
//  * Weights (1.2 MB) do not fit on chip, so every tile streams them from L2:
//    the host packs all layers once per call into the exact order the kernel
//    consumes them, as 1 KiB fragments (64 lanes x 16 bytes), 16 to a 16 KiB
//    slot.  Waves 0-3 copy slots L2 -> LDS with buffer_load ... lds into a
//    ring of six (96 KiB); four are in flight while one is read.  Every slot
//    is dead once the next one is acquired, so the bookkeeping is fixed:
//    acquiring slot q waits for this wave's copies of q (the 16 copies issued
//    after them may still be in flight) and passes one workgroup barrier,
//    after which no wave reads slot q-1 again; slot q+5 is copied into q-1's
//    place once slot q's first MFMAs are issued.
//  * The network inputs come through their own LDS tiles (x 32 KiB, d 16
//    KiB), copied by waves 4-7 a whole stretch of layers ahead: the next
//    tile's x once layer 6 has read this tile's, its d once layer 11 has.
//    Only waves 4-7 copy them, so their HBM latency never holds up a wait
//    for a ring slot (vmcnt counts a wave's own loads, in order).
//  * Bias of a hidden layer: one extra MFMA per accumulator block, the bias
//    fragment (bias in k = 0) times a constant B operand that is 1 in k = 0,
//    is each accumulator's first product, so the epilogue is only the fp16
//    conversion and ReLU (in packed fp16: max commutes with RNE rounding).
//    A SIMD issues at most one VALU instruction every four cycles, so an MFMA
//    (32 cycles of the matrix pipe) in place of 16 VALU adds is the cheaper
//    side.  With two waves per SIMD, one wave's epilogue, copies and scalar
//    work issue while the other's MFMAs run.
//  * The density and colour heads add their bias in fp32 and are stored
//    through buffer descriptors bounded to the tile's valid rows.
#include <hip/hip_runtime.h>

#include <mutex>
#include <type_traits>
#include <utility>

#include "../../include/gpipes.h"
#include "gp_device.hpp"
#include "gp_host.hpp"
#include "gp_kernels.hpp"
#include "stages.hpp"

namespace gp {
namespace nerf {

constexpr int NW = 8;              // waves per workgroup, two per SIMD
constexpr int RB = 1;              // 32-row blocks per wave
constexpr int NT = NW * kWave;
constexpr int ROWS = 32 * RB * NW; // rows per tile
constexpr int FRAG = 1024;         // one A operand: 64 lanes x 16 bytes
constexpr int FPS = 16;            // fragments per slot
constexpr int SLOT = FPS * FRAG;   // bytes per ring slot
constexpr int NS = 6;              // ring slots
constexpr int RW = 4;              // waves 0 .. RW-1 copy the ring; the others copy x and d
constexpr int CPW = FPS / RW;      // 1 KiB ring copies per copying wave per slot
constexpr int XBUF = ROWS * 64 * 2;  // one tile of x (Kx <= 64)
constexpr int DBUF = ROWS * 32 * 2;  // one tile of d (Kd <= 32)
constexpr int XCPW = XBUF / FRAG / (NW - RW), DCPW = DBUF / FRAG / (NW - RW);  // input copies per wave
constexpr int kOutStores = 8 * 2 * RB;  // trunk output stores per wave and tile (epi_out)

// Local slot map of one tile's weight stream (76 slots, 1.25 MB).
constexpr int S_L1 = 0, S_L2 = 2, S_L6 = 34, S_L7 = 44, S_L9 = 60, S_L10 = 62, S_L11 = 70, S_L12 = 75, S_TOTAL = 76;

// Bias tables (fp16 in global memory).  Hidden layers: per feature block fb a
// 64-entry A-operand column, bias[32 fb + lane] for lanes < 32 and 0 for the
// upper half (k = 8..15).  Heads: plain vectors of 64.
constexpr int BF_L1 = 0, BF_L2 = 512, BF_L6 = 2560, BF_L7 = 3072, BF_L10 = 4096, BF_L11 = 4608, BF_END = 4864;
constexpr int BH_L9 = BF_END, BH_L12 = BF_END + 64, B_TOTAL = BF_END + 128;
// LDS: ring, x tile, d tile, the hidden-layer bias table as fp16, then the
// head biases as fp32.
constexpr int BIAS_BYTES = BF_END * 2 + 128 * 4;
constexpr int L_X = NS * SLOT, L_D = L_X + XBUF, L_B = L_D + DBUF, LDS_BYTES = L_B + BIAS_BYTES;
static_assert(LDS_BYTES <= 160 * 1024, "LDS");

struct Args {
  const half_t* x;       // [M][Kx]
  const half_t* d;       // [M][Kd]
  const char* stream;    // S_TOTAL slots
  const half_t* bias;    // B_TOTAL
  half_t* out_r;         // [M][Na]
  half_t* out_rgb;       // [M][Nrgb]
  int64_t M;
  int Kx, Kd, Na, Nrgb, rgb_act;
};

// B-operand k-order of a k-block fed from registers: position p holds input
// feature 16 kb + sigma(p) (the accumulator layout of the layer before).
__host__ __device__ constexpr int sigma(int p) { return p < 4 ? p : p < 8 ? p + 4 : p < 12 ? p - 4 : p; }

// Slot kinds.  A slot holds 16 fragments of one layer, read and multiplied
// as four groups of four: FB feature blocks per input k-block, starting at
// k-block KB0; the layer's first NEXT k-blocks take their B operand from the
// x or d tile, the rest from registers; HB: the layer's bias enters through
// the MFMA (hidden layers).
//   1-2 layer 1, 3-10 a 256 -> 256 layer, 11-20 layer 6, 21-22 layer 9,
//   23-27 layer 11, 28 layer 12.
struct Kind {
  int fb, kb0, next, hb;
};
__host__ __device__ constexpr Kind kind_info(int k) {
  return k <= 2    ? Kind{8, 2 * (k - 1), 4, 1}
         : k <= 10 ? Kind{8, 2 * (k - 3), 0, 1}
         : k <= 20 ? Kind{8, 2 * (k - 11), 4, 1}
         : k <= 22 ? Kind{2, 8 * (k - 21), 0, 0}
         : k <= 27 ? Kind{4, 4 * (k - 23), 4, 1}
                   : Kind{2, 0, 0, 0};
}

template <int... I, class F>
__device__ __forceinline__ void static_for(std::integer_sequence<int, I...>, F&& f) {
  (f(std::integral_constant<int, I>{}), ...);
}

// E: F16 or BF16, the element type of x, d, the weights, biases and outputs.
// TRUNK: only layers 1-8 (NerfA, apps/nerf_a/torch/model.py:5-38): the weight
// stream ends before the density head, no d is read, and out_r receives the
// trunk's ReLU output, [M][256].
template <typename E, bool TRUNK = false>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(2, 2))) void nerf_fused_kernel(Args p) {
  constexpr int ST = TRUNK ? S_L9 : S_TOTAL;  // slots per tile
  __shared__ __attribute__((aligned(1024))) char smem[LDS_BYTES];
  GP_LDS char* const ring = (GP_LDS char*)smem;
  GP_LDS half_t* const bfrag = (GP_LDS half_t*)(smem + L_B);
  GP_LDS float* const bhead = (GP_LDS float*)(smem + L_B + BF_END * 2);

  const int tid = threadIdx.x;
  const int lane0 = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool ring_wave = wave < RW;
  const int G = gridDim.x;
  // Tile and slot counts fit in 32 bits: the host limits M to 2^31 - 1.
  const int ntiles = (int)((p.M + ROWS - 1) / ROWS);
  const int my = (ntiles - (int)blockIdx.x + G - 1) / G;  // tiles blockIdx.x + k G, k < my

  for (int i = tid; i < BF_END / 8; i += NT) ((GP_LDS h8*)bfrag)[i] = ((const h8*)p.bias)[i];
  if (tid < 128) bhead[tid] = E::val(p.bias[BF_END + tid]);
  __syncthreads();

  auto tile_r0 = [&](int k) { return ((int64_t)blockIdx.x + (int64_t)k * G) * ROWS; };

  // ---------------------------------------------------------- input tiles
  // Waves RW .. NW-1 copy tile k's x rows (or d rows) into the x (d) buffer,
  // chunk c = (NW - RW) i + (wave - RW) being copy i.  A tile past the last
  // one copies nothing (range 0) and only zeroes a dead buffer, so every such
  // wave always has the same copies in flight: x of tile k+1 is issued after
  // layer 6 of tile k, d of tile k+1 after layer 11.
  auto copy_input = [&](int k, bool is_x) {
    if (ring_wave) return;
    const int K = is_x ? p.Kx : p.Kd;
    const int64_t row0 = tile_r0(k);
    const int64_t left = k < my ? p.M - row0 : 0;
    const int rows = left <= 0 ? 0 : left < ROWS ? (int)left : ROWS;
    // The range is rounded up to whole 16-byte copies; the bytes past the last
    // valid row lie in the same 16-byte block (so the same page) and land only
    // in rows that are never stored.
    const __amdgpu_buffer_rsrc_t r = make_rsrc((is_x ? p.x : p.d) + row0 * K, (rows * K * 2 + 15) & ~15);
    GP_LDS char* const dst = (GP_LDS char*)smem + (is_x ? L_X : L_D);
    const int n = is_x ? XCPW : DCPW;
    for (int i = 0; i < n; ++i) {
      const int c = (NW - RW) * i + (wave - RW);
      dma16_buf_so(r, 16 * lane0, c * FRAG, dst + c * FRAG);
    }
  };

  // ---------------------------------------------------------------- ring
  // Global slot q = k ST + l (tile k, local slot l) lives in ring slot
  // q % NS.  `cur` is the ring slot of the last acquired slot; (iss_k, iss_l)
  // the next slot to copy, which goes to ring slot (cur + NS - 1) % NS.
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(p.stream, ST * SLOT);
  int cur = NS - 1, iss_k = 0, iss_l = 0;
  // Copy the next slot into ring slot `rs` (ring waves; chunk c = RW i + wave
  // is copy i).  Branch-free apart from the wave test, so that a slot's MFMAs
  // and its copies form one basic block the scheduler can interleave.  Past
  // the last slot (iss_k == my) the range is 0: the copies read nothing and
  // zero a dead slot, and every acquire finds the same copies in flight.
  auto issue = [&](int rs) {
    const __amdgpu_buffer_rsrc_t r = iss_k < my ? rw : make_rsrc(p.stream, 0);
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
  // Order of the first copies: x and d of tile 0, then the ring.
  copy_input(0, true);
  if constexpr (!TRUNK) copy_input(0, false);
  for (int i = 0; i < NS - 1; ++i) issue(i);
  // Acquire the next slot in stream order: a ring wave waits for its own
  // copies of it (the CPW (NS - 2) copies issued after them may still be in
  // flight; an input wave has at most XCPW + DCPW < that in flight, so the
  // wait is a no-op for it), then one barrier.  The copy that refills the
  // ring slot of the previous one (dead from the barrier on) is issued by
  // refill(), after the first MFMAs of the new slot.  Every acquire is
  // followed by exactly one refill() before the next acquire.
  static_assert(XCPW + DCPW <= CPW * (NS - 2), "input copies in flight");
  // OUT_STORES: the trunk's output stores of the previous tile (issued after
  // every ring copy still in flight, and counted by vmcnt in issue order like
  // them) are left in flight too.
  auto acquire = [&](auto out_stores) {
    wait_vmcnt<CPW * (NS - 2) + decltype(out_stores)::value>();
    lds_barrier();
    cur = cur == NS - 1 ? 0 : cur + 1;
  };
  auto refill = [&] { issue(cur == 0 ? NS - 1 : cur - 1); };

  f16x acc[8][RB];  // [feature block][row block]
  h8 act[16][RB];   // B operands of register-fed k-blocks: [k-block][row block]
  h8 xin[4][RB];    // B operands of the x / d k-blocks: [k-block][row block]
  h8 fa[2][4];     // A fragments, double-buffered (see run_layer)
  // B operand that is 1 at k = 0 and 0 elsewhere: lanes 0-31 hold k = 0..7.
  h8 ones = {};
  ones[0] = __builtin_bit_cast(half_t, lane0 < 32 ? E::kOne : (unsigned short)0);

  for (int k = 0; k < my; ++k) {
    const int64_t r0 = tile_r0(k);
    const int vrows = p.M - r0 < ROWS ? (int)(p.M - r0) : ROWS;

    auto cur_slot = [&] { return (GP_LDS const char*)(ring + cur * SLOT); };

    // Read this wave's rows of the x (d) tile, K columns per row, into xin
    // (NKB k-blocks; zero for columns >= K and k-blocks past NKB).  Called
    // right after an acquire whose barrier follows the input waves' wait for
    // the tile's copies.
    auto take_input = [&](bool is_x, int K) {
      GP_LDS const char* const b = (GP_LDS const char*)smem + (is_x ? L_X : L_D);
      const int nkb = is_x ? 4 : 2;
      const int lane = opaque(lane0), lr = lane & 31, lh = lane >> 5;
      // K as an opaque vector value: the column masks below are rebuilt here
      // instead of being hoisted out of the tile loop (dozens of live lane
      // masks would spill).
      const int Kv = opaque(K);
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        const int e0 = (32 * RB * wave + 32 * rb + lr) * Kv + 8 * lh;
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
          // valid halves of this lane's 8 columns 16 kb + 8 lh ..
          const int n = kb < nkb ? min(max(Kv - 16 * kb - 8 * lh, 0), 8) : 0;
          h8 v = {};
          if (kb < nkb) {
            if ((K & 7) == 0) {
              v = *(GP_LDS const h8*)(b + (e0 + 16 * kb) * 2);
            } else {
#pragma unroll
              for (int e = 0; e < 8; ++e) v[e] = *(GP_LDS const half_t*)(b + (e0 + 16 * kb + e) * 2);
            }
          }
          u32x4 w = __builtin_bit_cast(u32x4, v);
#pragma unroll
          for (int i = 0; i < 4; ++i) w[i] &= n >= 2 * i + 2 ? 0xffffffffu : n == 2 * i + 1 ? 0xffffu : 0u;
          xin[kb][rb] = __builtin_bit_cast(h8, w);
        }
      }
    };

    // Read group g (fragments 4g .. 4g+3) of the current slot into fa[BUF].
    auto fetch = [&](auto gc, auto bufc) {
      constexpr int g = decltype(gc)::value, buf = decltype(bufc)::value;
      GP_LDS const char* const s = cur_slot() + 4 * g * FRAG + 16 * lane0;
#pragma unroll
      for (int i = 0; i < 4; ++i) fa[buf][i] = *(GP_LDS const h8*)(s + i * FRAG);
    };
    // The 8 MFMAs of group g of a slot of kind KD (4 fragments x 2 row blocks).
    auto mma = [&](auto kdc, auto gc, auto bufc) {
      constexpr Kind K = kind_info(decltype(kdc)::value);
      constexpr int g = decltype(gc)::value, buf = decltype(bufc)::value;
      static_for(std::make_integer_sequence<int, 4>{}, [&](auto ic) {
        constexpr int i = decltype(ic)::value;
        constexpr int fi = K.kb0 * K.fb + 4 * g + i;
        constexpr int kb = fi / K.fb, fb = fi % K.fb;
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
          h8 b;
          if constexpr (kb < K.next) b = xin[kb][rb];
          else b = act[kb - K.next][rb];
          acc[fb][rb] = E::mma(fa[buf][i], b, (kb == 0 && !K.hb) ? f16x{} : acc[fb][rb]);
        }
      });
    };
    // Hidden-layer bias: acc[fb][rb] = bias (x) ones, the first product of
    // every accumulator of the layer.
    auto bias_init = [&](auto FBc, int off) {
      constexpr int FB = decltype(FBc)::value;
#pragma unroll
      for (int fb = 0; fb < FB; ++fb) {
        h8 a = {};
        a[0] = bfrag[off + 64 * fb + lane0];
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) acc[fb][rb] = E::mma(a, ones, f16x{});
      }
    };
    using G0 = std::integral_constant<int, 0>;
    using G1 = std::integral_constant<int, 1>;
    using G2 = std::integral_constant<int, 2>;
    using G3 = std::integral_constant<int, 3>;

    // Hidden-layer epilogue: act[2 fb + s][rb] = relu?(acc) as 16-bit values.
    // Lane (row lr, half lh) holds, in element 4 g + e of block fb, feature
    // 32 fb + 8 g + 4 lh + e.  In bf16 the ReLU is a signed 16-bit integer
    // max on the rounded bits: a bf16 value with its sign bit set is a
    // negative integer and becomes +0, every other value stays.
    auto epi_hidden = [&](auto FBc, bool relu) {
      constexpr int FB = decltype(FBc)::value;
#pragma unroll
      for (int fb = 0; fb < FB; ++fb)
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
          h8 lo, hi;
          if constexpr (std::is_same_v<E, F16>) {
#pragma unroll
            for (int r = 0; r < 8; ++r) {
              lo[r] = (half_t)acc[fb][rb][r];
              hi[r] = (half_t)acc[fb][rb][8 + r];
            }
            if (relu) {
              lo = __builtin_elementwise_max(lo, h8{});
              hi = __builtin_elementwise_max(hi, h8{});
            }
          } else {
            const f16x& a = acc[fb][rb];
            lo = __builtin_shufflevector(E::cvt4(f4{a[0], a[1], a[2], a[3]}), E::cvt4(f4{a[4], a[5], a[6], a[7]}), 0, 1,
                                         2, 3, 4, 5, 6, 7);
            hi = __builtin_shufflevector(E::cvt4(f4{a[8], a[9], a[10], a[11]}), E::cvt4(f4{a[12], a[13], a[14], a[15]}),
                                         0, 1, 2, 3, 4, 5, 6, 7);
            if (relu) {
              lo = __builtin_bit_cast(h8, __builtin_elementwise_max(__builtin_bit_cast(s8, lo), s8{}));
              hi = __builtin_bit_cast(h8, __builtin_elementwise_max(__builtin_bit_cast(s8, hi), s8{}));
            }
          }
          act[2 * fb][rb] = lo;
          act[2 * fb + 1][rb] = hi;
        }
    };

    // Head epilogue: out[row][c] = fn(acc + bias) for c < N, rows < vrows.
    auto epi_head = [&](int boff, half_t* out, int N, int fn) {
      const __amdgpu_buffer_rsrc_t ro = make_rsrc(out + r0 * N, vrows * N * 2);
      const bool vec = (N & 3) == 0 && ((uintptr_t)out & 7) == 0;
      // Lane id and N as opaque values: the row / column indices and masks are
      // built here, where they are used, rather than early in the tile and
      // kept live through ten layers.
      const int lane = opaque(lane0), lr = lane & 31, lh = lane >> 5;
      const int Nv = opaque(N);
#pragma unroll
      for (int fb = 0; fb < 2; ++fb)
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
          const int row = 32 * RB * wave + 32 * rb + lr;
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const int c = 32 * fb + 8 * g + 4 * lh;
            const f4 bb = *(GP_LDS const f4*)(bhead + boff + c);
            f4 v;
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = apply_act(acc[fb][rb][4 * g + e] + bb[e], fn);
            const h4 h = E::cvt4(v);
            const int off = (row * Nv + c) * 2;
            if (vec) {
              if (c < Nv) buf_store_h4(ro, off, h);
            } else {
              // 16-bit words taken out with integer shifts: the b16 store of a
              // bit-cast vector element was compiled to store element 0 each time.
              const u32x2 w2 = __builtin_bit_cast(u32x2, h);
#pragma unroll
              for (int e = 0; e < 4; ++e)
                if (c + e < Nv)
                  __builtin_amdgcn_raw_buffer_store_b16((unsigned short)(w2[e >> 1] >> (16 * (e & 1))), ro, off + 2 * e,
                                                        0, 0);
            }
          }
        }
    };

    // Trunk output (TRUNK): out[row][f] = ReLU(acc) for the layer-8
    // accumulators, f = 32 fb + 8 g + 4 lh + e.  v_permlane32_swap trades
    // groups g = 2q+1 of the lower half-wave for groups g = 2q of the upper
    // one, so each lane holds eight consecutive features 32 fb + 16 q + 8 lh +
    // (0..7) and one 16-byte store per lane writes 32 bytes of each of 32 rows.
    // Each wave issues kOutStores 16-byte stores (8 feature blocks x 2).
    auto epi_out = [&] {
      const __amdgpu_buffer_rsrc_t ro = make_rsrc(p.out_r + r0 * 256, vrows * 256 * 2);
      const int lane = opaque(lane0), lr = lane & 31, lh = lane >> 5;
#pragma unroll
      for (int fb = 0; fb < 8; ++fb)
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
          const int row = 32 * RB * wave + 32 * rb + lr;
          u32x2 o[4];
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            f4 v;
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = __builtin_fmaxf(acc[fb][rb][4 * g + e], 0.f);
            o[g] = __builtin_bit_cast(u32x2, E::cvt4(v));
          }
#pragma unroll
          for (int q = 0; q < 2; ++q) {
            const auto lo = __builtin_amdgcn_permlane32_swap(o[2 * q][0], o[2 * q + 1][0], false, false);
            const auto hi = __builtin_amdgcn_permlane32_swap(o[2 * q][1], o[2 * q + 1][1], false, false);
            const u32x4 w = {(unsigned)lo[0], (unsigned)hi[0], (unsigned)lo[1], (unsigned)hi[1]};
            buf_store_u4(ro, (row * 256 + 32 * fb + 16 * q + 8 * lh) * 2, w);
          }
        }
    };

    // Slot program.  A slot is 4 groups of 4 fragments, read and multiplied
    // in turn; the next slot is acquired and its first group read right after
    // the last group's MFMAs are issued -- across layer boundaries too, where
    // the epilogue runs after the next layer's first fragments were requested.
    // Acquire the next slot and read its first group.
    using S0 = std::integral_constant<int, 0>;
    auto advance = [&] {
      acquire(S0{});
      fetch(G0{}, G0{});
    };
    // The N slots of one layer, of kinds KD0 .. KD0+N-1; `after` acquires what
    // follows the layer, between the last slot's parts.
    auto run_layer = [&](auto kd0c, auto nc, auto&& after) {
      constexpr int KD0 = decltype(kd0c)::value, N = decltype(nc)::value;
      static_for(std::make_integer_sequence<int, N>{}, [&](auto jc) {
        constexpr int j = decltype(jc)::value;
        using KD = std::integral_constant<int, KD0 + j>;
        // Two fragment buffers: group g + 1 is read while group g's MFMAs
        // issue, and the slot's last group issues after the next slot's
        // barrier (its fragments are in registers by then).
        fetch(G1{}, G1{});
        mma(KD{}, G0{}, G0{});
        refill();
        __builtin_amdgcn_sched_barrier(0);
        fetch(G2{}, G0{});
        mma(KD{}, G1{}, G1{});
        __builtin_amdgcn_sched_barrier(0);
        fetch(G3{}, G1{});
        mma(KD{}, G2{}, G0{});
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (j + 1 < N) advance();
        else after();
        mma(KD{}, G3{}, G1{});
      });
    };
    using C1 = std::integral_constant<int, 1>;
    using C2 = std::integral_constant<int, 2>;
    using C3 = std::integral_constant<int, 3>;
    using C5 = std::integral_constant<int, 5>;
    using C8 = std::integral_constant<int, 8>;
    using C10 = std::integral_constant<int, 10>;
    using C11 = std::integral_constant<int, 11>;
    using C21 = std::integral_constant<int, 21>;
    using C23 = std::integral_constant<int, 23>;
    using C28 = std::integral_constant<int, 28>;
    using E4 = std::integral_constant<int, 4>;
    using E8 = std::integral_constant<int, 8>;
    auto nothing = [] {};

    // Layer 1: x -> 256, ReLU.  The input waves wait for this tile's x copies
    // (this tile's d copies, issued after them, may still be in flight; in the
    // trunk, the previous tile's output stores, issued after them); the
    // acquire's barrier then publishes the x tile.
    if constexpr (TRUNK) {
      if (k == 0) {
        if (!ring_wave) wait_vmcnt<0>();
        advance();
      } else {
        if (!ring_wave) wait_vmcnt<kOutStores>();
        acquire(std::integral_constant<int, kOutStores>{});
        fetch(G0{}, G0{});
      }
    } else {
      if (!ring_wave) wait_vmcnt<DCPW>();
      advance();
    }
    take_input(true, p.Kx);
    bias_init(E8{}, BF_L1);
    run_layer(C1{}, C2{}, [&] { advance(); });
    epi_hidden(E8{}, true);
    // Layers 2-5, 7, 8 (ReLU) and 10 (bottleneck, linear): 256 -> 256.
    // Layer 6 ([h5 | x] -> 256) runs before 7, the density head before 10.
    // The trunk stops after layer 8 (i = 5) and stores it.
    constexpr int NI = TRUNK ? 6 : 7;
#pragma nounroll
    for (int i = 0; i < NI; ++i) {
      if (i == 4) {
        take_input(true, p.Kx);
        bias_init(E8{}, BF_L6);
        run_layer(C11{}, C10{}, [&] { advance(); });
        epi_hidden(E8{}, true);
        // every wave has read this tile's x (barriers have passed since):
        // the next tile's x goes into the buffer now
        copy_input(k + 1, true);
      }
      if (i == 6) {
        run_layer(C21{}, C2{}, [&] { advance(); });
        epi_head(BH_L9 - BF_END, p.out_r, p.Na, ACT_NONE);
      }
      bias_init(E8{}, i < 4 ? BF_L2 + 512 * i : i < 6 ? BF_L7 + 512 * (i - 4) : BF_L10);
      // what follows is another 256 -> 256 layer, layer 6 or the density
      // head; layer 11 is acquired after the input waves' wait below (the
      // trunk's next tile after its own)
      run_layer(C3{}, C8{}, [&] {
        if (i != NI - 1) advance();
      });
      if (TRUNK && i == NI - 1) break;
      epi_hidden(E8{}, i != 6);
    }
    if constexpr (TRUNK) {
      epi_out();
      continue;
    }
    // Layer 11 ([bottleneck | d] -> 128, ReLU): the input waves wait for this
    // tile's d copies (the next tile's x copies may still be in flight).
    if (!ring_wave) wait_vmcnt<XCPW>();
    advance();
    take_input(false, p.Kd);
    bias_init(E4{}, BF_L11);
    run_layer(C23{}, C5{}, [&] { advance(); });
    epi_hidden(E4{}, true);
    copy_input(k + 1, false);
    // Layer 12: 128 -> Nrgb.
    run_layer(C28{}, C1{}, nothing);
    epi_head(BH_L12 - BF_END, p.out_rgb, p.Nrgb, p.rgb_act);
  }
  // The ring and input copies issued past the last tile (empty ranges that
  // still write zeros into dead LDS slots) land before the waves exit.
  wait_vmcnt<0>();
}

// ------------------------------------------------------------------ packing
struct PackLayer {
  const half_t* w;  // [krows][n] (nn.Linear.weight.t())
  const half_t* b;  // [n] or null
  int slot0, fb, kb, next, ext_w, ext_koff, n, boff, head;
};
struct PackArgs {
  PackLayer L[12];
  char* stream;
  half_t* bias;
};

// One thread per 16-byte lane chunk of a fragment, then one per bias entry.
__global__ __launch_bounds__(256) void nerf_pack_kernel(PackArgs a) {
  const int gid = blockIdx.x * blockDim.x + threadIdx.x;
  constexpr int NFRAG_T = S_TOTAL * FPS * kWave;
  if (gid < NFRAG_T) {
    const int s = gid / (FPS * kWave), pos = (gid / kWave) % FPS, lane = gid % kWave;
#pragma unroll
    for (int li = 0; li < 12; ++li) {
      const PackLayer& L = a.L[li];
      const int nslot = (L.kb * L.fb + FPS - 1) / FPS;
      if (s < L.slot0 || s >= L.slot0 + nslot) continue;
      const int fi = (s - L.slot0) * FPS + pos, kb = fi / L.fb, fb = fi % L.fb;
      const int out = 32 * fb + (lane & 31), h = lane >> 5;
      h8 v = {};
      if (kb < L.kb && out < L.n) {
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          const int pp = 8 * h + q;
          int kin;
          if (kb < L.next) {
            const int c = 16 * kb + pp;
            kin = c < L.ext_w ? L.ext_koff + c : -1;
          } else {
            kin = 16 * (kb - L.next) + sigma(pp);
          }
          v[q] = kin >= 0 ? L.w[(int64_t)kin * L.n + out] : (half_t)0.f;
        }
      }
      *(h8*)(a.stream + (int64_t)s * SLOT + pos * FRAG + lane * 16) = v;
    }
    return;
  }
  const int t = gid - NFRAG_T;
  if (t >= B_TOTAL) return;
#pragma unroll
  for (int li = 0; li < 12; ++li) {
    const PackLayer& L = a.L[li];
    if (L.head) {
      if (t >= L.boff && t < L.boff + 64) {
        const int f = t - L.boff;
        a.bias[t] = (L.b && f < L.n) ? L.b[f] : (half_t)0.f;
      }
    } else if (t >= L.boff && t < L.boff + 64 * L.fb) {
      const int fb = (t - L.boff) / 64, ln = (t - L.boff) % 64, f = 32 * fb + ln;
      a.bias[t] = (L.b && ln < 32 && f < L.n) ? L.b[f] : (half_t)0.f;
    }
  }
}

}  // namespace nerf

size_t nerf_fused_workspace() { return (size_t)nerf::S_TOTAL * nerf::SLOT + (size_t)nerf::B_TOTAL * 2; }

// Scratch of the allocation-free entry point (gp_nerf_full_out_noalloc): the
// packed weight stream and bias tables, in a file-scope device array instead
// of the per-stream workspace.  Every GPU the library runs on holds its own
// copy until the process ends.  The packing kernel rewrites every byte the
// fused kernel reads on each call, so nothing has to start at zero.  All
// calls on one GPU share the array: eager calls are chained through one event
// per device, so that calls on different streams run one after the other
// (calls captured into a graph are not chained: replays that overlap race).
constexpr size_t kNerfScratchBytes =
    ((size_t)nerf::S_TOTAL * nerf::SLOT + (size_t)nerf::B_TOTAL * 2 + 255) & ~size_t(255);
static __device__ __align__(256) char scratch[kNerfScratchBytes];

int nerf_static_scratch(int dev, NerfScratch* out) {
  // In host code `scratch` names a host-side stand-in, never the device
  // memory: its device address is looked up once per device (with that device
  // current) and only that address is handed to kernels.  The device's event
  // is created at the same set-up step, so later calls create nothing.
  static std::mutex mu;
  static void* dev_ptr[64];
  static hipEvent_t dev_ev[64];
  static std::mutex dev_lock[64];
  if (dev < 0 || dev >= 64) return fail(GP_ERR_NO_DEVICE, "device index %d out of range", dev);
  std::lock_guard<std::mutex> lk(mu);
  if (dev_ptr[dev] == nullptr) {
    void* p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return fail_hip(e, "hipGetSymbolAddress (NeRF static scratch)");
    hipEvent_t ev = nullptr;
    e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
    if (e != hipSuccess) return fail_hip(e, "hipEventCreateWithFlags (NeRF static scratch)");
    dev_ev[dev] = ev;
    dev_ptr[dev] = p;
  }
  *out = NerfScratch{dev_ptr[dev], kNerfScratchBytes, dev_ev[dev], &dev_lock[dev]};
  return GP_OK;
}

bool nerf_fused_supported(int64_t Kx, int64_t Kd, int64_t Na, int64_t Nrgb) {
  return Kx >= 1 && Kx <= 64 && Kd >= 1 && Kd <= 32 && Na >= 1 && Na <= 64 && Nrgb >= 1 && Nrgb <= 64;
}

// Packs the weight stream and bias tables (all twelve layers, or the trunk's
// first eight), then launches the fused kernel.
static hipError_t fused_launch(bool trunk, int64_t M, int Kx, int Kd, int Na, int Nrgb, const void* x, const void* d,
                               const void* const* w, const void* const* b, int rgb_act, void* out_r, void* out_rgb,
                               void* ws, int num_cus, hipStream_t s, int dtype) {
  using namespace nerf;
  if (dtype != GP_DTYPE_F16 && dtype != GP_DTYPE_BF16) return hipErrorInvalidValue;
  if (M <= 0) return hipSuccess;
  if (M > (int64_t(1) << 31) - 1) return hipErrorInvalidValue;
  if (((uintptr_t)x & 15) || ((uintptr_t)d & 15) || ((uintptr_t)ws & 15)) return hipErrorInvalidValue;
  PackArgs pa{};
  // slot0, fb, kb, next, ext_w, ext_koff, n, boff, head
  const int H = 256;
  const int shape[12][9] = {
      {S_L1, 8, 4, 4, Kx, 0, H, BF_L1, 0},             {S_L2, 8, 16, 0, 0, 0, H, BF_L2, 0},
      {S_L2 + 8, 8, 16, 0, 0, 0, H, BF_L2 + 512, 0},   {S_L2 + 16, 8, 16, 0, 0, 0, H, BF_L2 + 1024, 0},
      {S_L2 + 24, 8, 16, 0, 0, 0, H, BF_L2 + 1536, 0}, {S_L6, 8, 20, 4, Kx, H, H, BF_L6, 0},
      {S_L7, 8, 16, 0, 0, 0, H, BF_L7, 0},             {S_L7 + 8, 8, 16, 0, 0, 0, H, BF_L7 + 512, 0},
      {S_L9, 2, 16, 0, 0, 0, Na, BH_L9, 1},            {S_L10, 8, 16, 0, 0, 0, H, BF_L10, 0},
      {S_L11, 4, 20, 4, Kd, H, 128, BF_L11, 0},        {S_L12, 2, 8, 0, 0, 0, Nrgb, BH_L12, 1},
  };
  const int nl = trunk ? 8 : 12;
  for (int i = 0; i < nl; ++i) {
    const int* sh = shape[i];
    pa.L[i] = {(const half_t*)w[i], (const half_t*)b[i], sh[0], sh[1], sh[2], sh[3], sh[4], sh[5], sh[6], sh[7],
               sh[8]};
  }
  // (The trunk's layers 9-12 stay zero: no slots, no bias entries.)
  pa.stream = (char*)ws;
  pa.bias = (half_t*)((char*)ws + (size_t)S_TOTAL * SLOT);
  const int nthreads = S_TOTAL * FPS * kWave + B_TOTAL;
  hipLaunchKernelGGL(nerf_pack_kernel, dim3((nthreads + 255) / 256), dim3(256), 0, s, pa);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const Args a{(const half_t*)x, (const half_t*)d, (const char*)ws, pa.bias, (half_t*)out_r, (half_t*)out_rgb,
               M, Kx, Kd, Na, Nrgb, rgb_act};
  const int64_t tiles = (M + ROWS - 1) / ROWS;
  const dim3 grid((unsigned)(tiles < num_cus ? tiles : num_cus));
  if (trunk) {
    if (dtype == GP_DTYPE_BF16)
      hipLaunchKernelGGL((nerf_fused_kernel<BF16, true>), grid, dim3(NT), 0, s, a);
    else
      hipLaunchKernelGGL((nerf_fused_kernel<F16, true>), grid, dim3(NT), 0, s, a);
  } else {
    if (dtype == GP_DTYPE_BF16)
      hipLaunchKernelGGL((nerf_fused_kernel<BF16, false>), grid, dim3(NT), 0, s, a);
    else
      hipLaunchKernelGGL((nerf_fused_kernel<F16, false>), grid, dim3(NT), 0, s, a);
  }
  return hipGetLastError();
}

hipError_t nerf_fused_launch(int64_t M, int Kx, int Kd, int Na, int Nrgb, const void* x, const void* d,
                             const void* const* w, const void* const* b, int rgb_act, void* out_r, void* out_rgb,
                             void* ws, int num_cus, hipStream_t s, int dtype) {
  return fused_launch(false, M, Kx, Kd, Na, Nrgb, x, d, w, b, rgb_act, out_r, out_rgb, ws, num_cus, s, dtype);
}

hipError_t nerf_trunk_launch(int64_t M, int Kx, const void* x, const void* const* w, const void* const* b, void* out,
                             void* ws, int num_cus, hipStream_t s, int dtype) {
  return fused_launch(true, M, Kx, 0, 0, 0, x, nullptr, w, b, GP_ACT_NONE, out, nullptr, ws, num_cus, s, dtype);
}

}  // namespace gp
