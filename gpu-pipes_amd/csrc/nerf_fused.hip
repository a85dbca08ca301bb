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
//  * A workgroup of four waves (one per SIMD) owns a tile of 256 rows; wave w
//    owns rows 64w .. 64w+63 as two 32-row blocks and computes every output
//    feature of every layer for them, as C^T = W^T X^T with
//    v_mfma_f32_32x32x16_f16: the MFMA A operand is a 32-feature x 16-k block
//    of the weights (a "fragment"), the B operand a 16-k x 32-row block of the
//    layer input.
//  * Activations stay in registers.  A 256-feature layer's accumulators fill
//    the 256 AGPRs; converted to fp16 they fill 128 VGPRs, and in exactly the
//    register layout of the next layer's B operands, because the accumulator
//    lane layout (4 features x 4 groups of one row) is a permutation of the B
//    operand layout (8 consecutive k of one row).  The permutation is folded
//    into the weight packing: B position p = 8h + q of k-block kb holds input
//    feature 16 kb + sigma(p), sigma swapping the middle two groups of four.
//  * Weights (1.2 MB) do not fit on chip, so every tile streams them from L2:
//    the host packs all layers once per call into the exact order the kernel
//    consumes them, as 1 KiB fragments (64 lanes x 16 bytes), 16 to a 16 KiB
//    slot.  Slots are copied L2 -> LDS with buffer_load ... lds into a ring of
//    nine (144 KiB); up to eight are in flight while one is read.  The
//    remaining 16 KiB of LDS hold every layer's bias.
//  * The network inputs travel through the same ring: a tile's x rows (twice:
//    for layer 1 and for the skip input of layer 6) and its d rows occupy
//    "pseudo-slots" of the stream whose copies read x or d instead of
//    weights, 128 rows per slot, zero-filled past the last valid row.
//  * Slot bookkeeping is per wave and wave-uniform: before a slot is read,
//    each wave waits until its own copies of that slot have landed (vmcnt
//    counts only the copies issued after it) and the workgroup passes one
//    barrier; the barrier also certifies that every wave has finished reading
//    the slots released at that point, which the copies then refill.
//  * Epilogues: bias (from LDS, added in fp32), ReLU in packed fp16 after RNE
//    rounding (max commutes with rounding), straight into the B-operand
//    registers; the density and colour heads are stored through buffer
//    descriptors bounded to the tile's valid rows.
#include <hip/hip_runtime.h>

#include <type_traits>
#include <utility>

#include "../../include/gpipes.h"
#include "gp_device.hpp"
#include "gp_kernels.hpp"
#include "stages.hpp"

namespace gp {
namespace nerf {

constexpr int NW = 4;
constexpr int NT = NW * kWave;
constexpr int ROWS = 64 * NW;      // rows per tile
constexpr int FRAG = 1024;         // one A operand: 64 lanes x 16 bytes
constexpr int FPS = 16;            // fragments per slot
constexpr int SLOT = FPS * FRAG;   // bytes per ring slot
constexpr int NS = 9;              // ring slots
constexpr int PART = 128;          // rows of x or d per pseudo-slot

// Local slot map of one tile's stream (82 slots, 1.31 MB).
constexpr int S_X1 = 0, S_L1 = 2, S_L2 = 4, S_X2 = 36, S_L6 = 38, S_L7 = 48, S_L9 = 64, S_L10 = 66, S_D = 74,
              S_L11 = 76, S_L12 = 81, S_TOTAL = 82;
// Bias table (2560 values): layers 1-8 at 256 i, then 9, 10, 11, 12.
constexpr int B_L9 = 2048, B_L10 = 2112, B_L11 = 2368, B_L12 = 2496, B_TOTAL = 2560;
constexpr int BIAS_BYTES = B_TOTAL * 4;  // held as fp32 in LDS
static_assert(NS * SLOT + BIAS_BYTES <= 160 * 1024, "LDS");

struct Args {
  const half_t* x;       // [M][Kx]
  const half_t* d;       // [M][Kd]
  const char* stream;    // S_TOTAL slots (pseudo-slot positions unused)
  const half_t* bias;    // B_TOTAL
  half_t* out_r;         // [M][Na]
  half_t* out_rgb;       // [M][Nrgb]
  int64_t M;
  int Kx, Kd, Na, Nrgb, rgb_act;
};

// B-operand k-order of a k-block fed from registers: position p holds input
// feature 16 kb + sigma(p) (the accumulator layout of the layer before).
__host__ __device__ constexpr int sigma(int p) { return p < 4 ? p : p < 8 ? p + 4 : p < 12 ? p - 4 : p; }

// Slot kinds.  A compute slot holds 16 fragments of one layer: FB feature
// blocks per input k-block, starting at k-block KB0; the layer's first NEXT
// k-blocks take their B operand from pseudo-slots (EXT 1: x for layer 1,
// 2: x for layer 6, 3: d for layer 11), the rest from registers.
//   1-2 layer 1, 3-10 a 256 -> 256 layer, 11-20 layer 6, 21-22 layer 9,
//   23-27 layer 11, 28 layer 12; 0 a pseudo-slot (nothing to compute).
struct Kind {
  int fb, kb0, next, ext;
};
__host__ __device__ constexpr Kind kind_info(int k) {
  return k <= 2    ? Kind{8, 2 * (k - 1), 4, 1}
         : k <= 10 ? Kind{8, 2 * (k - 3), 0, 0}
         : k <= 20 ? Kind{8, 2 * (k - 11), 4, 2}
         : k <= 22 ? Kind{2, 8 * (k - 21), 0, 0}
         : k <= 27 ? Kind{4, 4 * (k - 23), 4, 3}
                   : Kind{2, 0, 0, 0};
}
// Returns v unchanged in a scalar register, hiding its value from the
// optimiser so that values derived from it are not hoisted and kept live.
__device__ __forceinline__ int opaque_s(int v) {
  asm volatile("" : "+s"(v));
  return v;
}

template <int... I, class F>
__device__ __forceinline__ void static_for(std::integer_sequence<int, I...>, F&& f) {
  (f(std::integral_constant<int, I>{}), ...);
}

__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(1, 1))) void nerf_fused_kernel(Args p) {
  __shared__ __attribute__((aligned(1024))) char smem[NS * SLOT + BIAS_BYTES];
  GP_LDS char* const ring = (GP_LDS char*)smem;
  GP_LDS float* const btab = (GP_LDS float*)(smem + NS * SLOT);

  const int tid = threadIdx.x;
  const int lane = tid & 63, lr = lane & 31, lh = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int G = gridDim.x;
  const int64_t ntiles = (p.M + ROWS - 1) / ROWS;
  const int my = (int)((ntiles - blockIdx.x + G - 1) / G);  // tiles blockIdx.x + k G, k < my
  const int total = my * S_TOTAL;                            // slots this workgroup consumes

  for (int i = tid; i < B_TOTAL; i += NT) btab[i] = (float)p.bias[i];
  __syncthreads();

  // ---------------------------------------------------------------- copies
  // Global slot q (tile q / S_TOTAL, local slot q % S_TOTAL) goes to ring
  // slot q % NS; 16-byte chunk c = 4 i + wave of the slot is this wave's copy i.
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(p.stream, S_TOTAL * SLOT);
  auto tile_r0 = [&](int k) { return ((int64_t)blockIdx.x + (int64_t)k * G) * ROWS; };
  auto issue = [&](int q) {
    const int k = q / S_TOTAL, l = q - k * S_TOTAL;
    GP_LDS char* const dst = ring + (q % NS) * SLOT;
    __amdgpu_buffer_rsrc_t r = rw;
    int base = l * SLOT;
    const bool px = l == S_X1 || l == S_X1 + 1 || l == S_X2 || l == S_X2 + 1;
    if (px || l == S_D || l == S_D + 1) {
      const int part = l & 1;  // every pseudo-slot pair starts at an even slot
      const int K = px ? p.Kx : p.Kd;
      const int64_t row0 = tile_r0(k) + part * PART;
      const int64_t left = p.M - row0;
      const int rows = left <= 0 ? 0 : left < PART ? (int)left : PART;
      // The range is rounded up to whole 16-byte copies; the bytes past the
      // last valid row lie in the same 16-byte block (so the same page) and
      // land only in rows that are never stored.
      r = make_rsrc((px ? p.x : p.d) + row0 * K, (rows * K * 2 + 15) & ~15);
      base = 0;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = 4 * i + wave;
      dma16_buf_so(r, 16 * lane, base + c * FRAG, dst + c * FRAG);
    }
  };
  // Slots 0 .. NS-2 are copied ahead; acquiring slot q copies slot q + NS - 1
  // into the ring slot of q - 1, which every wave has finished reading when
  // it passes the barrier.  Until then the NS - 2 slots after q are in flight.
  for (int q = 0; q < total && q < NS - 1; ++q) issue(q);
  auto acquire = [&](int q) {
    if (q + NS - 2 < total) wait_vmcnt<4 * (NS - 2)>();
    else wait_vmcnt<0>();
    lds_barrier();
    if (q + NS - 1 < total) issue(q + NS - 1);
  };

  f16x acc[8][2];  // [feature block][row block]
  h8 act[16][2];   // B operands of register-fed k-blocks: [k-block][row block]
  h8 xin[4][2];    // B operands of the x / d k-blocks: [k-block][row block]
  h8 fa[2][4];     // A fragments of two groups in flight

  for (int k = 0; k < my; ++k) {
    const int qb = k * S_TOTAL;
    const int64_t r0 = tile_r0(k);
    const int vrows = p.M - r0 < ROWS ? (int)(p.M - r0) : ROWS;
    // LDS address of local slot l, recomputed at every use (opaque) rather
    // than hoisted: 82 live slot addresses would spill scalar registers.
    auto slot = [&](int l) { return (GP_LDS const char*)(ring + ((opaque_s(qb) + l) % NS) * SLOT); };

    // Acquire the pseudo-slot pair at local slots l0, l0+1 and read this
    // wave's rows of it (slot l0 + wave / 2 holds them, K columns per row)
    // into xin, zero for columns >= K.  Each half of the pair is read right
    // after it is acquired, so both are dead when the next slot is acquired.
    auto take_input = [&](int l0, int K) {
#pragma unroll
      for (int part = 0; part < 2; ++part) {
        if (qb + l0 + part < total) acquire(qb + l0 + part);
        if ((wave >> 1) == part) {
          GP_LDS const char* const b = slot(l0 + part);
#pragma unroll
          for (int rb = 0; rb < 2; ++rb) {
            const int e0 = ((64 * wave + 32 * rb + lr) & (PART - 1)) * K + 8 * lh;
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) {
              const int c0 = 16 * kb + 8 * lh;
              h8 v;
              if ((K & 7) == 0) {
                v = *(GP_LDS const h8*)(b + (e0 + 16 * kb) * 2);
              } else {
#pragma unroll
                for (int e = 0; e < 8; ++e) v[e] = *(GP_LDS const half_t*)(b + (e0 + 16 * kb + e) * 2);
#pragma unroll
                for (int e = 0; e < 8; ++e) v[e] = c0 + e < K ? v[e] : (half_t)0.f;
              }
              xin[kb][rb] = c0 < K ? v : h8{};
            }
          }
        }
      }
    };

    // Read group g (fragments 4g .. 4g+3) of local slot l into fa[BUF].
    auto fetch = [&](int l, auto gc, auto bufc) {
      constexpr int g = decltype(gc)::value, buf = decltype(bufc)::value;
      GP_LDS const char* const s = slot(l) + 4 * g * FRAG + 16 * lane;
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
        for (int rb = 0; rb < 2; ++rb) {
          h8 b;
          if constexpr (kb < K.next) b = xin[kb][rb];
          else b = act[kb - K.next][rb];
          acc[fb][rb] = mfma32(fa[buf][i], b, kb == 0 ? f16x{} : acc[fb][rb]);
        }
      });
    };
    using G0 = std::integral_constant<int, 0>;
    using G1 = std::integral_constant<int, 1>;
    using G2 = std::integral_constant<int, 2>;
    using G3 = std::integral_constant<int, 3>;

    // Hidden-layer epilogue: act[2 fb + s][rb] = relu?(acc + bias) in fp16.
    // Lane (row lr, half lh) holds, in element 4 g + e of block fb, feature
    // 32 fb + 8 g + 4 lh + e.
    auto epi_hidden = [&](auto FBc, int boff, bool relu) {
      constexpr int FB = decltype(FBc)::value;
#pragma unroll
      for (int fb = 0; fb < FB; ++fb) {
        f4 bb[4];
#pragma unroll
        for (int g = 0; g < 4; ++g) bb[g] = *(GP_LDS const f4*)(btab + boff + 32 * fb + 8 * g + 4 * lh);
#pragma unroll
        for (int rb = 0; rb < 2; ++rb) {
          h8 lo, hi;
#pragma unroll
          for (int r = 0; r < 8; ++r) {
            lo[r] = (half_t)(acc[fb][rb][r] + bb[r / 4][r % 4]);
            hi[r] = (half_t)(acc[fb][rb][8 + r] + bb[2 + r / 4][r % 4]);
          }
          if (relu) {
            lo = __builtin_elementwise_max(lo, h8{});
            hi = __builtin_elementwise_max(hi, h8{});
          }
          act[2 * fb][rb] = lo;
          act[2 * fb + 1][rb] = hi;
        }
      }
    };

    // Head epilogue: out[row][c] = fn(acc + bias) for c < N, rows < vrows.
    auto epi_head = [&](int boff, half_t* out, int N, int fn) {
      const __amdgpu_buffer_rsrc_t ro = make_rsrc(out + r0 * N, vrows * N * 2);
      const bool vec = (N & 3) == 0 && ((uintptr_t)out & 7) == 0;
#pragma unroll
      for (int fb = 0; fb < 2; ++fb)
#pragma unroll
        for (int rb = 0; rb < 2; ++rb) {
          const int row = 64 * wave + 32 * rb + lr;
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const int c = 32 * fb + 8 * g + 4 * lh;
            const f4 bb = *(GP_LDS const f4*)(btab + boff + c);
            f4 v;
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = apply_act(acc[fb][rb][4 * g + e] + bb[e], fn);
            const h4 h = __builtin_convertvector(v, h4);
            const int off = (row * N + c) * 2;
            if (vec) {
              if (c < N) buf_store_h4(ro, off, h);
            } else {
              // 16-bit words taken out with integer shifts: the b16 store of a
              // bit-cast vector element was compiled to store element 0 each time.
              const u32x2 w2 = __builtin_bit_cast(u32x2, h);
#pragma unroll
              for (int e = 0; e < 4; ++e)
                if (c + e < N)
                  __builtin_amdgcn_raw_buffer_store_b16((unsigned short)(w2[e >> 1] >> (16 * (e & 1))), ro, off + 2 * e,
                                                        0, 0);
            }
          }
        }
    };

    // Slot program.  A slot is 4 groups of 4 fragments; group g+1 is read
    // while group g is multiplied, and before the last group the next slot is
    // acquired and its first group read, so the barrier and the read latency
    // hide behind running MFMAs -- across layer boundaries too, where the
    // epilogue runs after the next layer's first fragments were requested.
    // Acquire local slot l (global qb + l; l may run into the next tile) and
    // read its first group.
    auto advance = [&](int l) {
      if (qb + l >= total) return;
      acquire(qb + l);
      fetch(l, G0{}, G0{});
    };
    // The slots of one layer: kinds KD0 .. KD0+N-1 at local slots l0 ...;
    // `after` acquires what follows the layer, between the last slot's parts.
    auto run_layer = [&](auto kd0c, auto nc, int l0, auto&& after) {
      constexpr int KD0 = decltype(kd0c)::value, N = decltype(nc)::value;
      static_for(std::make_integer_sequence<int, N>{}, [&](auto jc) {
        constexpr int j = decltype(jc)::value;
        using KD = std::integral_constant<int, KD0 + j>;
        const int l = l0 + j;
        fetch(l, G1{}, G1{});
        mma(KD{}, G0{}, G0{});
        fetch(l, G2{}, G0{});
        mma(KD{}, G1{}, G1{});
        fetch(l, G3{}, G1{});
        mma(KD{}, G2{}, G0{});
        if constexpr (j + 1 < N) advance(l + 1);
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

    // Layer 1: x -> 256, ReLU.
    take_input(S_X1, p.Kx);
    advance(S_L1);
    run_layer(C1{}, C2{}, S_L1, [&] { advance(S_L2); });
    epi_hidden(E8{}, 0, true);
    // Layers 2-5, 7, 8 (ReLU) and 10 (bottleneck, linear): 256 -> 256.
    // Layer 6 ([h5 | x] -> 256) runs before 7, the density head before 10.
#pragma nounroll
    for (int i = 0; i < 7; ++i) {
      if (i == 4) {
        take_input(S_X2, p.Kx);
        advance(S_L6);
        run_layer(C11{}, C10{}, S_L6, [&] { advance(S_L7); });
        epi_hidden(E8{}, 5 * 256, true);
      }
      if (i == 6) {
        run_layer(C21{}, C2{}, S_L9, [&] { advance(S_L10); });
        epi_head(B_L9, p.out_r, p.Na, ACT_NONE);
      }
      const int l0 = i < 4 ? S_L2 + 8 * i : i < 6 ? S_L7 + 8 * (i - 4) : S_L10;
      // what follows is another 256 -> 256 layer or the density head, or a
      // pseudo-slot pair (before layers 6 and 11), taken after the epilogue
      run_layer(C3{}, C8{}, l0, [&] {
        if (i != 3 && i != 6) advance(l0 + 8);
      });
      epi_hidden(E8{}, i < 4 ? 256 * (i + 1) : i < 6 ? 256 * (i + 2) : B_L10, i != 6);
    }
    // Layer 11 ([bottleneck | d] -> 128, ReLU) and layer 12 (128 -> Nrgb).
    take_input(S_D, p.Kd);
    advance(S_L11);
    run_layer(C23{}, C5{}, S_L11, [&] { advance(S_L12); });
    epi_hidden(E4{}, B_L11, true);
    run_layer(C28{}, C1{}, S_L12, nothing);
    epi_head(B_L12, p.out_rgb, p.Nrgb, p.rgb_act);
  }
}

// ------------------------------------------------------------------ packing
struct PackLayer {
  const half_t* w;  // [krows][n] (nn.Linear.weight.t())
  const half_t* b;  // [n] or null
  int slot0, fb, kb, next, ext_w, ext_koff, n, f, boff;
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
    if (t >= L.boff && t < L.boff + L.f) {
      const int f = t - L.boff;
      a.bias[t] = (L.b && f < L.n) ? L.b[f] : (half_t)0.f;
    }
  }
}

}  // namespace nerf

size_t nerf_fused_workspace() { return (size_t)nerf::S_TOTAL * nerf::SLOT + nerf::BIAS_BYTES; }

bool nerf_fused_supported(int64_t Kx, int64_t Kd, int64_t Na, int64_t Nrgb) {
  return Kx >= 1 && Kx <= 64 && Kd >= 1 && Kd <= 64 && Na >= 1 && Na <= 64 && Nrgb >= 1 && Nrgb <= 64;
}

hipError_t nerf_fused_launch(int64_t M, int Kx, int Kd, int Na, int Nrgb, const void* x, const void* d,
                             const void* const* w, const void* const* b, int rgb_act, void* out_r, void* out_rgb,
                             void* ws, int num_cus, hipStream_t s) {
  using namespace nerf;
  if (M <= 0) return hipSuccess;
  if (((uintptr_t)x & 15) || ((uintptr_t)d & 15) || ((uintptr_t)ws & 15)) return hipErrorInvalidValue;
  PackArgs pa{};
  // slot0, fb, kb, next, ext_w, ext_koff, n, f, boff
  const int H = 256;
  const int shape[12][9] = {
      {S_L1, 8, 4, 4, Kx, 0, H, H, 0},           {S_L2, 8, 16, 0, 0, 0, H, H, 256},
      {S_L2 + 8, 8, 16, 0, 0, 0, H, H, 512},     {S_L2 + 16, 8, 16, 0, 0, 0, H, H, 768},
      {S_L2 + 24, 8, 16, 0, 0, 0, H, H, 1024},   {S_L6, 8, 20, 4, Kx, H, H, H, 1280},
      {S_L7, 8, 16, 0, 0, 0, H, H, 1536},        {S_L7 + 8, 8, 16, 0, 0, 0, H, H, 1792},
      {S_L9, 2, 16, 0, 0, 0, Na, 64, B_L9},      {S_L10, 8, 16, 0, 0, 0, H, H, B_L10},
      {S_L11, 4, 20, 4, Kd, H, 128, 128, B_L11}, {S_L12, 2, 8, 0, 0, 0, Nrgb, 64, B_L12},
  };
  for (int i = 0; i < 12; ++i) {
    const int* sh = shape[i];
    pa.L[i] = {(const half_t*)w[i], (const half_t*)b[i], sh[0], sh[1], sh[2], sh[3], sh[4], sh[5], sh[6], sh[7],
               sh[8]};
  }
  pa.stream = (char*)ws;
  pa.bias = (half_t*)((char*)ws + (size_t)S_TOTAL * SLOT);
  const int nthreads = S_TOTAL * FPS * kWave + B_TOTAL;
  hipLaunchKernelGGL(nerf_pack_kernel, dim3((nthreads + 255) / 256), dim3(256), 0, s, pa);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const Args a{(const half_t*)x, (const half_t*)d, (const char*)ws, pa.bias, (half_t*)out_r, (half_t*)out_rgb,
               M, Kx, Kd, Na, Nrgb, rgb_act};
  const int64_t tiles = (M + ROWS - 1) / ROWS;
  const int64_t grid = tiles < num_cus ? tiles : num_cus;
  hipLaunchKernelGGL(nerf_fused_kernel, dim3((unsigned)grid), dim3(NT), 0, s, a);
  return hipGetLastError();
}

}  // namespace gp
