// Fused MeshGraphNet MLP for gfx950: Linear(K->128)+ReLU, Linear(128->128)+ReLU,
// Linear(128->128) [, LayerNorm(128)] in one persistent kernel.
//
// Reference behaviour: apps/mgn_fullmlp/pipelined/mgn_fullmlp_pl.cuh:83-252
// (three GEMM stage blocks + five LayerNorm blocks per pipeline row, chained by
// global-memory queues) and apps/mgn_linears/pipelined/mgn_linears_pl.cuh:176-212
// (the same chain without LayerNorm).  The oracle semantics are those of
// common/mlps.py:3-20 (MgnMlp), computed here with fp32 accumulation.
//
// MI355X design: one persistent workgroup of 8 waves per CU walks 64-row tiles.
// The reference's stage blocks become wave-specialised stages inside the CU:
//  * Stage A (waves 0-3, one per SIMD): layer 1.  Wave n keeps the W1 slice
//    for output features [32n, 32n+32) resident in AGPRs (K/16 MFMA A
//    fragments), streams X tiles HBM->LDS with buffer_load ... lds (16 B per
//    lane, whole 1 KiB wave transactions, non-temporal so the stream does not
//    evict L2, double-buffered, XOR-swizzled so the MFMA B-operand reads are
//    bank-conflict free), and writes
//    relu(X W1 + b1) in fp16 to one of two LDS handoff tiles.
//  * Stage B (waves 4-7, one per SIMD): layers 2 and 3 plus LayerNorm.  Layer
//    2 is split by feature (wave r computes features [32r, 32r+32) of all 64
//    rows from the handoff tile, W2 slice resident), its output is exchanged
//    through LDS, and layer 3 is split by row: wave r computes all 128
//    features of rows [16r, 16r+16) with v_mfma_f32_16x16x32_f16 and the whole
//    W3 resident in AGPRs.  Every row's 128 outputs then sit in four lanes of
//    one wave, so the LayerNorm (two-pass mean / variance, as the reference's
//    common/layer_norm_v2.cuh:42-70) is computed in-wave with two lane
//    exchanges and no cross-wave synchronisation.
//  * The handoff replaces the reference's global-memory queue
//    (common/mpmcq.cuh): a two-slot LDS ring with monotonic "full"/"free"
//    counters, so activations never leave the CU and stages A and B of
//    different tiles run concurrently on every SIMD (one A and one B wave per
//    SIMD share the matrix core).  All in-loop synchronisation is LDS
//    counters (one A-wave barrier per tile, one-sided waits elsewhere);
//    s_barrier is used only in the prologue.
//  * All chains are computed transposed, Y^T = W^T X^T, with
//    v_mfma_f32_32x32x16_f16; the bias is the accumulator's initial value.
//  * Prologue: the weights are copied HBM->LDS in their own row-major shape
//    (whole 1 KiB copies into the X buffers and hand-off slots) and every
//    wave reads its MFMA A fragments -- columns of W -- with the transposing
//    LDS read ds_read_b64_tr_b16; W3 follows into the hand-off slots once W1
//    and W2 are read, while the first X tile is copied into the X buffers.
//    Two copy latencies and no transposing LDS writes.
#include "gp_device.hpp"
#include "gp_kernels.hpp"

namespace gp {
namespace fused {

constexpr int TM = 64;          // rows per tile (two 32-row MFMA blocks)
constexpr int D = 128;          // hidden width of every MGN layer
constexpr int NWAVES = 8;       // 4 layer-1 waves + 4 layer-2/3/LN waves
constexpr int NTHREADS = NWAVES * kWave;
constexpr int ACT_STRIDE = D * 2 + 16;   // padded LDS row (bytes) of a 128-wide fp16 tile
constexpr int PF_L1 = 4;                 // layer-1 B-fragment prefetch depth (k-steps)
constexpr int PF_L2 = 2;                 // layer-2 B-fragment prefetch depth (k-steps)

template <int K>
struct Cfg {
  static_assert(K % 128 == 0 && K >= 128 && K <= 384, "K must be 128, 256 or 384");
  static constexpr int KS1 = K / 16;                 // MFMA k-steps of layer 1
  static constexpr int CPR = K / 8;                  // 16-byte chunks per X row
  static constexpr int XTILE = TM * K * 2;           // bytes per X tile
  static constexpr int XBUF = XTILE;                  // also W1 / W3 staging in the prologue
  static constexpr int DMA_INSTR = XTILE / 1024;     // wave-wide 1 KiB copies per tile
  static constexpr int DMA_PER_WAVE = DMA_INSTR / 4; // issued by the four A waves
  static_assert(DMA_INSTR % 4 == 0, "tile must split evenly over the A waves");
};

struct Params {
  const half_t* x;
  const half_t* w1;
  const half_t* b1;
  const half_t* w2;
  const half_t* b2;
  const half_t* w3;
  const half_t* b3;
  const half_t* gamma;
  const half_t* beta;
  half_t* out;
  int64_t M;
  float eps;
  // Gather front end (GATHER kernels only): X row e is
  // [nf[src[e]] | x[e] | nf[dst[e]]], nf is [N][128], indices are int32 or int64.
  const half_t* nf;
  int64_t N;
  const void* src;
  const void* dst;
  // Launch status: a wait that runs out of its `spin_limit` polls aborts the
  // workgroup, which then skips its output stores and records the timeout in
  // *status for this launch's epoch (gp_pipeline_check reports it).
  unsigned long long* status;
  uint32_t epoch;
  int spin_limit;
};

// LDS synchronisation words (monotonic counters, one count per wave per tile).
struct Sync {
  int a_bar;    // barrier among the A waves
  int h_full;   // handoff tile written by the A waves
  int h_free;   // handoff tile read by the B waves
  int x2_full;  // layer-2 output tile written by the B waves
  int x2_free;  // layer-2 output tile read by the B waves
  int abort;    // set when a wait exceeds its spin bound
};

// Element types.  Tiles, fragments and LDS hold raw 16-bit values (typed h8 /
// h4 throughout); only the MFMAs, the fp32 -> 16-bit conversions and the
// parameter loads depend on the type.
struct ElemF16 {
  __device__ static f16x mma32(h8 a, h8 b, f16x c) { return mfma32(a, b, c); }
  __device__ static f4 mma16(h8 a, h8 b, f4 c) { return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0); }
  __device__ static h4 cvt4(f4 v) { return __builtin_convertvector(v, h4); }
  // relu(round(x)) == round(relu(x)): the ReLU runs on the packed fp16 values
  __device__ static h4 relu_cvt4(f4 v) { return __builtin_elementwise_max(cvt4(v), (h4){0, 0, 0, 0}); }
  __device__ static float load(const half_t* p, int i) { return (float)p[i]; }
};
typedef __bf16 bf8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf4 __attribute__((ext_vector_type(4)));
struct ElemBF16 {
  __device__ static f16x mma32(h8 a, h8 b, f16x c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf8, a), __builtin_bit_cast(bf8, b), c, 0, 0, 0);
  }
  __device__ static f4 mma16(h8 a, h8 b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf8, a), __builtin_bit_cast(bf8, b), c, 0, 0, 0);
  }
  // v_cvt_pk_bf16_f32: round to nearest even
  __device__ static h4 cvt4(f4 v) { return __builtin_bit_cast(h4, __builtin_convertvector(v, bf4)); }
  __device__ static h4 relu_cvt4(f4 v) { return cvt4(__builtin_elementwise_max(v, (f4){0.f, 0.f, 0.f, 0.f})); }
  __device__ static float load(const half_t* p, int i) {
    return __builtin_bit_cast(float, (unsigned)__builtin_bit_cast(unsigned short, p[i]) << 16);
  }
};

// Accumulator initialised with the bias: C element 4g+e of a lane holds the
// bias of feature fq + 8g + e (every row of the block shares it).
__device__ __forceinline__ f16x bias_frag(const float* bias, int fq) {
  f16x c;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const f4 v = *(const f4*)&bias[fq + 8 * g];
#pragma unroll
    for (int e = 0; e < 4; ++e) c[4 * g + e] = v[e];
  }
  return c;
}

// Two 32-row blocks sharing the A operand (weight fragments wf[0..KS)); B
// fragments come from LDS through ld(rb, s), fetched PF k-steps ahead.  The
// scheduling barriers fix the issue order (2*PF reads, then per k-step two
// MFMAs followed by the two reads of step s + PF), so 2*PF LDS reads stay in
// flight behind every MFMA instead of the one or two the default schedule
// leaves.  NPRE counts LDS reads the caller issues just before (the bias
// fragments), which the scheduler places in the first group.
template <typename E, int KS, int PF, int NPRE, int NHOOK, typename LD, typename HOOK>
__device__ __forceinline__ void gemm_2blk(const h8* wf, LD ld, f16x& acc0, f16x& acc1, HOOK hook) {
  static_assert(PF >= 1 && PF <= KS && NHOOK <= KS, "prefetch depth / hook steps");
  h8 q0[PF], q1[PF];
#pragma unroll
  for (int p = 0; p < PF; ++p) {
    q0[p] = ld(0, p);
    q1[p] = ld(1, p);
  }
  __builtin_amdgcn_sched_group_barrier(0x100, 2 * PF + NPRE, 0);
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    acc0 = E::mma32(wf[s], q0[s % PF], acc0);
    acc1 = E::mma32(wf[s], q1[s % PF], acc1);
    __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
    if (s + PF < KS) {
      q0[s % PF] = ld(0, s + PF);
      q1[s % PF] = ld(1, s + PF);
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
    }
    if (s < NHOOK) {
      hook(s);
      __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
    }
  }
}

template <typename E, int KS, int PF, int NPRE, typename LD>
__device__ __forceinline__ void gemm_2blk(const h8* wf, LD ld, f16x& acc0, f16x& acc1) {
  gemm_2blk<E, KS, PF, NPRE, 0>(wf, ld, acc0, acc1, [](int) {});
}

// ReLU + 16-bit rounding of an accumulator into this lane's row of an LDS
// activation tile.
template <typename E>
__device__ __forceinline__ void store_relu_row(GP_LDS char* act_row, int fq, const f16x& a) {
#pragma unroll
  for (int g = 0; g < 4; ++g)
    *(GP_LDS h4*)(act_row + (fq + 8 * g) * 2) = E::relu_cvt4((f4){a[4 * g], a[4 * g + 1], a[4 * g + 2], a[4 * g + 3]});
}

// Weight staging for the prologue: the weight matrices are copied HBM->LDS
// in their own shape (the staged-rows layout of gp_device.hpp), copy j
// holding rows 4j .. 4j+3; the eight waves take copies wave, wave + 8, ...
// The copies land in LDS buffers that are otherwise the X tiles and the
// hand-off slots: copy j goes to the first buffer while it lasts (n copies),
// then to the second.  (Separate buffers, not one array, so that the
// compiler keeps them apart in the main loop.)
struct WSpan {
  GP_LDS char* a;
  int n;
  GP_LDS char* b;
  __device__ GP_LDS char* block(int j) const { return j < n ? a + j * 1024 : b + (j - n) * 1024; }
};
template <int R>
__device__ __forceinline__ void weight_dma(const half_t* W, WSpan dst, int wave, int lane) {
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(W, R * D * 2);
  const int voff = wrow_voff(lane, D * 2);
  static_assert((R / 4) % NWAVES == 0, "every wave issues the same number of copies");
#pragma unroll
  for (int i = 0; i < R / 4 / NWAVES; ++i) {
    const int j = wave + NWAVES * i;
    dma16_buf_so(rs, voff, j * (4 * D * 2), dst.block(j));
  }
}
// Lane j of each 16-lane group receives W[kb + e][fb + j], e = 0..7 (kb a
// multiple of 8, fb of 16).
__device__ __forceinline__ h8 w_col8(const WSpan& w, int kb, int fb, int m) {
  return wrows_col8(w.block(kb >> 2), w.block((kb >> 2) + 1), fb, m);
}

// s_memrealtime at five points of the weight prologue, in the phase-timer
// build only (the product build's marks are empty).
#ifdef GP_PHASE_TIMERS
struct PrologueMarks {
  unsigned long long t[5] = {0, 0, 0, 0, 0};
  __device__ void mark(int i) { t[i] = __builtin_amdgcn_s_memrealtime(); }
};
#else
struct PrologueMarks {
  __device__ void mark(int) {}
};
#endif

// Prologue shared by both stages: W1 (into the X buffers) and W2 (into the
// hand-off slots) are copied at once; take12(w1, w2) then reads the caller's
// fragments.  W3 follows into the hand-off slots once every wave has its W1
// and W2 fragments, and early() -- the first X tile's copies, from the A waves
// -- goes into the X buffers at the same time; take3(w3) reads W3.  pre()
// runs while the first copies are in flight.  EARLY_OPS: the copies early()
// issues, which the W3 wait leaves in flight (the barriers after it wait for
// LDS traffic only).
template <int K, int EARLY_OPS, typename Pre, typename T12, typename Early, typename T3>
__device__ __forceinline__ void stage_weights_dma(const Params& p, WSpan xsp, WSpan hsp, PrologueMarks& pm, int wave,
                                                  int lane, Pre pre, T12 take12, Early early, T3 take3) {
  weight_dma<K>(p.w1, xsp, wave, lane);
  weight_dma<D>(p.w2, hsp, wave, lane);
  pre();
  wait_vmcnt<0>();
  pm.mark(0);
  __syncthreads();
  pm.mark(1);
  take12(xsp, hsp);
  __syncthreads();  // W1 and W2 read by every wave
  pm.mark(2);
  weight_dma<D>(p.w3, hsp, wave, lane);
  early();
  wait_vmcnt<EARLY_OPS>();
  pm.mark(3);
  lds_barrier();
  take3(hsp);
  lds_barrier();  // the hand-off slots return to their tiles
  pm.mark(4);
}

// Sum of a value over the four lanes l, l^16, l^32, l^48 (the lanes that
// share l % 16), returned in all of them: v_permlane16_swap / 32_swap exchange
// rows of 16 lanes without going through LDS.
__device__ __forceinline__ float sum_lanes_16_32(float x) {
  const unsigned u = __builtin_bit_cast(unsigned, x);
  const auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  const float y = __builtin_bit_cast(float, (unsigned)a[0]) + __builtin_bit_cast(float, (unsigned)a[1]);
  const unsigned w = __builtin_bit_cast(unsigned, y);
  const auto b = __builtin_amdgcn_permlane32_swap(w, w, false, false);
  return __builtin_bit_cast(float, (unsigned)b[0]) + __builtin_bit_cast(float, (unsigned)b[1]);
}

// Stores output features [32j, 32j+32) of row l16 from the fp16 groups of a
// 16x16 accumulator pair: hv[t] holds features 16(2j+t) + 4q4 + (0..3) in
// lane (l16, q4).  v_permlane16_swap trades one group between lanes q4 and
// q4^1, after which each lane holds eight consecutive features (q4 = 0: +0,
// 1: +16, 2: +8, 3: +24), so one 16-byte store per lane writes 64
// contiguous bytes of each of the 16 rows -- half the store instructions
// and twice the segment length of four-feature stores.
__device__ __forceinline__ void store_row_pair(half_t* row, const h4 (&hv)[2], int j, int q4, bool ok) {
  const u32x2 a = __builtin_bit_cast(u32x2, hv[0]);
  const u32x2 b = __builtin_bit_cast(u32x2, hv[1]);
  const auto lo = __builtin_amdgcn_permlane16_swap(a[0], b[0], false, false);
  const auto hi = __builtin_amdgcn_permlane16_swap(a[1], b[1], false, false);
  const u32x4 w = {(unsigned)lo[0], (unsigned)hi[0], (unsigned)lo[1], (unsigned)hi[1]};
  if (ok) *(u32x4*)((char*)row + 64 * j + (q4 & 1) * 32 + (q4 >> 1) * 16) = w;
}

// Phase timers, compiled in only with GP_PHASE_TIMERS (libgpipes_phase.so, a
// diagnostic build): every wave adds the s_memtime ticks (shader clock
// cycles) of each phase of its tile loop into acc[], and at exit lane 0 of
// wave w of workgroup b (b < kPhaseGroups) writes slot group (b * NWAVES + w):
// acc[0..7], then the loop's total ticks, its s_memrealtime ticks (100 MHz),
// the tiles it ran, the launch's grid size, the s_memrealtime values at
// kernel entry, at the loop's start and at its end, and the five prologue
// marks.  The product build's timer is empty and costs nothing.
constexpr int kPhaseGroups = 256;
constexpr int kPhaseSlots = 20;
#ifdef GP_PHASE_TIMERS
__device__ unsigned long long g_phase[kPhaseGroups * NWAVES * kPhaseSlots];
struct PhaseTimer {
  unsigned long long acc[8] = {0, 0, 0, 0, 0, 0, 0, 0}, last = 0, t0 = 0, r0 = 0;
  __device__ void start() {
    t0 = last = __builtin_amdgcn_s_memtime();
    r0 = __builtin_amdgcn_s_memrealtime();
  }
  __device__ void tile() { last = __builtin_amdgcn_s_memtime(); }
  __device__ void mark(int i) {
    const unsigned long long t = __builtin_amdgcn_s_memtime();
    acc[i] += t - last;
    last = t;
  }
  __device__ void finish(int wave, int lane, int nt, unsigned long long entry, const PrologueMarks& pm) {
    const unsigned long long t = __builtin_amdgcn_s_memtime(), r = __builtin_amdgcn_s_memrealtime();
    if (lane != 0 || blockIdx.x >= kPhaseGroups) return;
    unsigned long long* o = g_phase + ((int64_t)blockIdx.x * NWAVES + wave) * kPhaseSlots;
    for (int i = 0; i < 8; ++i) o[i] = acc[i];
    o[8] = t - t0;
    o[9] = r - r0;
    o[10] = (unsigned long long)nt;
    o[11] = gridDim.x;
    o[12] = entry;
    o[13] = r0;
    o[14] = r;
    for (int i = 0; i < 5; ++i) o[15 + i] = pm.t[i];
  }
};
__device__ __forceinline__ unsigned long long phase_entry() { return __builtin_amdgcn_s_memrealtime(); }
#else
struct PhaseTimer {
  __device__ void start() {}
  __device__ void tile() {}
  __device__ void mark(int) {}
  __device__ void finish(int, int, int, unsigned long long, const PrologueMarks&) {}
};
__device__ __forceinline__ unsigned long long phase_entry() { return 0; }
#endif

// GATHER_IDX: 0 = X given; 4 / 8 = gather, index bytes.  E: ElemF16 / ElemBF16.
template <int K, bool LN, int GATHER_IDX = 0, typename E = ElemF16>
__global__ __launch_bounds__(NTHREADS) __attribute__((amdgpu_waves_per_eu(2, 2)))
void mgn_fused_kernel(Params p) {
  const unsigned long long t_entry = phase_entry();  // phase-timer build only (0 otherwise)
  PrologueMarks pro_t;
  using C = Cfg<K>;
  constexpr bool GATHER = GATHER_IDX != 0;
  static_assert(!GATHER || K == 3 * D, "the gather front end builds 384-wide rows");
  // LDS layout of an X tile: row r, 16-byte logical chunk c (of K/8) lives at
  // (c / 16) * XSEG + r * XROW + ((c ^ r) & 15) * 16 -- XOR-swizzled within
  // groups of 16 chunks.  A plain tile is row-major (XROW = 2K, XSEG = 256);
  // a gathered tile is segment-major (XROW = 256, XSEG = 64 * 256), so every
  // 1 KiB copy comes from one source array.
  constexpr int XROW = GATHER ? 256 : K * 2;
  constexpr int XSEG = GATHER ? TM * 256 : 256;
  __shared__ __attribute__((aligned(1024))) char xs0[C::XBUF];
  __shared__ __attribute__((aligned(1024))) char xs1[C::XBUF];
  __shared__ __attribute__((aligned(16))) char hand0[TM * ACT_STRIDE];  // layer-1 output, slot 0
  __shared__ __attribute__((aligned(16))) char hand1[TM * ACT_STRIDE];  // layer-1 output, slot 1
  __shared__ __attribute__((aligned(16))) char act2[TM * ACT_STRIDE];   // layer-2 output
  __shared__ __attribute__((aligned(16))) float prm[5][D];  // b1, b2, b3, gamma, beta
  __shared__ Sync sy;
  __shared__ __attribute__((aligned(16))) char idxs[GATHER ? 2 : 1][GATHER ? 2048 : 16];  // gather indices: [tile & 1][src | dst]

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int lr = lane & 31;   // row within a 32-row block (32x32 B / C column)
  const int lh = lane >> 5;   // half of the k-chunk / feature quad (32x32 layout)
  const int n = wave & 3;     // feature slice (A, B layer 2) / row block (B layer 3)
  const bool stage_a = wave < 4;

  const int64_t M = p.M;
  const int64_t ntiles = (M + TM - 1) / TM;
  const int64_t G = gridDim.x;
  const int64_t t0 = blockIdx.x;
  if (t0 >= ntiles) return;
  const int nt = (int)((ntiles - 1 - t0) / G + 1);  // tiles of this workgroup

  // bias / LayerNorm parameters, loaded while the first weight slab is in flight
  auto load_prm = [&]() {
    if (tid < D) {
      prm[0][tid] = E::load(p.b1, tid);
      prm[1][tid] = E::load(p.b2, tid);
      prm[2][tid] = E::load(p.b3, tid);
      if (LN) {
        prm[3][tid] = E::load(p.gamma, tid);
        prm[4][tid] = E::load(p.beta, tid);
      }
    }
  };
  if (tid == 0) sy = Sync{0, 0, 0, 0, 0, 0};

  const int fq = 32 * n + 4 * lh;  // 32x32 accumulator group g covers features fq + 8g + (0..3)
  const int arow0 = lr * ACT_STRIDE, arow1 = (32 + lr) * ACT_STRIDE;
  GP_LDS int* const ab = (GP_LDS int*)&sy.abort;
  const int lim = p.spin_limit;
  // prologue weight staging: W1 in the X buffers, W2 then W3 in the hand-off slots
  static_assert(2 * C::XBUF >= K * D * 2 && 2 * TM * ACT_STRIDE >= D * D * 2, "staged weights must fit");
  const WSpan xspan{(GP_LDS char*)xs0, C::XBUF / 1024, (GP_LDS char*)xs1};
  const WSpan hspan{(GP_LDS char*)hand0, TM * ACT_STRIDE / 1024, (GP_LDS char*)hand1};

  if (stage_a) {
    // ------------------------------------------------------------- stage A
    // X tiles are copied HBM->LDS by the four A waves (wave n issues the
    // 1 KiB wave copies n, n+4, ...).  LDS chunk slot q = 64*i + lane holds
    // row r = q / CPR, physical chunk p = q % CPR, which is logical chunk
    // c = p ^ (r & 15) of that row.  The copy goes through a buffer descriptor
    // whose base is the tile and whose size ends at row M, so rows past M are
    // zero-filled by the hardware range check (their results are never
    // stored).  voff[] are this lane's byte offsets within the tile.
    int voff[C::DMA_PER_WAVE];
#pragma unroll
    for (int ii = 0; ii < C::DMA_PER_WAVE; ++ii) {
      const int q = (ii * 4 + n) * kWave + lane;
      const int r = q / C::CPR;
      const int c = (q - r * C::CPR) ^ (r & 15);
      voff[ii] = (r * K + c * 8) * 2;
    }
    // Descriptor of tile k (empty past the last tile: a copy through it
    // writes zeros to LDS without touching memory).
    // (Gather: the tile of x, whose rows are 128 wide.)
    constexpr int XW = GATHER ? D : K;  // x row width (halves)
    auto tile_rsrc = [&](int k) {
      const int64_t row0 = (t0 + (int64_t)k * G) * TM;
      const int64_t left = (M - row0) * (XW * 2);
      const int bytes = left <= 0 ? 0 : (left < TM * XW * 2 ? (int)left : TM * XW * 2);
      return make_rsrc(p.x + (left > 0 ? row0 * XW : 0), bytes);
    };
    auto issue = [&](int k, GP_LDS char* buf) {
      const __amdgpu_buffer_rsrc_t rsrc = tile_rsrc(k);
#pragma unroll
      for (int ii = 0; ii < C::DMA_PER_WAVE; ++ii) dma16_buf_nt(rsrc, voff[ii], buf + (ii * 4 + n) * 1024);
    };

    // W1 fragment for k-step s: lane holds W1[16s + 8*lh + e][32n + lr].
    // (Non-gather: the first X tile is copied during the W3 part of the prologue.)
    h8 w1f[C::KS1];
    stage_weights_dma<K, GATHER ? 0 : C::DMA_PER_WAVE>(p, xspan, hspan, pro_t, wave, lane, load_prm,
        [&](const WSpan& w1, const WSpan&) {
#pragma unroll
          for (int s = 0; s < C::KS1; ++s) w1f[s] = w_col8(w1, 16 * s + 8 * lh, 32 * n + 16 * ((lane >> 4) & 1), lane & 15);
        },
        [&]() {
          if constexpr (!GATHER) issue(0, (GP_LDS char*)xs0);
        },
        [](const WSpan&) {});
#pragma unroll
    for (int s = 0; s < C::KS1; ++s) asm volatile("" : "+a"(w1f[s]));

    int abar = 0;
    int& abar0 = abar;
    // ---- gather front end ----
    // Copy ii (0..11) of wave n moves segment ii / 4 (0: nf[src], 1: x, 2:
    // nf[dst]) of tile rows 16 (ii & 3) + r0 (r0 = 4n + lane / 16, four rows
    // per copy), logical chunk gc of each row.  The gathered rows' byte
    // offsets in nf (goff) are computed once per tile from the indices, which
    // are copied into LDS (idxs) two tiles ahead by wave 0.  An index outside
    // [0, N) selects an offset past the table: the range check returns zeros.
    const int r0 = 4 * n + (lane >> 4);
    const int gc = (lane & 15) ^ (r0 & 15);
    const __amdgpu_buffer_rsrc_t nf_rsrc = make_rsrc(p.nf, GATHER ? (int)(p.N * (D * 2)) : 0);
    int goff[GATHER ? 8 : 1];  // [src q0..q3, dst q0..q3]
    // All eight indices of a lane are read before any is used, with one LDS
    // read each (both halves of an int64 index at once) and no branches, so
    // their latencies overlap instead of adding up.
    auto gather_offsets = [&](int k) {
      if constexpr (GATHER) {
        unsigned lo[8], hi[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const GP_LDS char* ib =
              (const GP_LDS char*)idxs[k & 1] + (i >> 2) * 1024 + (16 * (i & 3) + r0) * GATHER_IDX;
          if constexpr (GATHER_IDX == 8) {
            const u32x2 v = *(const GP_LDS u32x2*)ib;
            lo[i] = v[0];
            hi[i] = v[1];
          } else {
            lo[i] = *(const GP_LDS unsigned*)ib;
            hi[i] = 0u;
          }
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {  // [src q0..q3, dst q0..q3]
          const bool ok = (hi[i] == 0u) & (lo[i] < (unsigned)p.N);
          goff[i] = ok ? (int)(lo[i] * (unsigned)(D * 2) + gc * 16) : (int)0xFFFFFFF0u;
        }
      }
    };
    auto gather_copy = [&](int ii, __amdgpu_buffer_rsrc_t xrsrc, GP_LDS char* buf) {
      const int seg = ii >> 2, q = ii & 3;
      GP_LDS char* dst = buf + seg * XSEG + (16 * q + 4 * n) * 256;
      if (seg == 1)
        dma16_buf_nt(xrsrc, (16 * q + r0) * 256 + gc * 16, dst);
      else
        dma16_buf(nf_rsrc, goff[(seg >> 1) * 4 + q], dst);
    };
    // Indices of tile k's 64 rows: src into idxs[k & 1][0..), dst at +1024
    // (64 x GATHER_IDX bytes each; lanes past the tile copy zeros into the
    // unused upper part).
    auto index_copy = [&](int k, int which) {
      const int64_t row0 = (t0 + (int64_t)k * G) * TM;
      const int64_t left = (M - row0) * GATHER_IDX;
      const int bytes = left <= 0 ? 0 : (left < TM * GATHER_IDX ? (int)left : TM * GATHER_IDX);
      const char* base = (const char*)(which ? p.dst : p.src) + (left > 0 ? row0 * GATHER_IDX : 0);
      dma16_buf_nt(make_rsrc(base, bytes), lane * 16, (GP_LDS char*)idxs[k & 1] + which * 1024);
    };

    if constexpr (GATHER) {
      if (n == 0) {
        index_copy(0, 0);
        index_copy(0, 1);
        index_copy(1, 0);
        index_copy(1, 1);
      }
      wait_vmcnt<0>();
      group_barrier((GP_LDS int*)&sy.a_bar, abar0, 4, lane, ab, lim);
      gather_offsets(0);
      const __amdgpu_buffer_rsrc_t rsrc = tile_rsrc(0);
#pragma unroll
      for (int ii = 0; ii < C::DMA_PER_WAVE; ++ii) gather_copy(ii, rsrc, (GP_LDS char*)xs0);
    }

    const int xa = lh ^ (lr & 15);  // chunk (2s+lh) of rows lr, lr+32 lands at (2s ^ xa) in its 16-group
    const int xrow = lr * XROW;

    PhaseTimer pt;  // A phases: 0 X wait, 1 A barrier, 2 layer 1, 3 hand-off wait, 4 hand-off store
    auto tile_a = [&](GP_LDS char* xs, GP_LDS char* xnext, GP_LDS char* hand, int k) {
      // X(k) is the only copy in flight.  After the barrier it has landed for
      // every A wave and every A wave is done with tile k-1, whose buffer is
      // refilled with X(k+1) at once.
      pt.tile();
      wait_vmcnt<0>();
      pt.mark(0);
      group_barrier((GP_LDS int*)&sy.a_bar, abar, 4, lane, ab, lim);
      pt.mark(1);
      // Layer 1; the copies of X(k+1) into xnext are issued between its
      // MFMAs, so a busy memory pipeline stalls the copies, not the MFMAs.
      // (Gather: tile k+1's indices landed with X(k); tile k+2's are copied
      // into the index buffer tile k's indices used.)
      gather_offsets(k + 1);
      const __amdgpu_buffer_rsrc_t nrsrc = tile_rsrc(k + 1);
      f16x acc0 = bias_frag(prm[0], fq), acc1 = acc0;
      gemm_2blk<E, C::KS1, PF_L1, 4, C::DMA_PER_WAVE>(w1f, [&](int rb, int s) {
        const int off = (s >> 3) * XSEG + (((2 * s) ^ xa) & 15) * 16;
        return *(const GP_LDS h8*)(xs + xrow + rb * (32 * XROW) + off);
      }, acc0, acc1, [&](int ii) {
        if constexpr (GATHER) {
          gather_copy(ii, nrsrc, xnext);
          if (n == 0 && ii < 2) index_copy(k + 2, ii);
        } else {
          dma16_buf_nt(nrsrc, voff[ii], xnext + (ii * 4 + n) * 1024);
        }
      });

      // Handoff slot k%2 was last read by stage B for tile k-2.
      pt.mark(2);
      if (k >= 2) lds_wait_geq((GP_LDS int*)&sy.h_free, 4 * (k - 1), ab, lim);
      pt.mark(3);
      store_relu_row<E>(hand + arow0, fq, acc0);
      store_relu_row<E>(hand + arow1, fq, acc1);
      lds_signal((GP_LDS int*)&sy.h_full, lane);
      pt.mark(4);
    };

    pt.start();
    for (int k = 0; k < nt; k += 2) {
      tile_a((GP_LDS char*)xs0, (GP_LDS char*)xs1, (GP_LDS char*)hand0, k);
      if (k + 1 < nt) tile_a((GP_LDS char*)xs1, (GP_LDS char*)xs0, (GP_LDS char*)hand1, k + 1);
    }
    wait_vmcnt<0>();  // the (empty) copy issued during the last tile has landed before the waves exit
    pt.finish(wave, lane, nt, t_entry, pro_t);
  } else {
    // ------------------------------------------------------------- stage B
    // W2 (32x32x16 A operand): lane holds W2[16s + 8*lh + e][32n + lr].
    // W3 (16x16x32 A operand) for feature block fb, k-step ks: lane holds
    // W3[32ks + 8*(lane/16) + e][16fb + lane%16] -- all 128 features.
    const int l16 = lane & 15, q4 = lane >> 4;
    h8 w2f[D / 16];
    h8 w3f[8][4];
    stage_weights_dma<K, 0>(p, xspan, hspan, pro_t, wave, lane, load_prm, [&](const WSpan&, const WSpan& w2) {
#pragma unroll
      for (int s = 0; s < D / 16; ++s) w2f[s] = w_col8(w2, 16 * s + 8 * lh, 32 * n + 16 * ((lane >> 4) & 1), lane & 15);
    }, []() {}, [&](const WSpan& w3) {
#pragma unroll
      for (int fb = 0; fb < 8; ++fb)
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) w3f[fb][ks] = w_col8(w3, 32 * ks + 8 * q4, 16 * fb, l16);
    });
#pragma unroll
    for (int s = 0; s < D / 16; ++s) asm volatile("" : "+v"(w2f[s]));
#pragma unroll
    for (int fb = 0; fb < 8; ++fb)
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) asm volatile("" : "+a"(w3f[fb][ks]));

    const int xrow3 = (16 * n + l16) * ACT_STRIDE;  // this lane's layer-3 row in act2

    // Each SIMD runs one A and one B wave.  B is the consumer and carries
    // the waits of the layer-2 -> layer-3 exchange: giving it issue priority
    // keeps the four B waves in step, and A fills the gaps.
    __builtin_amdgcn_s_setprio(1);

    // B phases: 0 hand-off wait, 1 layer 2, 2 exchange-free wait, 3 exchange
    // store, 4 exchange-full wait, 5 layer 3 issue, 6 LayerNorm and stores
    PhaseTimer pt;
    auto tile_b = [&](GP_LDS char* hand, int k) {
      pt.tile();
      // layer 2 bias: its LDS reads overlap the hand-off wait
      f16x acc0 = bias_frag(prm[1], fq), acc1 = acc0;
      lds_wait_geq((GP_LDS int*)&sy.h_full, 4 * (k + 1), ab, lim);
      pt.mark(0);

      // layer 2, features [32n, 32n+32) of all 64 rows, from the handoff tile
      gemm_2blk<E, D / 16, PF_L2, 4>(w2f, [&](int rb, int s) {
        return *(const GP_LDS h8*)(hand + (rb ? arow1 : arow0) + (2 * s + lh) * 16);
      }, acc0, acc1);
      lds_signal((GP_LDS int*)&sy.h_free, lane);  // B operands are in registers: release the slot
      pt.mark(1);

      // exchange: act2 was last read (layer 3) for tile k-1
      if (k >= 1) lds_wait_geq((GP_LDS int*)&sy.x2_free, 4 * k, ab, lim);
      pt.mark(2);
      store_relu_row<E>((GP_LDS char*)act2 + arow0, fq, acc0);
      store_relu_row<E>((GP_LDS char*)act2 + arow1, fq, acc1);
      lds_signal((GP_LDS int*)&sy.x2_full, lane);
      pt.mark(3);
      // layer 3 bias (features 16fb + 4q4 + (0..3)): its reads overlap the exchange wait
      f4 y[8];
#pragma unroll
      for (int fb = 0; fb < 8; ++fb) y[fb] = *(const f4*)&prm[2][16 * fb + 4 * q4];
      lds_wait_geq((GP_LDS int*)&sy.x2_full, 4 * (k + 1), ab, lim);
      pt.mark(4);

      // layer 3, all features of rows [16n, 16n+16): eight independent
      // accumulator chains, issued k-step-major so no MFMA waits on the one before
      h8 bf[4];
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) bf[ks] = *(const GP_LDS h8*)((GP_LDS char*)act2 + xrow3 + (32 * ks + 8 * q4) * 2);
      lds_signal((GP_LDS int*)&sy.x2_free, lane);
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
#pragma unroll
        for (int fb = 0; fb < 8; ++fb) y[fb] = E::mma16(w3f[fb][ks], bf[ks], y[fb]);

      pt.mark(5);
      const int64_t grow = (t0 + (int64_t)k * G) * TM + 16 * n + l16;
      half_t* const orow = p.out + grow * D;
      // After a timed-out wait the tile's inputs are not trustworthy: store nothing.
      const bool st = grow < M && lds_load_relaxed(ab) == 0;
      if constexpr (LN) {
        // Lanes l16, l16+16, l16+32, l16+48 hold the row's 128 features.
        float s = 0.f;
#pragma unroll
        for (int fb = 0; fb < 8; ++fb) s += (y[fb][0] + y[fb][1]) + (y[fb][2] + y[fb][3]);
        const float mu = sum_lanes_16_32(s) * (1.f / D);
        float v = 0.f;
#pragma unroll
        for (int fb = 0; fb < 8; ++fb)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float d = y[fb][e] - mu;
            v = __builtin_fmaf(d, d, v);
          }
        const float rstd = rsqrtf(sum_lanes_16_32(v) * (1.f / D) + p.eps);
        const float nmr = -mu * rstd;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          h4 hv[2];
#pragma unroll
          for (int t = 0; t < 2; ++t) {
            const int fb = 2 * j + t;
            const f4 gm = *(const f4*)&prm[3][16 * fb + 4 * q4];
            const f4 bt = *(const f4*)&prm[4][16 * fb + 4 * q4];
            f4 z;
#pragma unroll
            for (int e = 0; e < 4; ++e) z[e] = __builtin_fmaf(__builtin_fmaf(y[fb][e], rstd, nmr), gm[e], bt[e]);
            hv[t] = E::cvt4(z);
          }
          store_row_pair(orow, hv, j, q4, st);
        }
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const h4 hv[2] = {E::cvt4(y[2 * j]), E::cvt4(y[2 * j + 1])};
          store_row_pair(orow, hv, j, q4, st);
        }
      }
      pt.mark(6);
    };

    pt.start();
    for (int k = 0; k < nt; k += 2) {
      tile_b((GP_LDS char*)hand0, k);
      if (k + 1 < nt) tile_b((GP_LDS char*)hand1, k + 1);
    }
    pt.finish(wave, lane, nt, t_entry, pro_t);
  }
  // The abort word is sticky and is set before the wave that set it gets
  // here, so the workgroup's timeout is reported at least once.
  if (lds_load_relaxed(ab) != 0 && lane == 0) status_fail(p.status, p.epoch, kErrTimeout);
}

}  // namespace fused

// ---------------------------------------------------------------------------
// Host launcher
// ---------------------------------------------------------------------------
template <int K, bool LN, int GI = 0, typename E = fused::ElemF16>
static hipError_t launch_fused(const MgnArgs& a, int grid, hipStream_t stream) {
  fused::Params p{(const half_t*)a.x,  (const half_t*)a.w1, (const half_t*)a.b1, (const half_t*)a.w2,
                  (const half_t*)a.b2, (const half_t*)a.w3, (const half_t*)a.b3, (const half_t*)a.gamma,
                  (const half_t*)a.beta, (half_t*)a.out, a.M, a.eps, (const half_t*)a.nf, a.N, a.src, a.dst,
                  a.status, a.epoch, a.spin_limit > 0 ? a.spin_limit : kSpinLimit};
  hipLaunchKernelGGL((fused::mgn_fused_kernel<K, LN, GI, E>), dim3(grid), dim3(fused::NTHREADS), 0, stream, p);
  return hipGetLastError();
}

int mgn_phase_timers_read(void* dst, int64_t bytes) {
#ifdef GP_PHASE_TIMERS
  const int64_t need = (int64_t)sizeof(fused::g_phase);
  if (dst == nullptr || bytes < need) return -1;
  return hipMemcpyFromSymbol(dst, HIP_SYMBOL(fused::g_phase), need, 0, hipMemcpyDeviceToHost) == hipSuccess ? 0 : -2;
#else
  (void)dst;
  (void)bytes;
  return -3;
#endif
}

hipError_t mgn_fused_launch(const MgnArgs& a, int num_cus, hipStream_t stream) {
  if (a.status == nullptr) return hipErrorInvalidValue;  // every launch reports to a status word
  const int64_t ntiles = (a.M + fused::TM - 1) / fused::TM;
  const int grid = (int)(ntiles < num_cus ? ntiles : num_cus);
  const bool ln = a.gamma != nullptr;
  if (a.nf != nullptr) {  // gather front end (K = 384 = 3 x 128), fp16
    if (a.K != 384 || a.dtype != GP_DTYPE_F16) return hipErrorInvalidValue;
    if (a.idx_bytes == 4)
      return ln ? launch_fused<384, true, 4>(a, grid, stream) : launch_fused<384, false, 4>(a, grid, stream);
    if (a.idx_bytes == 8)
      return ln ? launch_fused<384, true, 8>(a, grid, stream) : launch_fused<384, false, 8>(a, grid, stream);
    return hipErrorInvalidValue;
  }
  using B = fused::ElemBF16;
  if (a.dtype == GP_DTYPE_BF16) {
    switch (a.K) {
      case 384: return ln ? launch_fused<384, true, 0, B>(a, grid, stream) : launch_fused<384, false, 0, B>(a, grid, stream);
      case 256: return ln ? launch_fused<256, true, 0, B>(a, grid, stream) : launch_fused<256, false, 0, B>(a, grid, stream);
      case 128: return ln ? launch_fused<128, true, 0, B>(a, grid, stream) : launch_fused<128, false, 0, B>(a, grid, stream);
      default: return hipErrorInvalidValue;
    }
  }
  if (a.dtype != GP_DTYPE_F16) return hipErrorInvalidValue;
  switch (a.K) {
    case 384: return ln ? launch_fused<384, true>(a, grid, stream) : launch_fused<384, false>(a, grid, stream);
    case 256: return ln ? launch_fused<256, true>(a, grid, stream) : launch_fused<256, false>(a, grid, stream);
    case 128: return ln ? launch_fused<128, true>(a, grid, stream) : launch_fused<128, false>(a, grid, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace gp
