// Device-side building blocks shared by every gpu-pipes kernel on gfx950.
//
// Everything here is written for CDNA4 wave64: MFMA operand fragments, the
// s_waitcnt immediates used to overlap LDS-DMA prefetch with compute, and a
// workgroup barrier that does not wait on in-flight global->LDS copies.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gp {

typedef _Float16 half_t;
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f16x __attribute__((ext_vector_type(16)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef float f2 __attribute__((ext_vector_type(2)));

#define GP_LDS __attribute__((address_space(3)))

constexpr int kWave = 64;

// ---------------------------------------------------------------------------
// s_waitcnt immediates (gfx9 encoding: vmcnt[3:0] | expcnt[6:4] |
// lgkmcnt[11:8] | vmcnt_hi[15:14]).  A field at its maximum means "do not
// wait on this counter".
// ---------------------------------------------------------------------------
constexpr int waitcnt_imm(int vm, int exp, int lgkm) {
  return (vm & 15) | ((exp & 7) << 4) | ((lgkm & 15) << 8) | (((vm >> 4) & 3) << 14);
}
constexpr int kWaitLgkm0 = waitcnt_imm(63, 7, 0);
constexpr int kWaitAll = waitcnt_imm(0, 0, 0);
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt field is 6 bits");
  __builtin_amdgcn_s_waitcnt(waitcnt_imm(N, 7, 15));
}

// Compiler-level fence: keeps the compiler from moving memory operations
// across this point without emitting any hardware wait.
__device__ __forceinline__ void compiler_fence() { asm volatile("" ::: "memory"); }

// Returns v unchanged, but hides its value from the optimiser so that
// expressions derived from it are recomputed where used instead of being
// hoisted out of loops and kept live in registers.
__device__ __forceinline__ int opaque(int v) {
  asm volatile("" : "+v"(v));
  return v;
}

// Workgroup barrier for LDS traffic only.  A HIP __syncthreads() carries a
// workgroup release fence, and on gfx950 a release fence must also drain
// every outstanding global->LDS DMA (vmcnt(0)), which would serialise the
// X-tile prefetch with compute.  This barrier only makes this wave's own
// ds_write results visible (lgkmcnt(0)) before s_barrier; callers wait for
// their DMA explicitly with wait_vmcnt<N>() where needed.
__device__ __forceinline__ void lds_barrier() {
  compiler_fence();
  __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
  __builtin_amdgcn_s_barrier();
  compiler_fence();
}

// ---------------------------------------------------------------------------
// LDS counters for synchronising a subset of the waves of a workgroup
// (s_barrier always involves every wave).  Counters only ever increase;
// a waiter spins until the counter reaches its target.  Each wave first
// drains its own LDS traffic (lgkmcnt(0)) so that everything it wrote
// before signalling is visible to the waves that observe the signal.
// ---------------------------------------------------------------------------
constexpr int kSpinLimit = 1 << 20;  // default poll bound (~0.1 s): a broken protocol ends instead of hanging

__device__ __forceinline__ int lds_load_relaxed(GP_LDS int* c) {
  return __hip_atomic_load((int*)c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// Record error `bits` for launch `epoch` in a status word: the word is lifted
// to (epoch << 32) first (an older launch's value reads as no error), then the
// bits are or-ed in.  Vector atomics at agent scope; one lane calls it.
constexpr unsigned kErrTimeout = 1;
__device__ __forceinline__ void status_fail(unsigned long long* word, uint32_t epoch, unsigned bits) {
  __hip_atomic_fetch_max(word, (unsigned long long)epoch << 32, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __builtin_amdgcn_s_waitcnt(waitcnt_imm(0, 7, 15));
  __hip_atomic_fetch_or(word, (unsigned long long)bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __builtin_amdgcn_s_waitcnt(waitcnt_imm(0, 7, 15));
}

// Add 1 to an LDS counter once per wave, after this wave's LDS writes.
__device__ __forceinline__ void lds_signal(GP_LDS int* c, int lane) {
  compiler_fence();
  __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
  if (lane == 0) __hip_atomic_fetch_add((int*)c, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  compiler_fence();
}

// Spin until an LDS counter is >= target (every lane reads the same word).
// If `limit` polls run out, the sticky abort word is set and every later wait
// of the workgroup returns at once, so the kernel always terminates; the
// kernel then skips its output stores and reports the timeout (status_fail).
__device__ __forceinline__ void lds_wait_geq(GP_LDS int* c, int target, GP_LDS int* abort, int limit) {
  compiler_fence();
  for (int it = 0;; ++it) {
    if (lds_load_relaxed(c) >= target || lds_load_relaxed(abort) != 0) break;
    if (it >= limit) {
      __hip_atomic_store((int*)abort, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      break;
    }
    __builtin_amdgcn_s_sleep(1);
  }
  compiler_fence();
}

// Barrier among the `nw` waves that share counter c; `gen` is this wave's
// running target (starts at 0, advanced by nw per barrier).
__device__ __forceinline__ void group_barrier(GP_LDS int* c, int& gen, int nw, int lane, GP_LDS int* abort,
                                              int limit) {
  gen += nw;
  lds_signal(c, lane);
  lds_wait_geq(c, gen, abort, limit);
}

// 16-byte global->LDS copy.  Lane i of the wave writes LDS bytes
// [lds_base + 16 i, lds_base + 16 i + 16); lds_base must be wave-uniform.
// The source address is per lane, so the LDS layout is chosen by picking
// which global chunk each lane fetches.
__device__ __forceinline__ void dma16(const void* gsrc, GP_LDS void* lds_base) {
  __builtin_amdgcn_global_load_lds(gsrc, lds_base, 16, 0, 0);
}

// Raw buffer descriptor over [base, base + nbytes) (gfx9 word 3: 0x00020000).
// Buffer accesses at offsets >= nbytes are discarded by the hardware range
// check: loads return zero, stores are dropped.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int nbytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, nbytes, 0x00020000);
}

// 16-byte buffer->LDS copy: lane i fetches rsrc[voffset .. voffset+16) into
// LDS bytes [lds_base + 16 i, lds_base + 16 i + 16).
__device__ __forceinline__ void dma16_buf(__amdgpu_buffer_rsrc_t rsrc, int voffset, GP_LDS void* lds_base) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, lds_base, 16, voffset, 0, 0, 0);
}
// The same with a wave-uniform byte offset in an SGPR (soffset) added to the
// per-lane voffset.
__device__ __forceinline__ void dma16_buf_so(__amdgpu_buffer_rsrc_t rsrc, int voffset, int soffset,
                                             GP_LDS void* lds_base) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, lds_base, 16, voffset, soffset, 0, 0);
}
// The same with the non-temporal cache policy (nt): for data read exactly
// once, which should not displace reusable lines from L2.
__device__ __forceinline__ void dma16_buf_nt(__amdgpu_buffer_rsrc_t rsrc, int voffset, GP_LDS void* lds_base) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, lds_base, 16, voffset, 0, 0, 2);
}

// 8-byte buffer load / store of four fp16 values at byte offset `off`.
// Accesses at or beyond the descriptor's range read zero / are dropped, which
// is how partial tiles are bounded without per-row branches.
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ h4 buf_load_h4(__amdgpu_buffer_rsrc_t rsrc, int off) {
  return __builtin_bit_cast(h4, __builtin_amdgcn_raw_buffer_load_b64(rsrc, off, 0, 0));
}
__device__ __forceinline__ void buf_store_h4(__amdgpu_buffer_rsrc_t rsrc, int off, h4 v) {
  __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, v), rsrc, off, 0, 0);
}
__device__ __forceinline__ void buf_store_u4(__amdgpu_buffer_rsrc_t rsrc, int off, u32x4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(v, rsrc, off, 0, 0);
}

// ---------------------------------------------------------------------------
// MFMA 32x32x16 f16 -> f32.  Operand layout (wave64):
//   A[i][k]: lane = i + 32*(k/8), element k%8          (32 rows x 16 k)
//   B[k][j]: lane = j + 32*(k/8), element k%8          (16 k x 32 cols)
//   C[i][j]: lane = j + 32*((i/4)%2), element (i%4) + 4*(i/8)
// ---------------------------------------------------------------------------
__device__ __forceinline__ f16x mfma32(h8 a, h8 b, f16x c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// Row (M index) of accumulator element v held by a lane in half `lh` (= lane/32).
__device__ __forceinline__ constexpr int c_row(int v, int lh) {
  return 8 * (v / 4) + 4 * lh + (v % 4);
}

__device__ __forceinline__ float relu(float v) { return v > 0.f ? v : 0.f; }

// x + (x of the lane 32 positions away), in every lane: one
// v_permlane32_swap (a VALU exchange of the two wave halves) instead of an
// LDS permute.
__device__ __forceinline__ float sum_lane_halves(float x) {
  const unsigned u = __builtin_bit_cast(unsigned, x);
  const auto p = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return __builtin_bit_cast(float, (unsigned)p[0]) + __builtin_bit_cast(float, (unsigned)p[1]);
}

// ---------------------------------------------------------------------------
// Weight rows staged in LDS.  A weight matrix W (rows of 128 16-bit values)
// is copied HBM->LDS in its own row-major shape, 256 bytes per row, four rows
// per 1 KiB copy, with 16-byte chunk c of row r at chunk position
// c ^ 4 (r % 4).  Lane l of a copy fetches row l/16 of the copy's four,
// chunk (l % 16) ^ 4 (l / 16): wrow_voff is that byte offset for a row
// stride of `stride` bytes.
// ---------------------------------------------------------------------------
__device__ __forceinline__ int wrow_voff(int lane, int stride) {
  const int r = lane >> 4;
  return r * stride + ((lane & 15) ^ (4 * r)) * 16;
}

// MFMA A fragments are columns of W (consecutive k of one feature).
// ds_read_b64_tr_b16 transposes within each group of 16 lanes: when lane m of
// the group points at the four 16-bit values S[m][0..3], lane j receives
// S[4e + j/4][j % 4], e = 0..3.  With lane m pointing at row kb + m/4,
// features fb + 4 (m % 4) .. +3 (kb a multiple of 4, fb of 16), lane j
// receives W[kb + e][fb + j].  blk is the LDS address of row kb.  The 32
// lanes of a wave half read four rows x 64 bytes that the swizzle puts in
// four different chunk groups, so the read is conflict free.
typedef short s4 __attribute__((ext_vector_type(4)));
typedef short s8 __attribute__((ext_vector_type(8)));
__device__ __forceinline__ s4 wrows_col4(const GP_LDS char* blk, int fb, int m) {
  const int r = m >> 2, f = fb + 4 * (m & 3);
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((GP_LDS s4*)(blk + r * 256 + (((f >> 3) ^ (4 * r)) * 16) + (f & 7) * 2));
}
// Eight consecutive k: lane j receives W[kb + e][fb + j], e = 0..7, from the
// four-row blocks at blk0 (rows kb..kb+3) and blk1 (rows kb+4..kb+7).
__device__ __forceinline__ h8 wrows_col8(const GP_LDS char* blk0, const GP_LDS char* blk1, int fb, int m) {
  const s4 a = wrows_col4(blk0, fb, m), b = wrows_col4(blk1, fb, m);
  return __builtin_bit_cast(h8, __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7));
}

// ---------------------------------------------------------------------------
// Element types of the wide GEMM and the NeRF kernel.  Operands, bias,
// residual, affine and output are 16-bit values held as raw bits in half_t
// containers; only the MFMA form, the conversions to / from fp32 and the
// value 1.0 differ.  Arithmetic is fp32.
typedef __bf16 bf8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
struct F16 {
  static constexpr unsigned short kOne = 0x3C00;
  __device__ static f16x mma(h8 a, h8 b, f16x c) { return mfma32(a, b, c); }
  __device__ static float val(half_t h) { return (float)h; }
  __device__ static h4 cvt4(f4 v) { return __builtin_convertvector(v, h4); }
  __device__ static h2 cvt2(f2 v) { return __builtin_convertvector(v, h2); }
  __device__ static half_t cvt1(float v) { return (half_t)v; }
};
struct BF16 {
  static constexpr unsigned short kOne = 0x3F80;
  __device__ static f16x mma(h8 a, h8 b, f16x c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf8, a), __builtin_bit_cast(bf8, b), c, 0, 0, 0);
  }
  __device__ static float val(half_t h) {
    return __builtin_bit_cast(float, (unsigned)__builtin_bit_cast(unsigned short, h) << 16);
  }
  // v_cvt_pk_bf16_f32: round to nearest even
  __device__ static h4 cvt4(f4 v) { return __builtin_bit_cast(h4, __builtin_convertvector(v, bf4)); }
  __device__ static h2 cvt2(f2 v) { return __builtin_bit_cast(h2, __builtin_convertvector(v, bf2)); }
  __device__ static half_t cvt1(float v) { return __builtin_bit_cast(half_t, (__bf16)v); }
};

}  // namespace gp
