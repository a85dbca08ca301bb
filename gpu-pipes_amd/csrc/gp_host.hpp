// Host-side helpers shared by the C ABI translation units.
#pragma once

#include <hip/hip_runtime.h>

#include "gp_kernels.hpp"

namespace gp {

// Record a failure message for gp_last_error() and return `code`.
int fail(int code, const char* fmt, ...);
int fail_hip(hipError_t e, const char* what);
void clear_error();

// Current device id and CU count; fails unless the device is gfx950.
int current_device_info(int* dev_out, int* num_cus);

// Validate an MGN call (shapes, pointers, alignment).
int check_mgn_args(const MgnArgs& a);

// Stage-chained implementation (workgroup stages linked by L2 ring queues).
// split_ln: the reference's layout with separate LayerNorm workers.
int mgn_pipelined_run(const MgnArgs& a, bool split_ln, int dev, int num_cus, hipStream_t stream);

// Identity pipelines through ring queues (tests the queue protocol).
int pipe_route_run(int64_t M, const void* x, void* out, void* out2, int route, int max_pipes, int dev, int num_cus,
                   hipStream_t stream);

// Queue arenas, one per (device, stream), zeroed when allocated and when the
// queue layout changes; each call returns a new launch epoch.  arena_last
// returns the arena and epoch of the last call.
constexpr uint32_t kArenaLayoutMgn = 1;    // mgn_pipelined Queues
constexpr uint32_t kArenaLayoutRoute = 2;  // route kernels (+1 for the split layout)
int arena_acquire(int dev, hipStream_t stream, size_t bytes, uint32_t layout, void** base, uint32_t* epoch);
int arena_last(int dev, hipStream_t stream, void** base, uint32_t* epoch);

// Scratch memory of the wide operators, one per (device, stream), grown on
// demand (a grow synchronises the stream); contents are not preserved.
int workspace_acquire(int dev, hipStream_t stream, size_t bytes, void** base);

bool aligned16(const void* p);

}  // namespace gp
