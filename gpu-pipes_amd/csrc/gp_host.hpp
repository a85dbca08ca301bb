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
int mgn_pipelined_run(const MgnArgs& a, int dev, int num_cus, hipStream_t stream);

}  // namespace gp
