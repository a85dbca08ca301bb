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

// The reference's queue-chained layouts of the bert_addln_ffn and nerf_a apps
// (stage workgroups linked by L2 ring queues; pipe_add / pipe_concat stages
// fed from queues).  H 128 / FF 512 and Kx a multiple of 8 up to 128 only.
int bert_addln_pipelined_run(const BertAddlnArgs& a, int dev, int num_cus, hipStream_t stream);
// The bert_ffn app's queue-chained layout (four W1 column slices, two W2 +
// residual + LayerNorm workers), H 128 / FF 512 only.
int bert_ffn_pipelined_run(const BertFfnArgs& a, int dev, int num_cus, hipStream_t stream);
int nerf_a_pipelined_run(const NerfAArgs& a, int dev, int num_cus, hipStream_t stream);

// Identity pipelines through ring queues (tests the queue protocol).
int pipe_route_run(int64_t M, const void* x, void* out, void* out2, int route, int max_pipes, int dev, int num_cus,
                   hipStream_t stream);

// Queue arenas, one per (device, stream), zeroed when allocated and when the
// queue layout changes; each call returns a new launch epoch.
constexpr uint32_t kArenaLayoutMgn = 1;    // mgn_pipelined Queues
constexpr uint32_t kArenaLayoutRoute = 2;  // route kernels (+1 for the split layout)
constexpr uint32_t kArenaLayoutBertAddln = 4;
constexpr uint32_t kArenaLayoutNerfA = 5;
constexpr uint32_t kArenaLayoutGemmLn = 6;  // LayerNorm-epilogue GEMMs: partial row statistics
constexpr uint32_t kArenaLayoutBertFfn = 7;
constexpr uint32_t kArenaLayoutMgnSplit = 8;  // mgn_pipelined's split-LayerNorm layout
constexpr uint32_t kArenaLayoutRouteReload = 9;  // the one-slot route of 64-row entries
// GP_ERR_INVALID_ARG if `stream` is capturing into a graph: the queue-chained
// launches call it before any other HIP call (a replay would reuse the
// captured queue epoch).
int refuse_capture(hipStream_t stream);
int arena_acquire(int dev, hipStream_t stream, size_t bytes, uint32_t layout, void** base, uint32_t* epoch);

// Scratch memory of the wide operators, one per (device, stream), grown on
// demand (a grow synchronises the stream); contents are not preserved.
int workspace_acquire(int dev, hipStream_t stream, size_t bytes, void** base);

// Launch status (status.hip).  status_acquire gives a launch on (dev, stream)
// its device status word and a new epoch, and records it as the stream's last
// reporting launch; status_note records a word kept elsewhere (the pipelined
// kernels' arena); status_last returns the stream's last record, which
// gp_pipeline_check reads.  A word reads as a failure of the launch when its
// high 32 bits equal the launch's epoch and its low bits are non-zero.
int status_acquire(int dev, hipStream_t stream, unsigned long long** word, uint32_t* epoch);
void status_note(int dev, hipStream_t stream, unsigned long long* word, uint32_t epoch);
int status_last(int dev, hipStream_t stream, unsigned long long** word, uint32_t* epoch);
// Poll bound of the device-side waits of later launches: the test hook
// gp_set_wait_limit's value, or dflt when none is set.
long long wait_limit(long long dflt);
void set_wait_limit(long long polls);

bool aligned16(const void* p);

}  // namespace gp
