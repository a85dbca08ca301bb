// Queue arenas for the pipelined kernels.
//
// The reference keeps one process-global queue buffer per app, allocated on
// first use and never freed (mgn_fullmlp_pl.cuh:255-266), shared by every
// stream and device.  Here an arena is kept per (device, stream): launches on
// one stream are ordered by the stream, launches on different streams use
// different arenas.  An arena is zeroed once when allocated; afterwards every
// launch gets a fresh epoch number and the device code treats counters of
// older epochs as zero, so no per-launch reset is needed -- as long as the
// launches share a queue layout.  A launch with a different layout (another
// kernel, whose payload may lie where this one's counters are) zeroes the
// arena once first.
//
// Workspaces hold the intermediates of the unpipelined wide operators (the
// BERT FFN's transposed weights and activation chunks): one per (device,
// stream), grown on demand, never zeroed.
#include <hip/hip_runtime.h>

#include <map>
#include <mutex>
#include <utility>

#include "../../include/gpipes.h"
#include "gp_host.hpp"

namespace gp {

namespace {
// True when work enqueued on `stream` is being captured into a graph.
bool capturing(hipStream_t stream) {
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  return hipStreamIsCapturing(stream, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone;
}
}  // namespace

int refuse_capture(hipStream_t stream) {
  if (capturing(stream))
    return fail(GP_ERR_INVALID_ARG,
                "queue-chained launches cannot be captured into a graph (each launch takes a new queue epoch)");
  return GP_OK;
}

namespace {
struct ArenaRec {
  void* base = nullptr;
  size_t bytes = 0;
  uint32_t epoch = 0;   // last epoch handed out
  uint32_t layout = 0;  // queue layout of the last launch (0: none)
};
std::mutex g_mu;
std::map<std::pair<int, hipStream_t>, ArenaRec> g_arenas;
}  // namespace

int arena_acquire(int dev, hipStream_t stream, size_t bytes, uint32_t layout, void** base, uint32_t* epoch) {
  // A graph would replay the captured epoch, and counters left by the
  // previous replay would then satisfy the next replay's waits.
  if (int rc = refuse_capture(stream)) return rc;
  std::lock_guard<std::mutex> lk(g_mu);
  ArenaRec& a = g_arenas[{dev, stream}];
  if (a.bytes >= bytes && a.layout != layout) {
    // Another kernel's queue layout used this memory: its payload bytes could
    // sit where this layout keeps counters, so the arena is zeroed again
    // (ordered on the stream, after the previous launch).
    hipError_t e = hipMemsetAsync(a.base, 0, a.bytes, stream);
    if (e != hipSuccess) return fail_hip(e, "hipMemsetAsync (queue arena)");
  }
  a.layout = layout;
  if (a.bytes < bytes) {
    if (a.base) {
      // the old arena may still be in use by work queued on this stream
      hipError_t e = hipStreamSynchronize(stream);
      if (e != hipSuccess) return fail_hip(e, "hipStreamSynchronize (arena growth)");
      e = hipFree(a.base);
      if (e != hipSuccess) return fail_hip(e, "hipFree (arena growth)");
      a.base = nullptr;
      a.bytes = 0;
    }
    hipError_t e = hipMalloc(&a.base, bytes);
    if (e != hipSuccess) return fail_hip(e, "hipMalloc (queue arena)");
    e = hipMemsetAsync(a.base, 0, bytes, stream);
    if (e != hipSuccess) return fail_hip(e, "hipMemsetAsync (queue arena)");
    a.bytes = bytes;
    a.epoch = 0;
  }
  if (++a.epoch == 0) a.epoch = 1;  // epoch 0 is the zeroed state
  *base = a.base;
  *epoch = a.epoch;
  return GP_OK;
}

namespace {
struct WorkRec {
  void* base = nullptr;
  size_t bytes = 0;
};
std::map<std::pair<int, hipStream_t>, WorkRec> g_work;
}  // namespace

int workspace_acquire(int dev, hipStream_t stream, size_t bytes, void** base) {
  // A captured graph would keep the workspace address, which a later, larger
  // call on the stream frees.
  if (capturing(stream))
    return fail(GP_ERR_INVALID_ARG,
                "calls that use the per-stream workspace cannot be captured into a graph "
                "(the allocation-free entry points can)");
  std::lock_guard<std::mutex> lk(g_mu);
  WorkRec& w = g_work[{dev, stream}];
  if (w.bytes < bytes) {
    if (w.base) {
      hipError_t e = hipStreamSynchronize(stream);  // earlier launches may still use it
      if (e != hipSuccess) return fail_hip(e, "hipStreamSynchronize (workspace growth)");
      e = hipFree(w.base);
      if (e != hipSuccess) return fail_hip(e, "hipFree (workspace growth)");
      w.base = nullptr;
      w.bytes = 0;
    }
    hipError_t e = hipMalloc(&w.base, bytes);
    if (e != hipSuccess) return fail_hip(e, "hipMalloc (workspace)");
    w.bytes = bytes;
  }
  *base = w.base;
  return GP_OK;
}

}  // namespace gp
