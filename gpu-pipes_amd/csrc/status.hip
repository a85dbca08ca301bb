// Launch status words: where a kernel whose device-side waits are bounded
// records that a wait ran out, so that gp_pipeline_check can report it.
//
// The reference has no such report: its queue waits spin forever
// (common/mpmcq.cuh:83,104).  Here a kernel that gives up a wait writes
// (epoch << 32) | error bits into its launch's status word and ends normally.
//
// The fused kernels take their word from a file-scope device array, so the
// entry points that launch them allocate nothing.  Every GPU holds its own copy
// of the array at its own address, found once per device with
// hipGetSymbolAddress; each (device, stream) pair keeps one slot of it, and
// every launch takes a new epoch of its device, so a word left by an earlier
// launch never reads as an error of a later one.  The array is zero when the
// library is loaded (epoch 0 is never handed out).  The pipelined kernels keep
// their word in their queue arena instead and register it with status_note().
#include <hip/hip_runtime.h>

#include <atomic>
#include <map>
#include <mutex>
#include <utility>

#include "../../include/gpipes.h"
#include "gp_host.hpp"

namespace gp {

constexpr int kStatusSlots = 4096;  // (device, stream) pairs before slots are shared
static __device__ __align__(256) unsigned long long status_words[kStatusSlots];

namespace {
struct DevStatus {
  unsigned long long* base = nullptr;  // device address of status_words on this device
  uint32_t epoch = 0;                  // last epoch handed out on this device
  int next_slot = 0;
};
struct LastLaunch {
  unsigned long long* word = nullptr;
  uint32_t epoch = 0;
};
std::mutex g_status_mu;
DevStatus g_devs[64];
std::map<std::pair<int, hipStream_t>, int> g_slots;
std::map<std::pair<int, hipStream_t>, LastLaunch> g_last;
std::atomic<long long> g_wait_limit{0};
}  // namespace

int status_acquire(int dev, hipStream_t stream, unsigned long long** word, uint32_t* epoch) {
  if (dev < 0 || dev >= 64) return fail(GP_ERR_NO_DEVICE, "device index %d out of range", dev);
  std::lock_guard<std::mutex> lk(g_status_mu);
  DevStatus& d = g_devs[dev];
  if (d.base == nullptr) {
    // The caller made `dev` current; this also loads the code object there.
    hipError_t e = hipGetSymbolAddress((void**)&d.base, HIP_SYMBOL(status_words));
    if (e != hipSuccess) {
      d.base = nullptr;
      return fail_hip(e, "hipGetSymbolAddress (launch status words)");
    }
  }
  auto it = g_slots.find({dev, stream});
  int slot;
  if (it == g_slots.end()) {
    slot = d.next_slot;
    d.next_slot = (d.next_slot + 1) % kStatusSlots;
    g_slots[{dev, stream}] = slot;
  } else {
    slot = it->second;
  }
  if (++d.epoch == 0) d.epoch = 1;
  *word = d.base + slot;
  *epoch = d.epoch;
  g_last[{dev, stream}] = LastLaunch{*word, *epoch};
  return GP_OK;
}

void status_note(int dev, hipStream_t stream, unsigned long long* word, uint32_t epoch) {
  std::lock_guard<std::mutex> lk(g_status_mu);
  g_last[{dev, stream}] = LastLaunch{word, epoch};
}

int status_last(int dev, hipStream_t stream, unsigned long long** word, uint32_t* epoch) {
  std::lock_guard<std::mutex> lk(g_status_mu);
  auto it = g_last.find({dev, stream});
  if (it == g_last.end() || it->second.word == nullptr)
    return fail(GP_ERR_INVALID_ARG, "no launch that reports its status on this stream");
  *word = it->second.word;
  *epoch = it->second.epoch;
  return GP_OK;
}

long long wait_limit(long long dflt) {
  const long long v = g_wait_limit.load(std::memory_order_relaxed);
  return v > 0 ? v : dflt;
}

void set_wait_limit(long long polls) { g_wait_limit.store(polls > 0 ? polls : 0, std::memory_order_relaxed); }

}  // namespace gp
