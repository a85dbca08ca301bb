// Persistent multi-workgroup pipelines on MI355X: role assignment by XCD.
//
// The reference lays a pipeline out as a grid column of stage blocks
// (blockIdx.x = stage, blockIdx.y = pipeline row, mgn_fullmlp_pl.cuh:237-251)
// and relies on A100's single L2.  MI355X has eight XCDs with private L2s,
// and a ring queue is only coherent through L2 when producer and consumer sit
// on the same XCD.  So roles are not derived from blockIdx: every workgroup
// reads its hardware XCC id, takes a ticket from its XCD's counter, and after
// a grid-wide barrier the tickets of each XCD are cut into whole pipelines of
// S stage workgroups.  Workgroups left over on an XCD stay idle.
//
// Stages spin on each other, so every workgroup of a launch must be resident
// at once.  The launchers size the grid to the occupancy limit (workgroups
// per CU x CUs) and launch normally: on an otherwise idle GPU the whole grid
// is resident.  If it is not (other work holds CUs), the grid barrier's
// bounded wait runs out, every workgroup leaves with the launch's timeout
// bit set, and gp_pipeline_check reports it.
#pragma once

#include "pipes.hpp"

namespace gp {

constexpr int kMaxXcc = 16;
constexpr int kXcdHint = 8;  // XCDs of an MI355X (launch sizing only; roles use the hardware id)

// Control block at the start of a pipeline arena (zeroed once at allocation).
struct PipeCtl {
  QCounter xcd[kMaxXcc];  // per-XCD ticket counters
  QCounter arrive;        // grid barrier
  QCounter err;           // (epoch << 32) | error bits of the launch (QueueCtx::err)
};

struct Role {
  int pipe;    // global pipeline index, or -1 when idle
  int stage;   // stage index within the pipeline
  int npipes;  // pipelines in this launch
};

__device__ __forceinline__ int xcc_id() {
  // HW_REG_XCC_ID (hwreg 20), bits [3:0]: the XCD this wave runs on
  return __builtin_amdgcn_s_getreg((3 << 11) | (0 << 6) | 20) & (kMaxXcc - 1);
}

// Atomically take the next ticket of counter c in this epoch.
// The atomics are complete when this returns (the ticket must be counted
// before the workgroup arrives at the grid barrier).
__device__ __forceinline__ uint32_t qticket(QCounter* c, uint32_t epoch) {
  const unsigned long long base = (unsigned long long)epoch << 32;
  __hip_atomic_fetch_max(&c->v, base, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __builtin_amdgcn_s_waitcnt(kWaitAll);
  const uint32_t t = (uint32_t)__hip_atomic_fetch_add(&c->v, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __builtin_amdgcn_s_waitcnt(kWaitAll);
  return t;
}

// Workgroup-collective role assignment for pipelines of S stage workgroups.
// XCD y holds p_y = floor(tickets_y / S) pipelines.  Pipelines are numbered
// round-robin over the XCDs (local index l of every XCD before l + 1), so a
// cap of max_pipes > 0 keeps the first max_pipes of that order and the active
// pipelines spread over the XCDs.  A launch with no complete pipeline sets
// kErrNoPipes.
__device__ inline Role assign_role(PipeCtl* ctl, int S, const QueueCtx& ctx, int max_pipes = 0) {
  __shared__ Role role;
  if (threadIdx.x == 0) {
    const int x = xcc_id();
    const int ticket = (int)qticket(&ctl->xcd[x], ctx.epoch);
    qcommit(&ctl->arrive, ctx.epoch);
    // grid barrier: every workgroup has taken its ticket
    bool ok = true;
    for (int it = 0;; ++it) {
      const unsigned long long v = __hip_atomic_load(&ctl->arrive.v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (qcount(v, ctx.epoch) >= gridDim.x) break;
      if (it >= ctx.limit) {
        q_fail(ctx, kErrTimeout);
        ok = false;
        break;
      }
      __builtin_amdgcn_s_sleep(4);
    }
    const int local = ticket / S;
    int p[kMaxXcc];
    int total = 0, index = 0;
#pragma unroll
    for (int y = 0; y < kMaxXcc; ++y) {
      const unsigned long long v = __hip_atomic_load(&ctl->xcd[y].v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      p[y] = (int)qcount(v, ctx.epoch) / S;
      total += p[y];
    }
#pragma unroll
    for (int y = 0; y < kMaxXcc; ++y) index += (p[y] < local ? p[y] : local) + (y < x && p[y] > local ? 1 : 0);
    const int npipes = max_pipes > 0 && max_pipes < total ? max_pipes : total;
    const bool active = ok && local < p[x] && index < npipes;
    if (blockIdx.x == 0 && ok && npipes == 0) q_fail(ctx, kErrNoPipes);
    role = Role{active ? index : -1, ticket % S, npipes};
  }
  __syncthreads();
  const Role r = role;
  __syncthreads();
  return r;
}

}  // namespace gp
