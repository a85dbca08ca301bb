// Stage-chaining API for gfx950: tile views, readers / writers and the
// inter-workgroup ring queue.
//
// Reference: common/pipes.cuh:7-108 (MemoryReader, read_striped_input,
// NullReader, QueueReader, SplitQueueReader, MemoryWriter, QueueWriter,
// SplitQueueWriter, NullWriter), common/mpmcq.cuh:10-115 (QueueSlot,
// MpmcRingQueue) and common/common.cuh:3-6 (TensorView).  The names, the
// acquire / release call pattern and the round-robin split semantics are the
// reference's; the queue protocol is redesigned for MI355X:
//
//  * Every reader / writer call is workgroup-collective (all threads call it);
//    one thread spins and the result is broadcast with a barrier.  The
//    reference's per-warp spinning (mpmcq.cuh:79-88) has no wave64 analogue.
//  * A slot has two monotonic 64-bit counters, "full" (producer commits) and
//    "empty" (consumer commits), each on its own 128-byte line, tagged with the
//    launch epoch in the high 32 bits.  Nothing is ever reset, so there is no
//    reset race (mpmcq.cuh:42-54, 68-75) and back-to-back launches need no
//    memset: a counter from an older epoch reads as zero.
//  * Release: the producer's payload stores are complete in L2 (vmcnt(0) in
//    every wave, then a barrier) before the commit atomic.  Acquire: after the
//    consumer observes the counter, its payload loads carry the agent-scope
//    cache policy (SC1), so they are served by L2, not by a stale L1 line.
//    The reference has no fences at all
//    (mpmcq.cuh:34-40).  Producer and consumer must share an XCD (one L2):
//    the pipelined kernels assign stage roles by the hardware XCC id.
//  * Waits are bounded: on timeout an error word is set and every later wait
//    of the launch returns at once, so a broken pipeline ends instead of
//    hanging; the host reports it as GP_ERR_TIMEOUT.
//  * TensorView carries the number of valid rows, so the last, partial tile of
//    an arbitrary M is handled (the reference drops it, mgn_fullmlp_pl.cuh:84).
#pragma once

#include "gp_device.hpp"

namespace gp {

// common/common.cuh:3-6: non-owning fp16 tile view.  `stride` is the row
// stride in elements (0 = one row broadcast to all rows, e.g. a bias);
// `rows` is the number of valid rows of the tile.
struct TensorView {
  half_t* data;
  int stride;
  int rows;
};

// ---------------------------------------------------------------------------
// Launch context shared by every queue of a kernel launch.
// ---------------------------------------------------------------------------
struct QueueCtx {
  uint32_t epoch;            // launch epoch (never 0)
  unsigned long long* err;   // (epoch << 32) | error bits; bits of this epoch abort all waits
  int limit;                 // polls before a wait gives up (kQueueSpinLimit unless a test lowers it)
};

constexpr int kQueueSpinLimit = 1 << 22;  // default: polls of ~1 us before a wait gives up
constexpr unsigned kErrNoPipes = 2;  // the launch held no complete pipeline

__device__ __forceinline__ bool q_aborted(const QueueCtx& c) {
  const unsigned long long v = __hip_atomic_load(c.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return (uint32_t)(v >> 32) == c.epoch && (uint32_t)v != 0;
}

__device__ __forceinline__ void q_fail(const QueueCtx& c, unsigned bits) { status_fail(c.err, c.epoch, bits); }

struct alignas(128) QCounter {
  unsigned long long v;  // (epoch << 32) | count
  char pad[120];
};

__device__ __forceinline__ uint32_t qcount(unsigned long long v, uint32_t epoch) {
  return (uint32_t)(v >> 32) == epoch ? (uint32_t)v : 0u;
}

// Count one commit on `c` in this epoch (thread-level; called by one thread).
// The max lifts a counter left by an older launch to (epoch << 32) | 0; it
// must be complete before the add, so the wave waits for it in between.  Only
// a slot's first round of the launch needs it (first = seq < N): the protocol
// orders every later commit of that counter after the first one.  The add is
// not waited for: nothing this workgroup does next depends on its completion.
__device__ __forceinline__ void qcommit(QCounter* c, uint32_t epoch, bool first = true) {
  const unsigned long long base = (unsigned long long)epoch << 32;
  if (first) {
    __hip_atomic_fetch_max(&c->v, base, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_s_waitcnt(kWaitAll);
  }
  __hip_atomic_fetch_add(&c->v, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Workgroup-collective: wait until count(c) >= target.  Returns false if the
// launch was aborted (timeout here or elsewhere).
__device__ __forceinline__ bool qwait(QCounter* c, uint32_t target, const QueueCtx& ctx) {
  __shared__ int ok;
  if (threadIdx.x == 0) {
    int r = 1;
    for (int it = 0;; ++it) {
      const unsigned long long v = __hip_atomic_load(&c->v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (qcount(v, ctx.epoch) >= target) break;
      if (q_aborted(ctx)) {
        r = 0;
        break;
      }
      if (it >= ctx.limit) {
        q_fail(ctx, kErrTimeout);
        r = 0;
        break;
      }
      __builtin_amdgcn_s_sleep(4);
    }
    ok = r;
  }
  __syncthreads();
  const bool res = ok != 0;
  __syncthreads();  // `ok` is reused by the next wait
  return res;
}

// Acquire side.  A queue's producers and consumers run on different CUs of one
// XCD, and the vector L1 of a CU is not kept coherent with stores from other
// CUs.  `buffer_inv sc0` (the L1 invalidate of a workgroup-scope acquire) does
// not drop those lines either: a one-slot queue of 16 KiB entries, re-read by
// its consumer every tile, delivered the slot's previous round from L1.  So
// every load of a queue payload carries the agent-scope cache policy (SC1),
// which reads the L2 that the producer's stores reached, and no invalidate is
// issued: the agent-scope acquire fence (`buffer_inv sc1`) would also drop the
// L2's lines of other memory types, which cost the pipelined MGN edge MLP 0.88
// against 0.63 ms per call.  The counters and the row count are read with
// agent-scope atomic / volatile loads, which bypass the L1 as well.
constexpr int kQueueLoadAux = 16;  // cache-policy bits of a buffer load: SC1

// 16 bytes at element `off` of a tile view, from a queue payload (Q, the SC1
// policy) or from memory.  Loads of a queue view stay below its row count.
template <bool Q>
__device__ __forceinline__ h8 view_load_h8(const TensorView& v, int64_t off) {
  if constexpr (Q) {
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(v.data, v.rows * v.stride * 2);
    return __builtin_bit_cast(h8, __builtin_amdgcn_raw_buffer_load_b128(rs, (int)(off * 2), 0, kQueueLoadAux));
  } else {
    return *(const h8*)(v.data + off);
  }
}

// Release side, workgroup-collective: every store of every wave is complete
// in L2 once this returns.
__device__ __forceinline__ void stores_complete() {
  __builtin_amdgcn_s_waitcnt(kWaitAll);
  __syncthreads();
}

// ---------------------------------------------------------------------------
// Queue payloads
// ---------------------------------------------------------------------------
// mgn_fullmlp_pl.cuh:13-21: a queue entry is an [M][D] fp16 tile.
template <int MBLK, int D>
struct QueueEntry2D {
  static constexpr int kRows = MBLK, kCols = D;
  half_t buf[MBLK][D];
  __device__ half_t* as_ptr() { return &buf[0][0]; }
  __device__ TensorView as_view(int rows) { return {as_ptr(), D, rows < 0 ? 0 : (rows > MBLK ? MBLK : rows)}; }
};

template <typename Entry>
struct alignas(128) QueueSlot {
  QCounter full;   // producer commits
  QCounter empty;  // consumer commits
  int rows;        // valid rows of the payload
  char pad[124];
  Entry data;
};

// Ring of N slots with NP producers and NC consumers per sequence number
// (mpmcq.cuh:66-115).  Sequence s lives in slot s % N, round s / N.
template <typename Entry, int N, int NP = 1, int NC = 1>
struct RingQueue {
  using Item = Entry;
  QueueSlot<Entry> slots[N];

  __device__ QueueSlot<Entry>& slot(int64_t seq) { return slots[seq % N]; }

  // Wait until the slot of `seq` has been drained by the previous round.
  __device__ Entry* write_wait(int64_t seq, const QueueCtx& ctx) {
    QueueSlot<Entry>& s = slot(seq);
    qwait(&s.empty, (uint32_t)(seq / N) * NC, ctx);
    return &s.data;
  }
  __device__ void write_commit(int64_t seq, int rows, const QueueCtx& ctx) {
    QueueSlot<Entry>& s = slot(seq);
    if (threadIdx.x == 0) s.rows = rows;
    stores_complete();
    if (threadIdx.x == 0) qcommit(&s.full, ctx.epoch, seq < N);
  }
  // Wait until all NP producers of `seq` have committed; returns the payload.
  // After an aborted wait the slot holds no tile of this launch: the view has
  // no rows, so the consumer stores nothing for it.
  __device__ Entry* read_wait(int64_t seq, int* rows, const QueueCtx& ctx) {
    QueueSlot<Entry>& s = slot(seq);
    const bool ok = qwait(&s.full, (uint32_t)(seq / N + 1) * NP, ctx);
    *rows = ok ? *(volatile int*)&s.rows : 0;
    return &s.data;
  }
  __device__ void read_commit(int64_t seq, const QueueCtx& ctx) {
    stores_complete();  // this workgroup's loads of the payload have returned
    if (threadIdx.x == 0) qcommit(&slot(seq).empty, ctx.epoch, seq < N);
  }
  // read_commit for a caller whose every wave has already waited for its
  // loads of the payload (vmcnt(0)) and passed a barrier since.
  __device__ void read_commit_landed(int64_t seq, const QueueCtx& ctx) {
    if (threadIdx.x == 0) qcommit(&slot(seq).empty, ctx.epoch, seq < N);
  }
  // Thread-level, no wait: have all NP producers of `seq` committed?  A
  // consumer that sees true may load the payload (with the SC1 policy).
  __device__ bool full_peek(int64_t seq, const QueueCtx& ctx) {
    const unsigned long long v = __hip_atomic_load(&slot(seq).full.v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return qcount(v, ctx.epoch) >= (uint32_t)(seq / N + 1) * NP;
  }
  __device__ int rows_of(int64_t seq) { return *(volatile int*)&slot(seq).rows; }
};

// ---------------------------------------------------------------------------
// Readers.  Concept: TensorView read_acquire(); void read_release(); void reset().
// kFromQueue tells a stage that the tile lives in another workgroup's output
// (the stage then orders its own payload loads after the acquire).
// ---------------------------------------------------------------------------

// pipes.cuh:7-19.  Walks tiles of `tile_rows` rows: tile i starts at
// base + i * stride elements; `rows_left` bounds the valid rows.
struct MemoryReader {
  static constexpr bool kFromQueue = false;
  __device__ void read_release_landed() { read_release(); }
  half_t* base;
  int64_t stride;
  int tile_stride;
  int tile_rows;
  int64_t rows_left0;
  int64_t row_step;
  int64_t offset = 0;
  int64_t rows_left = 0;

  __device__ MemoryReader(half_t* base_, int64_t stride_, int tile_stride_, int tile_rows_ = 1 << 30,
                          int64_t rows_left_ = int64_t(1) << 62, int64_t row_step_ = 0)
      : base(base_), stride(stride_), tile_stride(tile_stride_), tile_rows(tile_rows_), rows_left0(rows_left_),
        row_step(row_step_ ? row_step_ : tile_rows_), rows_left(rows_left_) {}

  __device__ TensorView read_acquire() {
    const int64_t r = rows_left < tile_rows ? rows_left : tile_rows;
    return {base + offset, tile_stride, (int)(r > 0 ? r : 0)};
  }
  __device__ void read_release() {
    offset += stride;
    rows_left -= row_step;
  }
  __device__ void reset() {
    offset = 0;
    rows_left = rows_left0;
  }
};

// pipes.cuh:21-25: the contiguous chunk of pipeline row `row`.
__device__ inline MemoryReader read_striped_input(half_t* base, int row, int num_iters, int mblk, int d,
                                                  int64_t total_rows) {
  const int64_t first = (int64_t)row * num_iters * mblk;
  return MemoryReader(base + first * d, (int64_t)mblk * d, d, mblk, total_rows - first);
}

// pipes.cuh:27-31
struct NullReader {
  static constexpr bool kFromQueue = false;
  __device__ void read_release_landed() {}
  __device__ TensorView read_acquire() { return {nullptr, 0, 0}; }
  __device__ void read_release() {}
  __device__ void reset() {}
};

// pipes.cuh:33-43
template <typename QT>
struct QueueReader {
  static constexpr bool kFromQueue = true;
  using Queue = QT;
  Queue* q;
  const QueueCtx* ctx;
  int64_t seq_n = 0;

  __device__ QueueReader(Queue* q_, const QueueCtx* ctx_) : q(q_), ctx(ctx_) {}
  __device__ TensorView read_acquire() {
    int rows = 0;
    auto* e = q->read_wait(seq_n, &rows, *ctx);
    return e->as_view(rows);
  }
  __device__ void read_release() {
    q->read_commit(seq_n, *ctx);
    ++seq_n;
  }
  // read_release once every wave's loads of the tile have landed (vmcnt(0),
  // then a barrier): the commit needs no second wait.
  __device__ void read_release_landed() {
    q->read_commit_landed(seq_n, *ctx);
    ++seq_n;
  }
  __device__ void reset() { seq_n = 0; }
  // Early look at the next tile (for a stage that copies it while working
  // on the current one).  peek_next: thread-level, no wait, before the
  // current tile's read_release.  After that release the peeked tile is the
  // current one: view(rows) is its payload; rows() (thread-level) its rows.
  __device__ bool peek_next() { return q->full_peek(seq_n + 1, *ctx); }
  __device__ int rows() { return q->rows_of(seq_n); }
  __device__ TensorView view(int rows_) { return q->slot(seq_n).data.as_view(rows_); }
};

// pipes.cuh:45-58: worker `seq_off` of `seq_stride` takes sequence numbers
// seq_off, seq_off + seq_stride, ...
template <typename QT>
struct SplitQueueReader {
  static constexpr bool kFromQueue = true;
  using Queue = QT;
  Queue* q;
  const QueueCtx* ctx;
  int64_t seq_n;
  int64_t seq_off;
  int64_t seq_stride;

  __device__ SplitQueueReader(Queue* q_, const QueueCtx* ctx_, int64_t off, int64_t stride)
      : q(q_), ctx(ctx_), seq_n(off), seq_off(off), seq_stride(stride) {}
  __device__ TensorView read_acquire() {
    int rows = 0;
    auto* e = q->read_wait(seq_n, &rows, *ctx);
    return e->as_view(rows);
  }
  __device__ void read_release() {
    q->read_commit(seq_n, *ctx);
    seq_n += seq_stride;
  }
  __device__ void read_release_landed() {
    q->read_commit_landed(seq_n, *ctx);
    seq_n += seq_stride;
  }
  __device__ void reset() { seq_n = seq_off; }
  // As QueueReader's: the next tile of this worker is seq_n + seq_stride.
  __device__ bool peek_next() { return q->full_peek(seq_n + seq_stride, *ctx); }
  __device__ int rows() { return q->rows_of(seq_n); }
  __device__ TensorView view(int rows_) { return q->slot(seq_n).data.as_view(rows_); }
};

// ---------------------------------------------------------------------------
// Writers.  Concept: TensorView write_acquire(int rows); void write_release();
// void reset().  write_acquire takes the number of valid rows being produced.
// ---------------------------------------------------------------------------

// pipes.cuh:60-72
struct MemoryWriter {
  static constexpr bool kReleaseBarrier = false;  // write_release passes no workgroup barrier
  // A memory output is read by no later stage of the launch: stages may store
  // it with the non-temporal policy in whole 128-byte lines, so that it does
  // not take the L2 lines the queues live in.
  static constexpr bool kStreamOut = true;
  half_t* base;
  int64_t stride;
  int tile_stride;
  int64_t offset = 0;
  int rows = 0;

  __device__ MemoryWriter(half_t* base_, int64_t stride_, int tile_stride_)
      : base(base_), stride(stride_), tile_stride(tile_stride_) {}
  __device__ TensorView write_acquire(int rows_) {
    rows = rows_;
    return {base + offset, tile_stride, rows_};
  }
  __device__ void write_release() { offset += stride; }
  __device__ void reset() { offset = 0; }
};

// pipes.cuh:74-84 (the reference resets the queue in the constructor, :80;
// epoch-tagged counters make that unnecessary).  `col0` offsets the view by
// that many columns: with NP > 1 producers, producer j writes its own column
// block of every entry (a layer wider than one GEMM stage, split by columns).
template <typename QT>
struct QueueWriter {
  static constexpr bool kReleaseBarrier = true;  // write_release: every wave's stores complete, then a barrier
  using Queue = QT;
  Queue* q;
  const QueueCtx* ctx;
  int64_t seq_n = 0;
  int rows = 0;
  int col0 = 0;

  __device__ QueueWriter(Queue* q_, const QueueCtx* ctx_, int col0_ = 0) : q(q_), ctx(ctx_), col0(col0_) {}
  __device__ TensorView write_acquire(int rows_) {
    rows = rows_;
    TensorView v = q->write_wait(seq_n, *ctx)->as_view(rows_);
    v.data += col0;
    return v;
  }
  __device__ void write_release() {
    q->write_commit(seq_n, rows, *ctx);
    ++seq_n;
  }
  __device__ void reset() { seq_n = 0; }
};

// pipes.cuh:86-102
template <typename QT>
struct SplitQueueWriter {
  static constexpr bool kReleaseBarrier = true;
  using Queue = QT;
  Queue* q;
  const QueueCtx* ctx;
  int64_t seq_n;
  int64_t seq_off;
  int64_t seq_stride;
  int rows = 0;

  __device__ SplitQueueWriter(Queue* q_, const QueueCtx* ctx_, int64_t off, int64_t stride)
      : q(q_), ctx(ctx_), seq_n(off), seq_off(off), seq_stride(stride) {}
  __device__ TensorView write_acquire(int rows_) {
    rows = rows_;
    return q->write_wait(seq_n, *ctx)->as_view(rows_);
  }
  __device__ void write_release() {
    q->write_commit(seq_n, rows, *ctx);
    seq_n += seq_stride;
  }
  __device__ void reset() { seq_n = seq_off; }
};

// Producer w of np writes rows [w R, (w + 1) R) of every entry, R = the
// entry's rows / np; an entry is full once all np have committed.  The row
// count an entry carries is its whole tile's, which every producer derives
// from the rows left in the input at that entry (rows_left, falling by
// row_step per entry), so the producers store the same value.
template <typename QT>
struct RowSplitQueueWriter {
  static constexpr bool kReleaseBarrier = true;
  using Queue = QT;
  using Entry = typename QT::Item;
  Queue* q;
  const QueueCtx* ctx;
  int64_t seq_n = 0;
  int row0;
  int64_t rows_left, rows_left0, row_step;

  __device__ RowSplitQueueWriter(Queue* q_, const QueueCtx* ctx_, int w, int np, int64_t rows_left_, int64_t row_step_)
      : q(q_), ctx(ctx_), row0(w * (Entry::kRows / np)), rows_left(rows_left_), rows_left0(rows_left_),
        row_step(row_step_) {}
  __device__ TensorView write_acquire(int rows_) {
    TensorView v = q->write_wait(seq_n, *ctx)->as_view(Entry::kRows);
    v.data += (int64_t)row0 * Entry::kCols;
    v.rows = rows_ < 0 ? 0 : rows_;
    return v;
  }
  __device__ void write_release() {
    const int64_t r = rows_left < Entry::kRows ? rows_left : Entry::kRows;
    q->write_commit(seq_n, r > 0 ? (int)r : 0, *ctx);
    ++seq_n;
    rows_left -= row_step;
  }
  __device__ void reset() {
    seq_n = 0;
    rows_left = rows_left0;
  }
};

// pipes.cuh:104-108
struct NullWriter {
  static constexpr bool kReleaseBarrier = false;
  __device__ TensorView write_acquire(int) { return {nullptr, 0, 0}; }
  __device__ void write_release() {}
  __device__ void reset() {}
};

}  // namespace gp
