// Host-thread model of the ring-queue protocol of gpu-pipes_amd/csrc/pipes.hpp
// and pipeline.hpp -- TEST INFRASTRUCTURE.
//
// Each workgroup of a pipelined kernel is a std::thread here; the queue
// counters are std::atomic<uint64_t> with the same (epoch << 32) | count
// encoding, the same epoch lift on a slot's first round, the same wait
// targets (producers wait for empty >= round * NC, consumers for
// full >= (round + 1) * NP), the same split round robin (worker w of S takes
// sequence numbers w, w + S, ...), the same bounded waits with a shared
// epoch-tagged error word, and the same row count carried with each entry.
// The GPU's ordering (stores complete, then the commit atomic; the acquire
// fence after the observed count) is expressed with release / acquire
// atomics, so ThreadSanitizer sees a data race if a payload could be read
// before it was written or overwritten before it was read.
//
// The reference's protocol (common/mpmcq.cuh:10-115, common/pipes.cuh:33-102)
// resets counters in the writer's constructor and has no fences; this model
// checks the redesigned protocol, not the reference's.
//
// Scenarios (each run over several launches on the same queue memory, with
// garbage from older epochs left in it): 1:1, one producer / two consumers,
// split / merge through three workers, four producers writing column blocks
// of one entry, partial last tiles, and a producer that stops early (the
// consumers' bounded waits must end the launch with the error set, and the
// consumers must not count a tile that never came).  Every tile must arrive
// exactly once, in order, with its payload and row count intact.
//
// Build: g++ -std=c++17 -O1 -g -pthread [-fsanitize=thread] queue_model.cpp
// Exit status 0 and "queue model: all scenarios passed" on success.
#include <atomic>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <functional>
#include <thread>
#include <vector>

namespace qm {

// Planted protocol mistakes (argv[1]), each of which the checks must catch:
//   1 the epoch lift is skipped, 2 a producer waits one round short,
//   3 commits are relaxed (no release; caught by ThreadSanitizer),
//   4 a split worker uses the wrong stride, 5 a consumer commits before it
//   has read the payload.
int g_mutant = 0;
long g_limit = 1L << 26;  // poll bound of the scenarios that must not time out

struct Ctx {
  uint32_t epoch;
  std::atomic<uint64_t>* err;
  long limit;  // polls before a wait gives up
};

uint32_t qcount(uint64_t v, uint32_t epoch) { return (uint32_t)(v >> 32) == epoch ? (uint32_t)v : 0u; }

void atomic_max(std::atomic<uint64_t>& a, uint64_t v) {
  uint64_t cur = a.load(std::memory_order_relaxed);
  while (cur < v && !a.compare_exchange_weak(cur, v, std::memory_order_relaxed)) {
  }
}

bool aborted(const Ctx& c) {
  const uint64_t v = c.err->load(std::memory_order_relaxed);
  return (uint32_t)(v >> 32) == c.epoch && (uint32_t)v != 0;
}

void fail(const Ctx& c, unsigned bits) {
  atomic_max(*c.err, (uint64_t)c.epoch << 32);
  c.err->fetch_or(bits, std::memory_order_relaxed);
}

// pipes.hpp qcommit: the first round of a slot lifts an older epoch's value.
void qcommit(std::atomic<uint64_t>& c, uint32_t epoch, bool first) {
  if (first && g_mutant != 1) atomic_max(c, (uint64_t)epoch << 32);
  c.fetch_add(1, g_mutant == 3 ? std::memory_order_relaxed : std::memory_order_release);
}

// pipes.hpp qwait: bounded; false if this or another wait of the launch gave up.
bool qwait(std::atomic<uint64_t>& c, uint32_t target, const Ctx& ctx) {
  for (long it = 0;; ++it) {
    if (qcount(c.load(std::memory_order_acquire), ctx.epoch) >= target) return true;
    if (aborted(ctx)) return false;
    if (it >= ctx.limit) {
      fail(ctx, 1);
      return false;
    }
    std::this_thread::yield();
  }
}

template <int ROWS, int COLS>
struct Entry {
  uint32_t buf[ROWS][COLS];
};

template <typename E, int N, int NP = 1, int NC = 1>
struct RingQueue {
  struct Slot {
    std::atomic<uint64_t> full{0}, empty{0};
    std::atomic<int> rows{0};
    E data;
  } slots[N];

  Slot& slot(int64_t seq) { return slots[seq % N]; }
  E* write_wait(int64_t seq, const Ctx& ctx) {
    const int64_t round = g_mutant == 2 ? (seq / N > 0 ? seq / N - 1 : 0) : seq / N;
    qwait(slot(seq).empty, (uint32_t)round * NC, ctx);
    return &slot(seq).data;
  }
  void write_commit(int64_t seq, int rows, const Ctx& ctx) {
    slot(seq).rows.store(rows, std::memory_order_relaxed);
    qcommit(slot(seq).full, ctx.epoch, seq < N);
  }
  E* read_wait(int64_t seq, int* rows, const Ctx& ctx) {
    const bool ok = qwait(slot(seq).full, (uint32_t)(seq / N + 1) * NP, ctx);
    *rows = ok ? slot(seq).rows.load(std::memory_order_relaxed) : 0;
    return &slot(seq).data;
  }
  void read_commit(int64_t seq, const Ctx& ctx) { qcommit(slot(seq).empty, ctx.epoch, seq < N); }
};

// Fill the garbage an older launch leaves behind: counters of epoch e-1 with
// large counts, error word of an older epoch with bits set.
template <typename Q>
void dirty(Q& q, uint32_t old_epoch) {
  for (auto& s : q.slots) {
    s.full.store(((uint64_t)old_epoch << 32) | 977u);
    s.empty.store(((uint64_t)old_epoch << 32) | 1201u);
    s.rows.store(12345);
  }
}

uint32_t tag(int64_t tile, int r, int c) { return (uint32_t)(tile * 131071 + r * 257 + c + 1); }

std::atomic<int> g_errors{0};
#define CHECK(cond, ...)                                   \
  do {                                                     \
    if (!(cond)) {                                         \
      if (g_errors < 20) {                                 \
        std::fprintf(stderr, "FAILED %s: ", #cond);        \
        std::fprintf(stderr, __VA_ARGS__);                 \
        std::fprintf(stderr, "\n");                        \
      }                                                    \
      ++g_errors;                                          \
    }                                                      \
  } while (0)

constexpr int R = 4, C = 8;  // a small tile: 4 rows x 8 columns
using E = Entry<R, C>;

int rows_of(int64_t tile, int64_t M) {
  const int64_t left = M - tile * R;
  return left <= 0 ? 0 : (left < R ? (int)left : R);
}

// Producer: T tiles, sequence numbers first, first + stride, ...
template <typename Q>
void produce(Q& q, const Ctx& ctx, int64_t M, int64_t T, int first, int stride, int col0, int ncols) {
  for (int64_t seq = first; seq < T; seq += stride) {
    E* e = q.write_wait(seq, ctx);
    const int rows = rows_of(seq, M);
    for (int r = 0; r < rows; ++r)
      for (int c = col0; c < col0 + ncols; ++c) e->buf[r][c] = tag(seq, r, c);
    q.write_commit(seq, rows, ctx);
  }
}

// Consumer: checks every tile it is given and records it in `seen`.
template <typename Q>
void consume(Q& q, const Ctx& ctx, int64_t M, int64_t T, int first, int stride, std::vector<int>& seen,
             bool expect_all) {
  for (int64_t seq = first; seq < T; seq += stride) {
    int rows = 0;
    E* e = q.read_wait(seq, &rows, ctx);
    if (g_mutant == 5) q.read_commit(seq, ctx);
    if (rows > 0) {
      CHECK(rows == rows_of(seq, M), "tile %lld rows %d, expected %d", (long long)seq, rows, rows_of(seq, M));
      bool ok = true;
      for (int r = 0; r < rows; ++r)
        for (int c = 0; c < C; ++c) ok = ok && e->buf[r][c] == tag(seq, r, c);
      CHECK(ok, "tile %lld payload corrupt", (long long)seq);
      seen[seq] += 1;
    } else {
      CHECK(!expect_all || aborted(ctx), "tile %lld arrived empty without an abort", (long long)seq);
    }
    if (g_mutant != 5) q.read_commit(seq, ctx);
  }
}

void run_threads(std::vector<std::function<void()>> fns) {
  std::vector<std::thread> th;
  for (auto& f : fns) th.emplace_back(f);
  for (auto& t : th) t.join();
}

void check_once(const std::vector<int>& seen, int64_t T, int times, const char* what) {
  for (int64_t t = 0; t < T; ++t) CHECK(seen[t] == times, "%s: tile %lld seen %d times", what, (long long)t, seen[t]);
}

// 1:1 pipe (QueueReader / QueueWriter)
void scenario_ident(uint32_t epoch, std::atomic<uint64_t>& err, int64_t M) {
  static RingQueue<E, 2> q;
  if (epoch == 1) dirty(q, 0);
  const Ctx ctx{epoch, &err, g_limit};
  const int64_t T = (M + R - 1) / R;
  std::vector<int> seen(T, 0);
  run_threads({[&] { produce(q, ctx, M, T, 0, 1, 0, C); }, [&] { consume(q, ctx, M, T, 0, 1, seen, true); }});
  check_once(seen, T, 1, "ident");
  CHECK(!aborted(ctx), "ident aborted");
}

// one producer, two consumers (MpmcRingQueue<E, N, 1, 2>)
void scenario_broadcast(uint32_t epoch, std::atomic<uint64_t>& err, int64_t M) {
  static RingQueue<E, 3, 1, 2> q;
  if (epoch == 1) dirty(q, 0);
  const Ctx ctx{epoch, &err, g_limit};
  const int64_t T = (M + R - 1) / R;
  std::vector<int> s1(T, 0), s2(T, 0);
  run_threads({[&] { produce(q, ctx, M, T, 0, 1, 0, C); }, [&] { consume(q, ctx, M, T, 0, 1, s1, true); },
               [&] { consume(q, ctx, M, T, 0, 1, s2, true); }});
  check_once(s1, T, 1, "broadcast consumer 1");
  check_once(s2, T, 1, "broadcast consumer 2");
}

// split / merge: 3 workers read q0 round robin (SplitQueueReader) and write q1
// round robin (SplitQueueWriter); one reader takes q1 in sequence order.
void scenario_split(uint32_t epoch, std::atomic<uint64_t>& err, int64_t M) {
  constexpr int S = 3;
  static RingQueue<E, S + 1> q0, q1;
  if (epoch == 1) {
    dirty(q0, 0);
    dirty(q1, 0);
  }
  const Ctx ctx{epoch, &err, g_limit};
  const int64_t T = (M + R - 1) / R;
  std::vector<int> seen(T, 0);
  std::vector<std::function<void()>> fns;
  fns.push_back([&] { produce(q0, ctx, M, T, 0, 1, 0, C); });
  const int stride = g_mutant == 4 ? S - 1 : S;
  for (int w = 0; w < S; ++w)
    fns.push_back([&, w] {
      for (int64_t seq = w; seq < T; seq += stride) {
        int rows = 0;
        E* in = q0.read_wait(seq, &rows, ctx);
        E* out = q1.write_wait(seq, ctx);
        for (int r = 0; r < rows; ++r)
          for (int c = 0; c < C; ++c) out->buf[r][c] = in->buf[r][c];
        q0.read_commit(seq, ctx);
        q1.write_commit(seq, rows, ctx);
      }
    });
  fns.push_back([&] { consume(q1, ctx, M, T, 0, 1, seen, true); });
  run_threads(fns);
  check_once(seen, T, 1, "split/merge");
}

// four producers write the column blocks of each entry (NP = 4), one consumer
void scenario_columns(uint32_t epoch, std::atomic<uint64_t>& err, int64_t M) {
  constexpr int NP = 4;
  static RingQueue<E, 2, NP, 1> q;
  if (epoch == 1) dirty(q, 0);
  const Ctx ctx{epoch, &err, g_limit};
  const int64_t T = (M + R - 1) / R;
  std::vector<int> seen(T, 0);
  std::vector<std::function<void()>> fns;
  for (int j = 0; j < NP; ++j) fns.push_back([&, j] { produce(q, ctx, M, T, 0, 1, j * (C / NP), C / NP); });
  fns.push_back([&] { consume(q, ctx, M, T, 0, 1, seen, true); });
  run_threads(fns);
  check_once(seen, T, 1, "column blocks");
}

// two producers write the row halves of each entry of a one-slot queue
// (RowSplitQueueWriter: NP = 2), both committing the whole tile's row count;
// one consumer.  Mutant 6: each producer commits only its own half's rows.
void scenario_rows(uint32_t epoch, std::atomic<uint64_t>& err, int64_t M) {
  constexpr int NP = 2, RH = R / NP;
  static RingQueue<E, 1, NP, 1> q;
  if (epoch == 1) dirty(q, 0);
  const Ctx ctx{epoch, &err, g_limit};
  const int64_t T = (M + R - 1) / R;
  std::vector<int> seen(T, 0);
  std::vector<std::function<void()>> fns;
  for (int j = 0; j < NP; ++j)
    fns.push_back([&, j] {
      for (int64_t seq = 0; seq < T; ++seq) {
        E* e = q.write_wait(seq, ctx);
        const int rows = rows_of(seq, M);
        const int mine = rows - j * RH < 0 ? 0 : (rows - j * RH > RH ? RH : rows - j * RH);
        for (int r = j * RH; r < j * RH + mine; ++r)
          for (int c = 0; c < C; ++c) e->buf[r][c] = tag(seq, r, c);
        q.write_commit(seq, g_mutant == 6 ? mine : rows, ctx);
      }
    });
  fns.push_back([&] { consume(q, ctx, M, T, 0, 1, seen, true); });
  run_threads(fns);
  check_once(seen, T, 1, "row halves");
}

// the producer stops after `stop` tiles: the consumer's bounded wait must end
// the launch with the error set; no tile that never came may be counted.
void scenario_stuck(uint32_t epoch, std::atomic<uint64_t>& err, int64_t M, int64_t stop) {
  static RingQueue<E, 2> q;
  if (epoch == 1) dirty(q, 0);
  const Ctx ctx{epoch, &err, 20000};
  const int64_t T = (M + R - 1) / R;
  std::vector<int> seen(T, 0);
  run_threads({[&] { produce(q, ctx, M, stop, 0, 1, 0, C); }, [&] { consume(q, ctx, M, T, 0, 1, seen, false); }});
  CHECK(aborted(ctx), "stuck pipeline not reported");
  for (int64_t t = 0; t < T; ++t)
    CHECK(seen[t] == (t < stop ? 1 : 0), "stuck: tile %lld seen %d times", (long long)t, seen[t]);
}

}  // namespace qm

int main(int argc, char** argv) {
  using namespace qm;
  if (argc > 1) g_mutant = std::atoi(argv[1]);
  if (g_mutant) g_limit = 200000;  // a broken protocol may stall: give up sooner
  std::atomic<uint64_t> err{((uint64_t)0 << 32) | 7u};  // an older launch's error bits
  const int64_t sizes[] = {1, R - 1, R, R + 1, 37 * R + 3, 2000 * R};
  uint32_t epoch = 1;
  for (int rep = 0; rep < 2; ++rep) {
    for (int64_t M : sizes) {
      scenario_ident(epoch++, err, M);
      scenario_broadcast(epoch++, err, M);
      scenario_split(epoch++, err, M);
      scenario_columns(epoch++, err, M);
      scenario_rows(epoch++, err, M);
    }
  }
  // a timed-out launch, then a clean launch on the same queues and error word
  scenario_stuck(epoch++, err, 50 * R, 17);
  scenario_ident(epoch++, err, 300 * R + 1);
  {
    const Ctx ctx{epoch - 1, &err, 1};
    CHECK(!aborted(ctx), "an older launch's error leaked into a clean launch");
  }
  if (g_errors.load()) {
    std::fprintf(stderr, "queue model: %d failures\n", g_errors.load());
    return 1;
  }
  std::printf("queue model: all scenarios passed (%u launches)\n", epoch - 1);
  return 0;
}
