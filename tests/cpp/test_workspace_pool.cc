// CPU test of the workspace bookkeeping (orator_amd/csrc/workspace_pool.hpp) with a fake
// allocator and fake stream events: growth is geometric and retires the old block; a retired
// block is freed once the event recorded at its retirement completes, and never earlier; a
// block handed out during a capture is kept until release_stream; threads get their own
// blocks and give them back when they exit; release frees exactly the stream's blocks.
#include <cstdio>
#include <cstdlib>
#include <map>
#include <set>
#include <thread>
#include <vector>

#include "../../orator_amd/csrc/workspace_pool.hpp"

using orator_hip::WorkspacePool;
using orator_hip::WsKey;

static std::set<void*> g_live;
static int g_syncs = 0;
static int g_allocs = 0;
// fake events: an event completes once its stream's "completed work counter" passes it
static std::map<const void*, int> g_queued;     // work items queued per stream
static std::map<const void*, int> g_completed;  // work items completed per stream
struct FakeEvent {
  const void* stream;
  int at;
};
static std::set<FakeEvent*> g_events;
static std::set<const void*> g_capturing;

static int fake_alloc(void** p, size_t bytes) {
  *p = std::malloc(bytes);
  g_live.insert(*p);
  ++g_allocs;
  return 0;
}
static void fake_free(void* p) {
  if (!g_live.erase(p)) {
    std::fprintf(stderr, "double or foreign free\n");
    std::exit(2);
  }
  std::free(p);
}
static int fake_sync(const void* s) {
  ++g_syncs;
  g_completed[s] = g_queued[s];
  return 0;
}
static void* fake_record(int, const void* s) {
  if (g_capturing.count(s)) return nullptr;
  auto* e = new FakeEvent{s, g_queued[s]};
  g_events.insert(e);
  return e;
}
static int fake_done(void* ev) {
  auto* e = static_cast<FakeEvent*>(ev);
  return g_completed[e->stream] >= e->at ? 1 : 0;
}
static void fake_destroy(void* ev) {
  auto* e = static_cast<FakeEvent*>(ev);
  if (!g_events.erase(e)) {
    std::fprintf(stderr, "double or foreign event destroy\n");
    std::exit(2);
  }
  delete e;
}

#define CHECK(c)                                                          \
  do {                                                                    \
    if (!(c)) {                                                           \
      std::fprintf(stderr, "%s:%d: CHECK(%s)\n", __FILE__, __LINE__, #c); \
      return 1;                                                           \
    }                                                                     \
  } while (0)

int main() {
  WorkspacePool pool(fake_alloc, fake_free, fake_sync, fake_record, fake_done, fake_destroy);
  const void* s1 = reinterpret_cast<const void*>(0x1000);
  const void* s2 = reinterpret_cast<const void*>(0x2000);
  const WsKey a{0, s1, std::this_thread::get_id()};
  void* p1 = pool.get(a, 100, false, nullptr);
  CHECK(p1 && pool.get(a, 50, false, nullptr) == p1);  // fits: same block
  g_queued[s1] = 1;                                    // work queued on p1
  void* p2 = pool.get(a, 1000000, false, nullptr);     // grows: new block, old one retired
  CHECK(p2 && p2 != p1 && g_live.count(p1) == 1 && pool.held_blocks() == 2);
  CHECK(g_syncs == 0);  // growth never waits on the stream
  // the retired block survives until the work queued before its retirement completes
  pool.reap();
  CHECK(g_live.count(p1) == 1);
  g_completed[s1] = 1;
  pool.reap();
  CHECK(g_live.count(p1) == 0 && pool.held_blocks() == 1 && g_events.empty());

  // geometric growth: 1000 requests creeping up by 4 KiB each retire O(log) blocks, and the
  // retired ones are freed as their work completes
  {
    const int allocs0 = g_allocs;
    size_t req = 1000000;
    for (int i = 0; i < 1000; ++i) {
      req += 4096;
      g_queued[s1] += 1;
      CHECK(pool.get(a, req, false, nullptr));
      g_completed[s1] = g_queued[s1] - 1;  // all but the latest launch finished
    }
    const int grown = g_allocs - allocs0;
    CHECK(grown > 0 && grown <= 8);  // 1.0 MB -> 5.1 MB at >= 1.5x per growth
    pool.reap();
    CHECK(pool.held_blocks() <= 2);
    g_completed[s1] = g_queued[s1];
    pool.reap();
    CHECK(pool.held_blocks() == 1);
    CHECK(WorkspacePool::grown_size(0, 1) == WorkspacePool::kGrain);
    CHECK(WorkspacePool::grown_size(1 << 20, (1 << 20) + 1) == (3u << 19));
  }

  // a block handed out while the stream is capturing is kept until release_stream, even
  // after the stream's work completes
  const WsKey c{0, s2, std::this_thread::get_id()};
  void* pc = pool.get(c, 4096, false, nullptr);  // reserved before the capture
  g_capturing.insert(s2);
  CHECK(pool.get(c, 2048, true, nullptr) == pc);  // used during the capture
  g_capturing.erase(s2);
  void* pc2 = pool.get(c, 1 << 20, false, nullptr);  // grows after the capture
  CHECK(pc2 && pc2 != pc);
  g_completed[s2] = g_queued[s2] = 5;
  pool.reap();
  CHECK(g_live.count(pc) == 1);  // a graph may still replay over it

  // a block retired while its stream is capturing gets its event once the capture is over
  {
    const WsKey d{0, s1, std::this_thread::get_id(), 3};
    void* q1 = pool.get(d, 100, false, nullptr);
    g_queued[s1] += 1;
    g_capturing.insert(s1);
    // growth under capture: the entry is marked captured, so the old block is kept until
    // release_stream as well
    void* q2 = pool.get(d, 1 << 20, true, nullptr);
    CHECK(q2 && q2 != q1 && g_live.count(q1) == 1);
    g_capturing.erase(s1);
    g_completed[s1] = g_queued[s1];
    pool.reap();
    CHECK(g_live.count(q1) == 1);
  }

  // threads: each gets its own block; an exiting thread's blocks are retired with an event
  // and freed once that work completes, so thread churn does not grow the map
  {
    const size_t entries0 = pool.entries();
    for (int i = 0; i < 50; ++i) {
      void* pt = nullptr;
      std::thread th([&] {
        pt = pool.get(WsKey{0, s1, std::this_thread::get_id()}, 100, false, nullptr);
        g_queued[s1] += 1;
        pool.thread_exit(std::this_thread::get_id());  // what the thread guard does
      });
      th.join();
      CHECK(pt && g_live.count(pt) == 1);
      g_completed[s1] = g_queued[s1];
      pool.reap();
      CHECK(g_live.count(pt) == 0);
    }
    CHECK(pool.entries() == entries0);
  }

  // another slot of the same stream and thread is a separate block; `fresh` tells a new block
  // (whose contents the caller must initialise) from a reused one
  bool fresh = false;
  void* ps = pool.get(WsKey{0, s1, std::this_thread::get_id(), 1}, 100, false, nullptr, &fresh);
  CHECK(ps && ps != p2 && fresh);
  CHECK(pool.get(WsKey{0, s1, std::this_thread::get_id(), 1}, 64, false, nullptr, &fresh) == ps &&
        !fresh);
  // another device is separate
  void* r = pool.get(WsKey{1, s1, std::this_thread::get_id()}, 10, false, nullptr);
  CHECK(r);
  // release of (dev 0, s1): one sync, frees every block of that stream only
  const int syncs = g_syncs;
  CHECK(pool.release_stream(0, s1) == 0 && g_syncs == syncs + 1);
  CHECK(!g_live.count(ps) && g_live.count(r) && g_live.count(pc) && g_live.count(pc2));
  CHECK(pool.release_stream(0, s2) == 0 && !g_live.count(pc) && !g_live.count(pc2));
  CHECK(pool.release_stream(1, s1) == 0);
  CHECK(pool.held_blocks() == 0 && g_live.empty() && g_events.empty());
  // releasing a stream with no blocks does not sync
  const int syncs2 = g_syncs;
  CHECK(pool.release_stream(0, s1) == 0 && g_syncs == syncs2);
  std::printf("workspace pool OK\n");
  return 0;
}
