// CPU test of the workspace bookkeeping (orator_amd/csrc/workspace_pool.hpp) with a fake
// allocator: growth retires instead of freeing, threads get their own blocks, release frees
// exactly the stream's blocks after one sync.
#include <cstdio>
#include <cstdlib>
#include <set>
#include <thread>

#include "../../orator_amd/csrc/workspace_pool.hpp"

using orator_hip::WorkspacePool;
using orator_hip::WsKey;

static std::set<void*> g_live;
static int g_syncs = 0;
static int fake_alloc(void** p, size_t bytes) {
  *p = std::malloc(bytes);
  g_live.insert(*p);
  return 0;
}
static void fake_free(void* p) {
  if (!g_live.erase(p)) {
    std::fprintf(stderr, "double or foreign free\n");
    std::exit(2);
  }
  std::free(p);
}
static int fake_sync(const void*) {
  ++g_syncs;
  return 0;
}

#define CHECK(c)                                                   \
  do {                                                             \
    if (!(c)) {                                                    \
      std::fprintf(stderr, "%s:%d: CHECK(%s)\n", __FILE__, __LINE__, #c); \
      return 1;                                                    \
    }                                                              \
  } while (0)

int main() {
  WorkspacePool pool(fake_alloc, fake_free, fake_sync);
  const void* s1 = reinterpret_cast<const void*>(0x1000);
  const void* s2 = reinterpret_cast<const void*>(0x2000);
  const WsKey a{0, s1, std::this_thread::get_id()};
  void* p1 = pool.get(a, 100, nullptr);
  CHECK(p1 && pool.get(a, 50, nullptr) == p1);  // fits: same block
  void* p2 = pool.get(a, 1000, nullptr);         // grows: new block, old one kept alive
  CHECK(p2 && p2 != p1 && g_live.count(p1) == 1 && pool.held_blocks() == 2);
  CHECK(g_syncs == 0);                           // growth never waits on the stream
  // another thread on the same stream gets its own block
  void* pt = nullptr;
  std::thread th([&] { pt = pool.get(WsKey{0, s1, std::this_thread::get_id()}, 100, nullptr); });
  th.join();
  CHECK(pt && pt != p1 && pt != p2 && pool.held_blocks() == 3);
  // another slot of the same stream and thread is a separate block
  void* ps = pool.get(WsKey{0, s1, std::this_thread::get_id(), 1}, 100, nullptr);
  CHECK(ps && ps != p2 && pool.held_blocks() == 4);
  // another stream and another device are separate
  void* q = pool.get(WsKey{0, s2, std::this_thread::get_id()}, 10, nullptr);
  void* r = pool.get(WsKey{1, s1, std::this_thread::get_id()}, 10, nullptr);
  CHECK(q && r && pool.held_blocks() == 6);
  // release of (dev 0, s1): one sync, frees p1, p2, the slot-1 block and the other thread's
  // block only
  CHECK(pool.release_stream(0, s1) == 0 && g_syncs == 1);
  CHECK(!g_live.count(p1) && !g_live.count(p2) && !g_live.count(pt) && !g_live.count(ps));
  CHECK(g_live.count(q) && g_live.count(r) && pool.held_blocks() == 2);
  // a later stream with the same handle value starts fresh
  void* p3 = pool.get(a, 10, nullptr);
  CHECK(p3 && pool.held_blocks() == 3);
  CHECK(pool.release_stream(0, s1) == 0 && pool.release_stream(0, s2) == 0 &&
        pool.release_stream(1, s1) == 0 && pool.held_blocks() == 0 && g_live.empty());
  // releasing a stream with no blocks does not sync
  const int syncs = g_syncs;
  CHECK(pool.release_stream(0, s1) == 0 && g_syncs == syncs);
  std::printf("workspace pool OK\n");
  return 0;
}
