// Bookkeeping of the library's device scratch, kept free of HIP so the host logic can be
// tested on a CPU with a fake allocator.
//
// One block per (device, stream, host thread) -- the reference keeps its GEMM scratch
// thread_local for the same reason (src/model/asr_gemm.cu:23-43): two threads that share a
// stream must not interleave their launches over one block.  A block that has to grow is
// retired, not freed: work already queued on the stream, or a graph captured over it, may
// still read the old address.  Retired and current blocks of a stream are freed together by
// release_stream(), which the owner of the stream calls once no such work or graph remains
// (stream destruction, decoder destruction).
#pragma once

#include <stddef.h>

#include <map>
#include <mutex>
#include <string>
#include <thread>
#include <tuple>
#include <vector>

namespace orator_hip {

struct WsKey {
  int dev;
  const void* stream;
  std::thread::id tid;
  int slot = 0;  // independent blocks for buffers that are live at the same time
  bool operator<(const WsKey& o) const {
    return std::tie(dev, stream, tid, slot) < std::tie(o.dev, o.stream, o.tid, o.slot);
  }
};

class WorkspacePool {
 public:
  // alloc returns 0 and sets *p on success; sync waits for a stream's queued work.
  using AllocFn = int (*)(void** p, size_t bytes);
  using FreeFn = void (*)(void* p);
  using SyncFn = int (*)(const void* stream);

  WorkspacePool(AllocFn a, FreeFn f, SyncFn s) : alloc_(a), free_(f), sync_(s) {}

  // The caller's block for key k, at least `bytes` long (nullptr and *err on failure).
  void* get(const WsKey& k, size_t bytes, std::string* err) {
    std::lock_guard<std::mutex> lock(mu_);
    Entry& e = map_[k];
    if (e.ptr && e.bytes >= bytes) return e.ptr;
    void* p = nullptr;
    if (alloc_(&p, bytes ? bytes : 1) != 0 || !p) {
      if (err) *err = "workspace allocation of " + std::to_string(bytes) + " bytes failed";
      return nullptr;
    }
    if (e.ptr) e.retired.push_back(e.ptr);  // may still be read by queued work or a graph
    e.ptr = p;
    e.bytes = bytes;
    return p;
  }

  // Frees every block (current and retired, all threads) of `stream` on device `dev` after
  // the stream's queued work has finished.  Returns the sync status (blocks are freed either
  // way: the caller is about to destroy the stream).
  int release_stream(int dev, const void* stream) {
    std::lock_guard<std::mutex> lock(mu_);
    int rc = 0;
    bool synced = false;
    for (auto it = map_.begin(); it != map_.end();) {
      if (it->first.dev != dev || it->first.stream != stream) {
        ++it;
        continue;
      }
      if (!synced) {
        rc = sync_(stream);
        synced = true;
      }
      for (void* p : it->second.retired) free_(p);
      if (it->second.ptr) free_(it->second.ptr);
      it = map_.erase(it);
    }
    return rc;
  }

  // Blocks held (current + retired) -- for tests.
  size_t held_blocks() const {
    std::lock_guard<std::mutex> lock(mu_);
    size_t n = 0;
    for (const auto& kv : map_) n += kv.second.retired.size() + (kv.second.ptr ? 1 : 0);
    return n;
  }

 private:
  struct Entry {
    void* ptr = nullptr;
    size_t bytes = 0;
    std::vector<void*> retired;
  };
  AllocFn alloc_;
  FreeFn free_;
  SyncFn sync_;
  mutable std::mutex mu_;
  std::map<WsKey, Entry> map_;
};

}  // namespace orator_hip
