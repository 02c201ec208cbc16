// Bookkeeping of the library's device scratch, kept free of HIP so the host logic can be
// tested on a CPU with a fake allocator and fake events.
//
// One block per (device, stream, host thread, slot) -- the reference keeps its GEMM scratch
// thread_local for the same reason (src/model/asr_gemm.cu:23-43): two threads that share a
// stream must not interleave their launches over one block.
//
// Bounded growth and release:
//  * a block grows geometrically (at least 1.5x the old size, rounded to 64 KiB), so a
//    stream whose requests creep upwards retires O(log) blocks, not one per call;
//  * a retired block may still be read by work queued on its stream: an event is recorded on
//    the stream at retirement and the block is freed by a later get() once that event has
//    completed (the default stream included);
//  * a block that was handed out while its stream was being captured into a graph may be
//    read by every replay of that graph: it is kept until release_stream(), which the owner
//    of the stream calls once the graphs are destroyed (stream destruction, decoder
//    destruction);
//  * when a host thread exits (thread_exit(), called from a thread_local guard) its blocks
//    are retired the same way, so thread churn does not grow the map.
// A stream the library has used is released with release_stream() before it is destroyed
// (orator_stream_destroy does both), or outlives the threads that used it.
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
  // record: an event after the work queued so far on (dev, stream), or nullptr when none can
  // be recorded now (the stream is being captured, or the call failed); done: 1 once the
  // event has completed, 0 while pending, < 0 on error; destroy frees the event.
  using RecordFn = void* (*)(int dev, const void* stream);
  using DoneFn = int (*)(void* ev);
  using DestroyFn = void (*)(void* ev);

  static constexpr size_t kGrain = size_t{64} << 10;

  WorkspacePool(AllocFn a, FreeFn f, SyncFn s, RecordFn r, DoneFn d, DestroyFn x)
      : alloc_(a), free_(f), sync_(s), record_(r), done_(d), destroy_(x) {}

  // The size a block for `bytes` gets when the current block holds `old` bytes.
  static size_t grown_size(size_t old, size_t bytes) {
    size_t n = bytes > old + old / 2 ? bytes : old + old / 2;
    if (n == 0) n = 1;
    return (n + kGrain - 1) / kGrain * kGrain;
  }

  // The caller's block for key k, at least `bytes` long (nullptr and *err on failure).
  // `capturing`: k.stream is being captured into a graph now.  *fresh (optional) is set when
  // the block was allocated by this call (its contents are undefined).
  void* get(const WsKey& k, size_t bytes, bool capturing, std::string* err,
            bool* fresh = nullptr) {
    std::lock_guard<std::mutex> lock(mu_);
    reap_locked();
    if (fresh) *fresh = false;
    Entry& e = map_[k];
    if (capturing) e.captured = true;
    if (e.ptr && e.bytes >= bytes) return e.ptr;
    const size_t n = grown_size(e.bytes, bytes);
    void* p = nullptr;
    if (alloc_(&p, n) != 0 || !p) {
      if (err) *err = "workspace allocation of " + std::to_string(n) + " bytes failed";
      return nullptr;
    }
    if (e.ptr) retire_locked(k.dev, k.stream, e.ptr, e.bytes, e.captured);
    e.ptr = p;
    e.bytes = n;
    if (fresh) *fresh = true;
    return p;
  }

  // Frees every block (current, retired, pending, all threads) of `stream` on device `dev`
  // after the stream's queued work has finished.  Returns the sync status (blocks are freed
  // either way: the caller is about to destroy the stream).
  int release_stream(int dev, const void* stream) {
    std::lock_guard<std::mutex> lock(mu_);
    int rc = 0;
    bool synced = false;
    auto sync_once = [&] {
      if (!synced) {
        rc = sync_(stream);
        synced = true;
      }
    };
    for (auto it = map_.begin(); it != map_.end();) {
      if (it->first.dev != dev || it->first.stream != stream) {
        ++it;
        continue;
      }
      sync_once();
      if (it->second.ptr) free_(it->second.ptr);
      it = map_.erase(it);
    }
    for (size_t i = 0; i < held_.size();) {
      Held& h = held_[i];
      if (h.dev != dev || h.stream != stream) {
        ++i;
        continue;
      }
      sync_once();
      if (h.ev) destroy_(h.ev);
      free_(h.ptr);
      held_[i] = held_.back();
      held_.pop_back();
    }
    return rc;
  }

  // Retires every block of host thread `tid`, which is exiting: an event is recorded on each
  // block's stream now (the thread's streams are alive while it runs) and the block is freed
  // once it completes, so threads that come and go do not grow the map.
  void thread_exit(std::thread::id tid) {
    std::lock_guard<std::mutex> lock(mu_);
    for (auto it = map_.begin(); it != map_.end();) {
      if (it->first.tid != tid) {
        ++it;
        continue;
      }
      if (it->second.ptr)
        retire_locked(it->first.dev, it->first.stream, it->second.ptr, it->second.bytes,
                      it->second.captured);
      it = map_.erase(it);
    }
  }

  // Frees the retired blocks whose event has completed (also done by every get()).
  void reap() {
    std::lock_guard<std::mutex> lock(mu_);
    reap_locked();
  }

  // Blocks and bytes held (current + retired) and the map's entries -- for tests and
  // diagnostics.
  size_t held_blocks() const {
    std::lock_guard<std::mutex> lock(mu_);
    size_t n = held_.size();
    for (const auto& kv : map_) n += kv.second.ptr ? 1 : 0;
    return n;
  }
  size_t held_bytes() const {
    std::lock_guard<std::mutex> lock(mu_);
    size_t n = 0;
    for (const auto& kv : map_) n += kv.second.bytes;
    for (const auto& h : held_) n += h.bytes;
    return n;
  }
  size_t entries() const {
    std::lock_guard<std::mutex> lock(mu_);
    return map_.size();
  }

 private:
  struct Entry {
    void* ptr = nullptr;
    size_t bytes = 0;
    bool captured = false;  // handed out during a capture: kept until release_stream
  };
  struct Held {
    int dev;
    const void* stream;
    void* ptr;
    void* ev;          // completion event of the work queued before retirement
    bool captured;     // kept until release_stream
    bool needs_event;  // retired without an event yet (record failed or the stream was capturing)
    size_t bytes;
  };

  void retire_locked(int dev, const void* stream, void* ptr, size_t bytes, bool captured) {
    Held h{dev, stream, ptr, nullptr, captured, false, bytes};
    if (!captured) {
      h.ev = record_(dev, stream);
      h.needs_event = h.ev == nullptr;
    }
    held_.push_back(h);
  }

  void reap_locked() {
    for (size_t i = 0; i < held_.size();) {
      Held& h = held_[i];
      if (h.captured) {
        ++i;
        continue;
      }
      if (h.needs_event) {
        h.ev = record_(h.dev, h.stream);
        h.needs_event = h.ev == nullptr;
        ++i;
        continue;
      }
      const int d = done_(h.ev);
      if (d == 0) {
        ++i;
        continue;
      }
      if (d < 0) {  // the event failed: fall back to waiting for the stream
        if (sync_(h.stream) != 0) {
          ++i;
          continue;
        }
      }
      destroy_(h.ev);
      free_(h.ptr);
      held_[i] = held_.back();
      held_.pop_back();
    }
  }

  AllocFn alloc_;
  FreeFn free_;
  SyncFn sync_;
  RecordFn record_;
  DoneFn done_;
  DestroyFn destroy_;
  mutable std::mutex mu_;
  std::map<WsKey, Entry> map_;
  std::vector<Held> held_;
};

}  // namespace orator_hip
