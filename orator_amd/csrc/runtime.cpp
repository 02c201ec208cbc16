// Library runtime: error reporting, the per-(device, stream, thread) workspace and the small
// device-plumbing surface of the C ABI (allocation, copies, streams, events).
#include <hip/hip_runtime.h>
#include <sys/syscall.h>
#include <unistd.h>

#include <cmath>
#include <atomic>
#include <thread>
#include <string>
#include <utility>

#include "internal.hpp"
#include "workspace_pool.hpp"

namespace orator_hip {

namespace {
thread_local std::string g_last_error;

int ws_alloc(void** p, size_t bytes) { return hipMalloc(p, bytes) == hipSuccess ? 0 : 1; }
void ws_free(void* p) { (void)hipFree(p); }
int ws_sync(const void* stream) {
  return hipStreamSynchronize(static_cast<hipStream_t>(const_cast<void*>(stream))) == hipSuccess
             ? 0
             : 1;
}
// true while `stream` is being captured (or when that cannot be told: then nothing recorded
// on it is trusted as a completion marker)
bool ws_capturing(hipStream_t stream) {
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(stream, &st) != hipSuccess) {
    (void)hipGetLastError();
    return true;
  }
  return st != hipStreamCaptureStatusNone;
}
void* ws_record(int dev, const void* stream_p) {
  hipStream_t stream = static_cast<hipStream_t>(const_cast<void*>(stream_p));
  int cur = -1;
  if (hipGetDevice(&cur) != hipSuccess) return nullptr;
  if (cur != dev && hipSetDevice(dev) != hipSuccess) return nullptr;
  hipEvent_t ev = nullptr;
  if (!ws_capturing(stream) &&
      hipEventCreateWithFlags(&ev, hipEventDisableTiming) == hipSuccess &&
      hipEventRecord(ev, stream) != hipSuccess) {
    (void)hipEventDestroy(ev);
    ev = nullptr;
  }
  if (cur != dev) (void)hipSetDevice(cur);
  (void)hipGetLastError();
  return ev;
}
int ws_done(void* ev) {
  const hipError_t e = hipEventQuery(static_cast<hipEvent_t>(ev));
  if (e == hipSuccess) return 1;
  (void)hipGetLastError();
  return e == hipErrorNotReady ? 0 : -1;
}
void ws_destroy(void* ev) { (void)hipEventDestroy(static_cast<hipEvent_t>(ev)); }
WorkspacePool& ws_pool() {
  // never destroyed: blocks may be in use until the process ends
  static WorkspacePool* pool =
      new WorkspacePool(ws_alloc, ws_free, ws_sync, ws_record, ws_done, ws_destroy);
  return *pool;
}
// Retires a worker thread's blocks when it exits.  The process's main thread skips this: its
// thread_local objects are destroyed at process exit, where no device call is made.
struct WsThreadGuard {
  bool armed = false;
  ~WsThreadGuard() {
    if (armed && static_cast<pid_t>(syscall(SYS_gettid)) != getpid())
      ws_pool().thread_exit(std::this_thread::get_id());
  }
};
thread_local WsThreadGuard g_ws_guard;
thread_local hipEvent_t g_ev_start = nullptr, g_ev_split = nullptr, g_ev_stop = nullptr;
}  // namespace

void take_timing_events(hipEvent_t* start, hipEvent_t* split_end, hipEvent_t* stop) {
  *start = g_ev_start;
  *split_end = g_ev_split;
  *stop = g_ev_stop;
  g_ev_start = g_ev_split = g_ev_stop = nullptr;
}

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

int check_hip(hipError_t e, const char* what) {
  if (e == hipSuccess) return ORATOR_OK;
  return fail(ORATOR_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

int check_launch(const char* what) { return check_hip(hipGetLastError(), what); }

int device_cu_count() {
  static std::atomic<int> cached[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 0;
  if (dev < 64 && cached[dev].load(std::memory_order_relaxed) > 0) return cached[dev];
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) n = 0;
  if (dev < 64 && n > 0) cached[dev].store(n, std::memory_order_relaxed);
  return n;
}

void* workspace(hipStream_t stream, size_t bytes, int slot, bool* fresh) {
  int dev = 0;
  if (check_hip(hipGetDevice(&dev), "hipGetDevice") != ORATOR_OK) return nullptr;
  std::string err;
  g_ws_guard.armed = true;
  void* p = ws_pool().get(WsKey{dev, stream, std::this_thread::get_id(), slot}, bytes,
                          ws_capturing(stream), &err, fresh);
  if (!p) (void)fail(ORATOR_ERR_HIP, err);
  return p;
}

int workspace_release(hipStream_t stream) {
  int dev = 0;
  if (int rc = check_hip(hipGetDevice(&dev), "hipGetDevice")) return rc;
  return ws_pool().release_stream(dev, stream) ? fail(ORATOR_ERR_HIP, "workspace release: sync")
                                               : ORATOR_OK;
}

}  // namespace orator_hip

using orator_hip::check_hip;
using orator_hip::fail;

extern "C" {

const char* orator_last_error(void) { return orator_hip::g_last_error.c_str(); }

int orator_version(void) { return 1; }

int orator_device_count(int* count) {
  if (!count) return fail(ORATOR_ERR_INVALID, "device_count: null");
  return check_hip(hipGetDeviceCount(count), "hipGetDeviceCount");
}

int orator_set_device(int device) { return check_hip(hipSetDevice(device), "hipSetDevice"); }

int orator_device_name(char* buf, int len) {
  if (!buf || len <= 0) return fail(ORATOR_ERR_INVALID, "device_name: bad buffer");
  int dev = 0;
  int rc = check_hip(hipGetDevice(&dev), "hipGetDevice");
  if (rc) return rc;
  hipDeviceProp_t prop;
  rc = check_hip(hipGetDeviceProperties(&prop, dev), "hipGetDeviceProperties");
  if (rc) return rc;
  std::string name = std::string(prop.name) + " (" + prop.gcnArchName + ", " +
                     std::to_string(prop.multiProcessorCount) + " CUs)";
  snprintf(buf, static_cast<size_t>(len), "%s", name.c_str());
  return ORATOR_OK;
}

int orator_malloc(void** ptr, size_t bytes) {
  if (!ptr) return fail(ORATOR_ERR_INVALID, "malloc: null");
  return check_hip(hipMalloc(ptr, bytes ? bytes : 1), "hipMalloc");
}

int orator_free(void* ptr) { return check_hip(hipFree(ptr), "hipFree"); }

int orator_memcpy_htod(void* dst, const void* src, size_t bytes) {
  return check_hip(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice), "hipMemcpy H2D");
}

int orator_memcpy_dtoh(void* dst, const void* src, size_t bytes) {
  return check_hip(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost), "hipMemcpy D2H");
}

int orator_memcpy_dtod(void* dst, const void* src, size_t bytes, void* stream) {
  return check_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice,
                                  static_cast<hipStream_t>(stream)),
                   "hipMemcpyAsync D2D");
}

int orator_memset(void* ptr, int value, size_t bytes, void* stream) {
  return check_hip(hipMemsetAsync(ptr, value, bytes, static_cast<hipStream_t>(stream)),
                   "hipMemsetAsync");
}

int orator_stream_create(void** stream) {
  if (!stream) return fail(ORATOR_ERR_INVALID, "stream_create: null");
  hipStream_t s = nullptr;
  const int rc = check_hip(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreate");
  *stream = s;
  return rc;
}

int orator_stream_destroy(void* stream) {
  // the stream's workspace blocks go with it (graphs captured on it must be destroyed first)
  const int rc = orator_hip::workspace_release(static_cast<hipStream_t>(stream));
  const int rc2 = check_hip(hipStreamDestroy(static_cast<hipStream_t>(stream)), "hipStreamDestroy");
  return rc ? rc : rc2;
}

int orator_stream_synchronize(void* stream) {
  return check_hip(hipStreamSynchronize(static_cast<hipStream_t>(stream)),
                   "hipStreamSynchronize");
}

int orator_device_synchronize(void) {
  return check_hip(hipDeviceSynchronize(), "hipDeviceSynchronize");
}

int orator_event_create(void** event) {
  if (!event) return fail(ORATOR_ERR_INVALID, "event_create: null");
  hipEvent_t e = nullptr;
  const int rc = check_hip(hipEventCreate(&e), "hipEventCreate");
  *event = e;
  return rc;
}

int orator_event_destroy(void* event) {
  return check_hip(hipEventDestroy(static_cast<hipEvent_t>(event)), "hipEventDestroy");
}

int orator_event_record(void* event, void* stream) {
  return check_hip(hipEventRecord(static_cast<hipEvent_t>(event), static_cast<hipStream_t>(stream)),
                   "hipEventRecord");
}

int orator_event_elapsed_ms(float* ms, void* start, void* stop) {
  if (!ms) return fail(ORATOR_ERR_INVALID, "event_elapsed: null");
  const int rc = check_hip(hipEventSynchronize(static_cast<hipEvent_t>(stop)), "hipEventSynchronize");
  if (rc) return rc;
  return check_hip(hipEventElapsedTime(ms, static_cast<hipEvent_t>(start),
                                       static_cast<hipEvent_t>(stop)),
                   "hipEventElapsedTime");
}

// ConformerLayer::BuildPosEmb (src/model/conformer_layer.cu:314-329): host-side relative
// positional encoding [2T-1, d_model] for positions T-1 .. -(T-1), evaluated with the float
// overloads of std::exp / log / sin / cos as the reference does.
int orator_build_pos_emb(float* pe, int T, int d_model) {
  if (T <= 0 || d_model <= 0) return ORATOR_OK;
  if (!pe) return fail(ORATOR_ERR_INVALID, "build_pos_emb: null pointer");
  const int P = 2 * T - 1;
  for (int idx = 0; idx < P; ++idx) {
    const float pos = static_cast<float>(T - 1 - idx);
    for (int i = 0; i < d_model; i += 2) {
      const float div = std::exp(-(std::log(10000.0f)) * static_cast<float>(i) / d_model);
      pe[static_cast<size_t>(idx) * d_model + i] = std::sin(pos * div);
      if (i + 1 < d_model) pe[static_cast<size_t>(idx) * d_model + i + 1] = std::cos(pos * div);
    }
  }
  return ORATOR_OK;
}

int orator_time_next_decode(void* start, void* split_end, void* stop) {
  orator_hip::g_ev_start = static_cast<hipEvent_t>(start);
  orator_hip::g_ev_split = static_cast<hipEvent_t>(split_end);
  orator_hip::g_ev_stop = static_cast<hipEvent_t>(stop);
  return ORATOR_OK;
}

int orator_workspace_reserve(size_t bytes, void* stream) {
  return orator_hip::workspace(static_cast<hipStream_t>(stream), bytes) ? ORATOR_OK
                                                                        : ORATOR_ERR_HIP;
}

int orator_workspace_stats(size_t* blocks, size_t* bytes) {
  orator_hip::ws_pool().reap();
  if (blocks) *blocks = orator_hip::ws_pool().held_blocks();
  if (bytes) *bytes = orator_hip::ws_pool().held_bytes();
  return ORATOR_OK;
}

}  // extern "C"
