// Context, memory, error and event entry points of libtensorium_hip.
// Mirrors TNNCuda's lifecycle (Create/Destroy/finish, nncuda.pas:448-469,
// 1575) with a status-code + last-error channel in place of SAFE_CALL's
// assert (nncuda.pas:237-275).
#include <atomic>
#include <cstdio>
#include <mutex>

#include "common.hpp"

namespace tnh {

namespace {
thread_local char g_err[512] = "";
std::atomic<bool> g_deterministic{false};
Context g_ctx;
bool g_live = false;
std::mutex g_mu;
}  // namespace

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int hip_status(hipError_t e, const char* what) {
  if (e == hipSuccess) return TNH_OK;
  if (e == hipErrorOutOfMemory) return fail(TNH_ERR_OUT_OF_MEMORY, "%s: %s", what, hipGetErrorString(e));
  return fail(TNH_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

bool deterministic() { return g_deterministic.load(std::memory_order_relaxed); }

Context* ctx() {
  if (!g_live) {
    fail(TNH_ERR_NOT_INITIALIZED, "tnh_init has not been called");
    return nullptr;
  }
  return &g_ctx;
}

int time_graph(Context* cx, const std::function<int(hipStream_t)>& launch, int reps, float& ms) {
  const hipStream_t ts = cx->tune_stream;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  hipGraph_t g = nullptr;
  hipGraphExec_t ge = nullptr;
  ms = 1e30f;
  int st = hip_status(hipEventCreate(&e0), "hipEventCreate");
  if (!st) st = hip_status(hipEventCreate(&e1), "hipEventCreate");
  if (!st) {
    st = hip_status(hipStreamBeginCapture(ts, hipStreamCaptureModeRelaxed), "hipStreamBeginCapture");
    if (!st) {
      for (int r = 0; r < reps && !st; ++r) st = launch(ts);
      const hipError_t ee = hipStreamEndCapture(ts, &g);
      if (!st) st = hip_status(ee, "hipStreamEndCapture");
    }
  }
  if (!st) st = hip_status(hipGraphInstantiate(&ge, g, nullptr, nullptr, 0), "hipGraphInstantiate");
  if (!st) st = hip_status(hipGraphLaunch(ge, ts), "hipGraphLaunch");
  for (int t = 0; t < 2 && !st; ++t) {
    (void)hipEventRecord(e0, ts);
    st = hip_status(hipGraphLaunch(ge, ts), "hipGraphLaunch");
    (void)hipEventRecord(e1, ts);
    if (!st) st = hip_status(hipEventSynchronize(e1), "hipEventSynchronize");
    float v = 0.f;
    if (!st && hipEventElapsedTime(&v, e0, e1) == hipSuccess && v / reps < ms) ms = v / reps;
  }
  (void)hipStreamSynchronize(ts);
  if (ge) (void)hipGraphExecDestroy(ge);
  if (g) (void)hipGraphDestroy(g);
  if (e0) (void)hipEventDestroy(e0);
  if (e1) (void)hipEventDestroy(e1);
  return st;
}

bool capturing(const Context* c) {
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone, ts = hipStreamCaptureStatusNone;
  return hipStreamIsCapturing(c->stream, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone ||
         (c->tune_stream &&
          (hipStreamIsCapturing(c->tune_stream, &ts) != hipSuccess || ts != hipStreamCaptureStatusNone));
}

namespace {

// One growable buffer per stream in `slots`.
void* stream_buffer(Context* c, std::vector<Context::WsSlot>& slots, size_t bytes) {
  Context::WsSlot* slot = nullptr;
  for (Context::WsSlot& w : slots)
    if (w.stream == c->stream) slot = &w;
  if (slot && bytes <= slot->bytes) return slot->ptr;
  // Nothing can be allocated under capture.  A stream without scratch of its
  // own gets none (its callers then run whole-K tilings, or compute without
  // the scratch): borrowing another stream's would race when both run.
  if (capturing(c)) return nullptr;
  if (!slot) {
    slots.push_back({c->stream, nullptr, 0});
    slot = &slots.back();
  }
  if (slot->ptr) {
    c->wsRetired.push_back(slot->ptr);
    slot->ptr = nullptr;
    slot->bytes = 0;
  }
  const size_t want = bytes + (bytes >> 2);
  if (hipMalloc(&slot->ptr, want) != hipSuccess) {
    (void)hipGetLastError();
    slot->ptr = nullptr;
    return nullptr;
  }
  slot->bytes = want;
  return slot->ptr;
}

}  // namespace

void* workspace(Context* c, size_t bytes) { return stream_buffer(c, c->ws, bytes); }

void* pack_buffer(Context* c, size_t bytes) { return stream_buffer(c, c->pk, bytes); }

int* tile_counters(Context* c) {
  for (const Context::WsSlot& w : c->cnt)
    if (w.stream == c->stream) return static_cast<int*>(w.ptr);
  if (capturing(c)) return nullptr;
  void* p = nullptr;
  const size_t bytes = static_cast<size_t>(kTileCounters) * sizeof(int);
  if (hipMalloc(&p, bytes) != hipSuccess) {
    (void)hipGetLastError();
    return nullptr;
  }
  // zeroed in stream order, before any kernel of this stream uses them
  if (hipMemsetAsync(p, 0, bytes, c->stream) != hipSuccess) {
    (void)hipGetLastError();
    (void)hipFree(p);
    return nullptr;
  }
  c->cnt.push_back({c->stream, p, bytes});
  return static_cast<int*>(p);
}

float* reduction_buffer(Context* c) {
  for (const Context::RedSlot& r : c->red)
    if (r.stream == c->stream) return r.ptr;
  float* p = nullptr;
  if (!c->redSpare.empty()) {
    p = c->redSpare.back();
    c->redSpare.pop_back();
  } else {
    if (capturing(c)) return nullptr;
    if (hipMalloc(&p, static_cast<size_t>(c->redFloats) * 4) != hipSuccess) {
      (void)hipGetLastError();
      return nullptr;
    }
  }
  c->red.push_back({c->stream, p});
  return p;
}

// Frees every buffer of the context and destroys its streams.
void release(Context& c) {
  for (const Context::WsSlot& w : c.ws)
    if (w.ptr) (void)hipFree(w.ptr);
  for (const Context::WsSlot& w : c.pk)
    if (w.ptr) (void)hipFree(w.ptr);
  for (const Context::WsSlot& w : c.cnt)
    if (w.ptr) (void)hipFree(w.ptr);
  for (void* p : c.wsRetired) (void)hipFree(p);
  for (const Context::RedSlot& r : c.red) (void)hipFree(r.ptr);
  for (float* p : c.redSpare) (void)hipFree(p);
  if (c.own_stream) (void)hipStreamDestroy(c.own_stream);
  if (c.tune_stream) (void)hipStreamDestroy(c.tune_stream);
  c = Context{};
}

}  // namespace tnh

using namespace tnh;

extern "C" const char* tnh_last_error(void) { return g_err; }

extern "C" int32_t tnh_device_count(int32_t* count) {
  TNH_ARG(count != nullptr, "device_count: NULL");
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess) {
    *count = 0;
    return hip_status(e, "hipGetDeviceCount");
  }
  *count = n;
  return TNH_OK;
}

extern "C" int32_t tnh_init(int32_t device) {
  std::lock_guard<std::mutex> lk(g_mu);
  int n = 0;
  if (int st = hip_status(hipGetDeviceCount(&n), "hipGetDeviceCount")) return st;
  TNH_ARG(device >= 0 && device < n, "init: device %d out of range (%d devices)", device, n);
  if (g_live) {
    if (g_ctx.device == device) return TNH_OK;
    (void)hipSetDevice(g_ctx.device);
    (void)hipStreamSynchronize(g_ctx.stream);
    release(g_ctx);
    g_live = false;
  }
  if (int st = hip_status(hipSetDevice(device), "hipSetDevice")) return st;
  Context c;
  int st = hip_status(hipStreamCreateWithFlags(&c.own_stream, hipStreamNonBlocking), "hipStreamCreate");
  if (!st) st = hip_status(hipStreamCreateWithFlags(&c.tune_stream, hipStreamNonBlocking), "hipStreamCreate");
  if (!st) st = conv_scratch_setup(device);
  for (int i = 0; i < kRedSpare && !st; ++i) {
    float* p = nullptr;
    st = hip_status(hipMalloc(&p, kRedFloats * 4), "hipMalloc(reduction partials)");
    if (!st) c.redSpare.push_back(p);
  }
  if (st) {
    release(c);
    return st;
  }
  int cus = 0;
  (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device);
  c.device = device;
  c.stream = c.own_stream;
  c.cu_count = cus > 0 ? cus : 256;
  c.redFloats = kRedFloats;
  g_ctx = c;
  g_live = true;
  return TNH_OK;
}

extern "C" int32_t tnh_finalize(void) {
  std::lock_guard<std::mutex> lk(g_mu);
  if (!g_live) return TNH_OK;
  (void)hipSetDevice(g_ctx.device);
  (void)hipStreamSynchronize(g_ctx.stream);
  release(g_ctx);
  g_live = false;
  return TNH_OK;
}

extern "C" int32_t tnh_set_deterministic(int32_t enable) {
  g_deterministic.store(enable != 0, std::memory_order_relaxed);
  return TNH_OK;
}

extern "C" int32_t tnh_synchronize(void) {
  TNH_REQUIRE_CTX(cx);
  return hip_status(hipStreamSynchronize(cx->stream), "hipStreamSynchronize");
}

extern "C" int32_t tnh_get_stream(void** stream) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(stream != nullptr, "get_stream: NULL");
  *stream = cx->stream;
  return TNH_OK;
}

extern "C" int32_t tnh_set_stream(void* stream) {
  TNH_REQUIRE_CTX(cx);
  cx->stream = static_cast<hipStream_t>(stream);  // NULL selects the HIP null stream
  return TNH_OK;
}

extern "C" int32_t tnh_reset_stream(void) {
  TNH_REQUIRE_CTX(cx);
  cx->stream = cx->own_stream;
  return TNH_OK;
}

extern "C" int32_t tnh_cu_count(int32_t* count) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(count != nullptr, "cu_count: NULL");
  *count = cx->cu_count;
  return TNH_OK;
}

extern "C" int32_t tnh_malloc(int64_t bytes, void** ptr) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(ptr != nullptr && bytes >= 0, "malloc: bad arguments");
  *ptr = nullptr;
  if (bytes == 0) return TNH_OK;
  return hip_status(hipMalloc(ptr, static_cast<size_t>(bytes)), "hipMalloc");
}

extern "C" int32_t tnh_free(void* ptr) {
  TNH_REQUIRE_CTX(cx);
  if (!ptr) return TNH_OK;
  pool_forget(ptr);
  return hip_status(hipFree(ptr), "hipFree");
}

extern "C" int32_t tnh_h2d(void* dst, const void* src, int64_t bytes) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(bytes >= 0, "h2d: negative size");
  if (bytes == 0) return TNH_OK;
  TNH_ARG(dst && src, "h2d: NULL pointer");
  if (int st = hip_status(hipMemcpyAsync(dst, src, static_cast<size_t>(bytes), hipMemcpyHostToDevice, cx->stream),
                          "hipMemcpyAsync(H2D)"))
    return st;
  return hip_status(hipStreamSynchronize(cx->stream), "hipStreamSynchronize");
}

extern "C" int32_t tnh_d2h(void* dst, const void* src, int64_t bytes) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(bytes >= 0, "d2h: negative size");
  if (bytes == 0) return TNH_OK;
  TNH_ARG(dst && src, "d2h: NULL pointer");
  if (int st = hip_status(hipMemcpyAsync(dst, src, static_cast<size_t>(bytes), hipMemcpyDeviceToHost, cx->stream),
                          "hipMemcpyAsync(D2H)"))
    return st;
  return hip_status(hipStreamSynchronize(cx->stream), "hipStreamSynchronize");
}

extern "C" int32_t tnh_event_create(void** ev) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(ev != nullptr, "event_create: NULL");
  hipEvent_t e = nullptr;
  if (int st = hip_status(hipEventCreate(&e), "hipEventCreate")) return st;
  *ev = e;
  return TNH_OK;
}

extern "C" int32_t tnh_event_destroy(void* ev) {
  TNH_REQUIRE_CTX(cx);
  if (!ev) return TNH_OK;
  return hip_status(hipEventDestroy(static_cast<hipEvent_t>(ev)), "hipEventDestroy");
}

extern "C" int32_t tnh_event_record(void* ev) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(ev != nullptr, "event_record: NULL");
  return hip_status(hipEventRecord(static_cast<hipEvent_t>(ev), cx->stream), "hipEventRecord");
}

extern "C" int32_t tnh_stream_create(void** stream) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(stream != nullptr, "stream_create: NULL");
  hipStream_t s = nullptr;  // default priority, like the context's own stream
  if (int st = hip_status(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreate")) return st;
  *stream = s;
  return TNH_OK;
}

extern "C" int32_t tnh_stream_destroy(void* stream) {
  TNH_REQUIRE_CTX(cx);
  if (!stream) return TNH_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  TNH_ARG(s != cx->own_stream && s != cx->tune_stream, "stream_destroy: the context's own stream");
  TNH_ARG(s != cx->stream, "stream_destroy: the stream is selected (tnh_reset_stream first)");
  // its work ends first: the scratch kept for this handle may go to a later
  // stream that gets the same handle
  if (int st = hip_status(hipStreamSynchronize(s), "hipStreamSynchronize")) return st;
  return hip_status(hipStreamDestroy(s), "hipStreamDestroy");
}

extern "C" int32_t tnh_stream_wait_event(void* ev) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(ev != nullptr, "stream_wait_event: NULL");
  return hip_status(hipStreamWaitEvent(cx->stream, static_cast<hipEvent_t>(ev), 0), "hipStreamWaitEvent");
}

extern "C" int32_t tnh_event_elapsed_ms(void* start, void* stop, float* ms) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(start && stop && ms, "event_elapsed: NULL");
  if (int st = hip_status(hipEventSynchronize(static_cast<hipEvent_t>(stop)), "hipEventSynchronize")) return st;
  return hip_status(hipEventElapsedTime(ms, static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(stop)),
                    "hipEventElapsedTime");
}

extern "C" int32_t tnh_graph_begin(void) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(cx->stream != nullptr, "graph_begin: the null stream cannot be captured (tnh_reset_stream first)");
  return hip_status(hipStreamBeginCapture(cx->stream, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
}

extern "C" int32_t tnh_graph_end(void** graphExec) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(graphExec != nullptr, "graph_end: NULL");
  *graphExec = nullptr;
  hipGraph_t g = nullptr;
  if (int st = hip_status(hipStreamEndCapture(cx->stream, &g), "hipStreamEndCapture")) return st;
  hipGraphExec_t ge = nullptr;
  const int st = hip_status(hipGraphInstantiate(&ge, g, nullptr, nullptr, 0), "hipGraphInstantiate");
  (void)hipGraphDestroy(g);
  if (st) return st;
  *graphExec = ge;
  return TNH_OK;
}

extern "C" int32_t tnh_graph_launch(void* graphExec) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(graphExec != nullptr, "graph_launch: NULL");
  return hip_status(hipGraphLaunch(static_cast<hipGraphExec_t>(graphExec), cx->stream), "hipGraphLaunch");
}

extern "C" int32_t tnh_graph_destroy(void* graphExec) {
  TNH_REQUIRE_CTX(cx);
  if (!graphExec) return TNH_OK;
  return hip_status(hipGraphExecDestroy(static_cast<hipGraphExec_t>(graphExec)), "hipGraphExecDestroy");
}
