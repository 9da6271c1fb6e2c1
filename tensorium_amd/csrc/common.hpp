// Shared host-side plumbing of libtensorium_hip: status codes, the
// thread-local last-error string, the per-process device context (one HIP
// stream, like TNNCuda's single stream, nncuda.pas:455) and argument checks.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <functional>
#include <vector>

#include "../../include/tensorium_hip.h"

namespace tnh {

// Records a formatted message for tnh_last_error() and returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

struct Context {
  int device = -1;
  hipStream_t own_stream = nullptr;  // created by tnh_init
  hipStream_t stream = nullptr;      // stream kernels are launched on
  hipStream_t tune_stream = nullptr; // private stream the autotuner captures its timing graphs on
  int cu_count = 0;
  int xcd_count = 8;
  // Library scratch (split-K partial sums), one buffer per stream the
  // library has launched on, grown on demand: work on different streams may
  // run concurrently, so it never shares scratch.
  struct WsSlot {
    hipStream_t stream;
    void* ptr;
    size_t bytes;
  };
  std::vector<WsSlot> ws;
  // Per-stream copies of reference-layout 3x3 weights repacked tap-major for
  // the call being made (pack_buffer), same growth rules as ws.
  std::vector<WsSlot> pk;
  // Per-stream arrival counters of the conv kernels' in-kernel tail
  // reductions (kTileCounters ints each), zeroed when allocated; every
  // launch that uses them leaves them zero.
  std::vector<WsSlot> cnt;
  // Outgrown scratch buffers: a graph captured earlier may still launch
  // kernels that address them, so they are freed only by tnh_finalize.
  std::vector<void*> wsRetired;
  // Partial sums of the multi-workgroup channel reductions (batch-norm
  // statistics and their deltas, bias gradients, addDots), redFloats floats
  // per stream the reductions have run on: reductions on different streams
  // may run concurrently, so no two streams share one.  tnh_init allocates
  // kRedSpare buffers up front, which streams first used under graph capture
  // (when nothing can be allocated) take; later streams allocate their own.
  struct RedSlot {
    hipStream_t stream;
    float* ptr;
  };
  std::vector<RedSlot> red;
  std::vector<float*> redSpare;
  int64_t redFloats = 0;
};

constexpr int64_t kRedFloats = int64_t(1) << 20;  // 4 MiB of reduction partials per stream
constexpr int kRedSpare = 4;

// True when the context stream (or the autotuner's stream) is being
// captured into a graph, so that nothing may be allocated.
bool capturing(const Context* c);

// The current stream's reduction-partials buffer (redFloats floats), or
// nullptr when the stream has none, no spare is left and none can be
// allocated (allocation failure, or the stream is being captured).
float* reduction_buffer(Context* c);

// Returns the current stream's scratch buffer of at least `bytes` on the
// context device, growing it (a new hipMalloc; the outgrown buffer stays
// allocated until tnh_finalize) when needed; returns nullptr when growing is
// not possible (allocation failure, or the stream or the tuning stream is
// being captured).
void* workspace(Context* c, size_t bytes);

constexpr int64_t kTileCounters = int64_t(1) << 16;

// The current stream's tail-tile arrival counters (kTileCounters ints, all
// zero between launches), or nullptr when the stream has none and they
// cannot be allocated now (allocation failure, or a capture in progress).
int* tile_counters(Context* c);

// The current stream's weight-repacking buffer of at least `bytes`, grown
// like workspace() (nullptr when it cannot be).
void* pack_buffer(Context* c, size_t bytes);

// Looks up, once per device and with that device current, the address of
// the no-allocation entry point's static scratch on it (conv.hip); called by
// tnh_init.
int conv_scratch_setup(int device);

// Forgets the maxpool forward geometry recorded for an indexes buffer at p
// (pool.hip); tnh_free calls it for every buffer it releases.
void pool_forget(const void* p);
// records that `indexes` holds the int64 indices of a 2x2 / stride 2 /
// padding 0 maxpool forward over [batch][C][h][w] (so tnh_maxpool_bwd finds
// the geometry)
void pool_remember_2x2(const int64_t* indexes, int64_t batch, int64_t C, int64_t h, int64_t w);
// True when the library recorded `indexes` as the indexes of a 2x2 stride-2
// maxpool (no offset) over [batch][C][h][w].
bool pool_is_2x2(const int64_t* indexes, int64_t batch, int64_t C, int64_t h, int64_t w);

// Deterministic mode (tnh_set_deterministic): no timing-based tuning and no
// split-K / tail-split tilings, so every process runs the same kernels and
// produces the same bits.
bool deterministic();

// Returns the live context or nullptr (after recording TNH_ERR_NOT_INITIALIZED).
Context* ctx();

// Times launch(stream) the way a captured network runs it: `reps` launches
// captured into a graph on the context's tuning stream, replayed twice after a
// warm-up replay; ms = the faster replay's time per launch.  The caller
// synchronizes its own stream first and keeps every buffer the launches touch
// allocated (nothing may be allocated during the capture).
int time_graph(Context* cx, const std::function<int(hipStream_t)>& launch, int reps, float& ms);

// Checks a launch or runtime call; returns TNH_OK or TNH_ERR_HIP with text.
int hip_status(hipError_t e, const char* what);

inline int launch_status(const char* what) { return hip_status(hipGetLastError(), what); }

}  // namespace tnh

#define TNH_REQUIRE_CTX(c)                 \
  tnh::Context* c = tnh::ctx();            \
  if (!c) return TNH_ERR_NOT_INITIALIZED;

#define TNH_ARG(cond, ...)                                   \
  do {                                                       \
    if (!(cond)) return tnh::fail(TNH_ERR_INVALID_ARG, __VA_ARGS__); \
  } while (0)
