// Max-pool forward/backward and nearest upsample forward/backward.
//
// Maxpool follows the CPU path of TMaxPoolLayer (nMaxPoolLayer.pas:265-455):
// window origin (i*sY + off, j*sX + off) with off = -pad div 2, out-of-range
// taps read as -MaxSingle, windows scanned n-major then m, strict '>' keeps
// the first maximum, indices are global flat int64, -1 when no tap beats
// -MaxSingle.  Backward: where windows overlap, a gather (each input element
// sums, in ascending output index, the order of the serial scatter at
// :501-512, the deltas of the windows whose recorded index is that element);
// where they do not, the scatter itself (one delta per input element).
//
// Upsample (nupsamplelayer.pas:83-113): forward out = scale*in per output
// pixel; backward gathers the stride^2 output pixels of each input pixel in
// raster order, in += scale*out each, bit-identical to the serial loop.
#include <cfloat>
#include <mutex>
#include <unordered_map>

#include "common.hpp"

namespace tnh {
namespace {

constexpr int kThreads = 256;

unsigned grid_for(int64_t n) {
  const int64_t b = (n + kThreads - 1) / kThreads;
  return static_cast<unsigned>(b < 65536 ? (b > 0 ? b : 1) : 65536);
}

#define GRID_STRIDE(i, n) \
  for (int64_t i = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; i < (n); i += int64_t(gridDim.x) * blockDim.x)

struct PoolGeom {
  int64_t C, H, W, OH, OW, size, sX, sY, off;
};

// maxpool_depth (the CPU branch of TMaxPoolLayer.forwardMaxPool,
// nMaxPoolLayer.pas:372-399): output channel g of pixel p is the max over
// input channels g, g + outC, g + 2*outC, ... < c, strict '>', from
// -MaxSingle, with the input's global index (-1 when nothing beats the
// start value).
__global__ __launch_bounds__(kThreads) void maxpool_depth_kernel(int64_t total, int64_t c, int64_t outC, int64_t hw,
                                                                 const float* __restrict__ in,
                                                                 float* __restrict__ out, int64_t* __restrict__ idx) {
  GRID_STRIDE(o, total) {
    const int64_t p = o % hw;
    const int64_t t = o / hw;
    const int64_t g = t % outC;
    const int64_t b = t / outC;
    float mx = -FLT_MAX;
    int64_t mi = -1;
    for (int64_t k = g; k < c; k += outC) {
      const int64_t index = (b * c + k) * hw + p;
      const float v = in[index];
      if (v > mx) {
        mi = index;
        mx = v;
      }
    }
    out[o] = mx;
    if (idx) idx[o] = mi;
  }
}

__global__ __launch_bounds__(kThreads) void maxpool_fwd_kernel(PoolGeom g, int64_t total, const float* __restrict__ in,
                                                               float* __restrict__ out, int64_t* __restrict__ idx) {
  GRID_STRIDE(o, total) {
    const int64_t j = o % g.OW;
    const int64_t t = o / g.OW;
    const int64_t i = t % g.OH;
    const int64_t plane = t / g.OH;  // b*C + k
    float mx = -FLT_MAX;
    int64_t mi = -1;
    for (int64_t n = 0; n < g.size; ++n) {
      const int64_t ch = g.off + i * g.sY + n;
      for (int64_t m = 0; m < g.size; ++m) {
        const int64_t cw = g.off + j * g.sX + m;
        const int64_t index = cw + g.W * (ch + g.H * plane);
        const bool ok = ch >= 0 && ch < g.H && cw >= 0 && cw < g.W;
        const float v = ok ? in[index] : -FLT_MAX;
        if (v > mx) {
          mi = index;
          mx = v;
        }
      }
    }
    out[o] = mx;
    if (idx) idx[o] = mi;
  }
}

// 2x2 windows with stride 2 and no padding offset, every tap inside the
// image (2*OH <= H, 2*OW <= W, W even): one thread per two adjacent outputs
// of a row reads a 4-float span of the two input rows (16-byte loads when W
// % 4 == 0, else two 8-byte loads each), scans the taps in the reference
// order (row-major, strict '>', -MaxSingle start) and writes the two values
// (8 bytes) and the two int64 indices (16 bytes).  32-bit index arithmetic;
// the recorded indices are 64-bit.
template <bool V4>
__global__ __launch_bounds__(kThreads) void maxpool2_fwd_kernel(int total, int OH, int OW2, int H, int W,
                                                                const float* __restrict__ in, float* __restrict__ out,
                                                                int64_t* __restrict__ idx) {
  for (int t = blockIdx.x * kThreads + threadIdx.x; t < total; t += gridDim.x * kThreads) {
    const int jp = t % OW2, r = t / OW2;  // r = plane*OH + i
    const int i = r % OH, plane = r / OH;
    const int x0 = 4 * jp;
    const int64_t row0 = (static_cast<int64_t>(plane) * H + 2 * i) * W;
    float a[8];
    if constexpr (V4) {
      const float4 u = *reinterpret_cast<const float4*>(in + row0 + x0);
      const float4 v = *reinterpret_cast<const float4*>(in + row0 + W + x0);
      a[0] = u.x; a[1] = u.y; a[2] = u.z; a[3] = u.w; a[4] = v.x; a[5] = v.y; a[6] = v.z; a[7] = v.w;
    } else {
      const float2 u0 = *reinterpret_cast<const float2*>(in + row0 + x0);
      const float2 u1 = *reinterpret_cast<const float2*>(in + row0 + x0 + 2);
      const float2 v0 = *reinterpret_cast<const float2*>(in + row0 + W + x0);
      const float2 v1 = *reinterpret_cast<const float2*>(in + row0 + W + x0 + 2);
      a[0] = u0.x; a[1] = u0.y; a[2] = u1.x; a[3] = u1.y; a[4] = v0.x; a[5] = v0.y; a[6] = v1.x; a[7] = v1.y;
    }
    float m[2];
    int64_t k[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      float mx = -FLT_MAX;
      int64_t mi = -1;
#pragma unroll
      for (int n = 0; n < 2; ++n)
#pragma unroll
        for (int c = 0; c < 2; ++c) {
          const float v = a[4 * n + 2 * h + c];
          if (v > mx) {
            mx = v;
            mi = row0 + static_cast<int64_t>(n) * W + x0 + 2 * h + c;
          }
        }
      m[h] = mx;
      k[h] = mi;
    }
    const int64_t o = static_cast<int64_t>(r) * (2 * OW2) + 2 * jp;
    *reinterpret_cast<float2*>(out + o) = make_float2(m[0], m[1]);
    if (idx) {
      idx[o] = k[0];
      idx[o + 1] = k[1];
    }
  }
}

// Backward as the reference's scatter, dIn[idx[o]] += delta[o]
// (TNNCuda.backwardMaxPool, nncuda.pas:1121), one thread per output with an
// atomic add, skipping index -1.  Where the windows do not overlap (size <=
// stride) each input element receives at most one delta, so the result is
// the serial loop's bit for bit and needs no geometry; where two outputs
// name one input, the order of their adds is unspecified (the gather below
// keeps the serial order there).  Each thread reads its index and delta once
// (coalesced) and touches only the element its index names.
// ATOMIC: the adds are atomic (indexes whose geometry the library does not
// know); otherwise plain read-modify-writes, for windows known not to
// overlap, where no two threads name one element.
template <bool ATOMIC>
__global__ __launch_bounds__(kThreads) void maxpool_scatter_kernel(int64_t total, const int64_t* __restrict__ idx,
                                                                   const float* __restrict__ delta,
                                                                   float* __restrict__ dIn) {
  GRID_STRIDE(o, total) {
    const int64_t k = idx[o];
    if (k < 0) continue;
    if constexpr (ATOMIC)
      atomicAdd(dIn + k, delta[o]);
    else
      dIn[k] = dIn[k] + delta[o];
  }
}

// first output row/col whose window can contain input coordinate p:
// smallest i with off + i*s + size - 1 >= p
__device__ inline int64_t first_win(int64_t p, int64_t off, int64_t s, int64_t size) {
  const int64_t t = p - off - size + 1;
  return t <= 0 ? 0 : (t + s - 1) / s;
}

__global__ __launch_bounds__(kThreads) void maxpool_bwd_kernel(PoolGeom g, int64_t total,
                                                               const int64_t* __restrict__ idx,
                                                               const float* __restrict__ delta,
                                                               float* __restrict__ dIn) {
  GRID_STRIDE(e, total) {  // e = global input index
    const int64_t x = e % g.W;
    const int64_t t = e / g.W;
    const int64_t y = t % g.H;
    const int64_t plane = t / g.H;
    const int64_t i0 = first_win(y, g.off, g.sY, g.size);
    const int64_t j0 = first_win(x, g.off, g.sX, g.size);
    int64_t i1 = y - g.off;  // last i with off + i*s <= y
    int64_t j1 = x - g.off;
    if (i1 < 0 || j1 < 0) continue;
    i1 = min(i1 / g.sY, g.OH - 1);
    j1 = min(j1 / g.sX, g.OW - 1);
    // dIn is read and written only where an index names e, so the kernel
    // touches no element that the scatter it replaces would not
    float v = 0.f;
    bool hit = false;
    for (int64_t i = i0; i <= i1; ++i)
      for (int64_t j = j0; j <= j1; ++j) {
        const int64_t o = (plane * g.OH + i) * g.OW + j;
        if (idx[o] == e) {
          if (!hit) v = dIn[e];
          v = v + delta[o];
          hit = true;
        }
      }
    if (hit) dIn[e] = v;
  }
}

__global__ __launch_bounds__(kThreads) void upsample_fwd_kernel(int64_t total, int64_t h, int64_t w, int64_t s,
                                                                float scale, const float* __restrict__ in,
                                                                float* __restrict__ out) {
  const int64_t OW = w * s, OH = h * s;
  GRID_STRIDE(o, total) {
    const int64_t x = o % OW;
    const int64_t t = o / OW;
    const int64_t y = t % OH;
    const int64_t c = t / OH;
    out[o] = scale * in[(c * h + y / s) * w + x / s];
  }
}

// 2x nearest with scale 1 is a pure replication: each thread reads one input
// float and writes a 2x2 output block with two 8-byte stores.
__global__ __launch_bounds__(kThreads) void upsample2_fwd_kernel(int64_t total, int64_t h, int64_t w, float scale,
                                                                 const float* __restrict__ in,
                                                                 float* __restrict__ out) {
  const int64_t OW = 2 * w;
  GRID_STRIDE(e, total) {  // e = input index
    const int64_t x = e % w;
    const int64_t t = e / w;  // c*h + y
    const float v = scale * in[e];
    const int64_t o = (2 * t) * OW + 2 * x;
    *reinterpret_cast<float2*>(out + o) = make_float2(v, v);
    *reinterpret_cast<float2*>(out + o + OW) = make_float2(v, v);
  }
}

// Channels-last nearest upsample, forward: out pixel (b, y, x) channel c =
// scale * in pixel (b, y / s, x / s) channel c.  One thread per input pixel
// and channel group: one load, s*s stores, so the index arithmetic (32-bit
// when the sizes allow: I = int) is paid once per input element.  Four
// channels per thread (16-byte loads and stores) when C, both pixel strides
// and both bases allow.
template <bool VEC, class I>
__global__ __launch_bounds__(kThreads) void upsample_nhwc_kernel(I total, I C, I h, I w, int s, float scale,
                                                                 const float* __restrict__ in, int64_t inPix,
                                                                 float* __restrict__ out, int64_t outPix) {
  constexpr int V = VEC ? 4 : 1;
  const I CV = C / V, OW = w * s;
  for (I e = static_cast<I>(blockIdx.x) * kThreads + threadIdx.x; e < total;
       e += static_cast<I>(gridDim.x) * kThreads) {  // e = (input pixel, channel group)
    const I cg = e % CV, ip = e / CV;
    const I x = ip % w, t = ip / w;
    const I y = t % h, b = t / h;
    const float* src = in + static_cast<int64_t>(ip) * inPix + cg * V;
    const int64_t o0 = (static_cast<int64_t>(b) * h + y) * s * OW + static_cast<int64_t>(x) * s;
    if constexpr (VEC) {
      const float4 v = *reinterpret_cast<const float4*>(src);
      const float4 sv = make_float4(scale * v.x, scale * v.y, scale * v.z, scale * v.w);
      for (int dy = 0; dy < s; ++dy)
        for (int dx = 0; dx < s; ++dx)
          *reinterpret_cast<float4*>(out + (o0 + static_cast<int64_t>(dy) * OW + dx) * outPix + cg * V) = sv;
    } else {
      const float sv = scale * *src;
      for (int dy = 0; dy < s; ++dy)
        for (int dx = 0; dx < s; ++dx) out[(o0 + static_cast<int64_t>(dy) * OW + dx) * outPix + cg] = sv;
    }
  }
}

// Channels-last max pool, forward values (the inference layout keeps no
// indices): output pixel (b, i, j), channel c = the maximum over the window
// at (i*sY + off, j*sX + off), scanned as maxpool_fwd_kernel scans it (rows,
// then columns, strict '>', from -MaxSingle), so the values are the NCHW
// kernel's bit for bit (the first of equal values, e.g. +0 / -0, is kept).
// A tap outside the image reads -MaxSingle in the reference, which never
// beats the start value: it is skipped.  One thread per output pixel and
// channel group (four channels, 16-byte loads and stores, when C, both pixel
// strides and both bases allow); pixel indices in I (32-bit when they fit),
// element offsets in 64 bits.
template <bool VEC, class I>
__global__ __launch_bounds__(kThreads) void maxpool_nhwc_kernel(I total, I CV, I H, I W, I OH, I OW, int size,
                                                                int sY, int sX, int off, const float* __restrict__ in,
                                                                int64_t inPix, float* __restrict__ out,
                                                                int64_t outPix) {
  constexpr int V = VEC ? 4 : 1;
  for (I e = static_cast<I>(blockIdx.x) * kThreads + threadIdx.x; e < total;
       e += static_cast<I>(gridDim.x) * kThreads) {  // e = (output pixel, channel group)
    const I cg = e % CV, op = e / CV;
    const I j = op % OW, t = op / OW;
    const I i = t % OH, b = t / OH;
    float mx[V];
#pragma unroll
    for (int q = 0; q < V; ++q) mx[q] = -FLT_MAX;
    const I y0 = i * sY + off, x0 = j * sX + off;
    for (int n = 0; n < size; ++n) {
      const I ch = y0 + n;
      if (ch < 0 || ch >= H) continue;
      for (int m = 0; m < size; ++m) {
        const I cw = x0 + m;
        if (cw < 0 || cw >= W) continue;
        const float* src = in + static_cast<int64_t>((b * H + ch) * W + cw) * inPix + cg * V;
        float v[V];
        if constexpr (VEC) {
          const float4 u = *reinterpret_cast<const float4*>(src);
          v[0] = u.x; v[1] = u.y; v[2] = u.z; v[3] = u.w;
        } else {
          v[0] = *src;
        }
#pragma unroll
        for (int q = 0; q < V; ++q)
          if (v[q] > mx[q]) mx[q] = v[q];
      }
    }
    float* dst = out + static_cast<int64_t>(op) * outPix + cg * V;
    if constexpr (VEC)
      *reinterpret_cast<float4*>(dst) = make_float4(mx[0], mx[1], mx[2], mx[3]);
    else
      *dst = mx[0];
  }
}

__global__ __launch_bounds__(kThreads) void upsample_bwd_kernel(int64_t total, int64_t h, int64_t w, int64_t s,
                                                                float scale, float* __restrict__ in,
                                                                const float* __restrict__ out, int zeroIn) {
  const int64_t OW = w * s;
  GRID_STRIDE(e, total) {
    const int64_t x = e % w;
    const int64_t t = e / w;
    const int64_t y = t % h;
    const int64_t c = t / h;
    float v = zeroIn ? 0.f : in[e];
    for (int64_t dy = 0; dy < s; ++dy)
      for (int64_t dx = 0; dx < s; ++dx) {
        const float p = scale * out[((c * h) * s + y * s + dy) * OW + x * s + dx];
        v = v + p;
      }
    in[e] = v;
  }
}

bool al8(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 7) == 0; }
bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// The 2x2 / stride-2 kernels apply: window origin 0, every tap inside the
// image, even output rows (pairs of outputs), 8-byte aligned input and
// output, 16-byte aligned indices, and 32-bit element counts.
bool pool2_fast(const PoolGeom& g, int64_t batch, const float* in, const float* out, const int64_t* idx) {
  return g.size == 2 && g.sX == 2 && g.sY == 2 && g.off == 0 && 2 * g.OH <= g.H && 2 * g.OW <= g.W && g.W % 2 == 0 &&
         g.OW % 2 == 0 && al8(in) && al8(out) && (!idx || al16(idx)) &&
         batch * g.C * g.H * g.W + 65536LL * kThreads < INT32_MAX;
}

// Forward geometry of the maxpool calls that wrote an indexes buffer, so
// that the backward (which, like TNNCuda.backwardMaxPool, receives only the
// output shape and the buffers) can run the gather in the reference's order.
// Keyed by the indexes pointer; a later forward into the same buffer
// replaces the entry.
struct PoolRecord {
  PoolGeom g;
  int64_t batch;
};
std::mutex g_pool_mu;
std::unordered_map<const int64_t*, PoolRecord> g_pool_geom;

}  // namespace

void pool_remember_2x2(const int64_t* indexes, int64_t batch, int64_t C, int64_t h, int64_t w) {
  std::lock_guard<std::mutex> lk(g_pool_mu);
  g_pool_geom[indexes] = PoolRecord{PoolGeom{C, h, w, (h - 2) / 2 + 1, (w - 2) / 2 + 1, 2, 2, 2, 0}, batch};
}

bool pool_is_2x2(const int64_t* indexes, int64_t batch, int64_t C, int64_t h, int64_t w) {
  std::lock_guard<std::mutex> lk(g_pool_mu);
  const auto it = g_pool_geom.find(indexes);
  if (it == g_pool_geom.end()) return false;
  const PoolRecord& r = it->second;
  const PoolGeom& g = r.g;
  return r.batch == batch && g.C == C && g.H == h && g.W == w && g.OH == h / 2 && g.OW == w / 2 && g.size == 2 &&
         g.sX == 2 && g.sY == 2 && g.off == 0;
}

void pool_forget(const void* p) {
  std::lock_guard<std::mutex> lk(g_pool_mu);
  g_pool_geom.erase(static_cast<const int64_t*>(p));
}

}  // namespace tnh

using namespace tnh;

extern "C" int32_t tnh_maxpool_fwd(int64_t batch, int64_t outC, int64_t outH, int64_t outW, const float* input,
                                   int64_t c, int64_t h, int64_t w, int64_t strideX, int64_t strideY, int64_t padding,
                                   int64_t kernelSize, int64_t* indexes, float* output) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(batch >= 0 && c > 0 && h > 0 && w > 0 && kernelSize > 0 && strideX > 0 && strideY > 0 && padding >= 0,
          "maxpool_fwd: bad geometry");
  TNH_ARG(input && output, "maxpool_fwd: NULL buffer");
  if (outC != c) {  // maxpool_depth: the output keeps the input's h x w (nMaxPoolLayer.pas:98-102)
    TNH_ARG(outC > 0 && outH == h && outW == w, "maxpool_fwd: outC %lld != c %lld (maxpool_depth) needs outH = h "
            "and outW = w", (long long)outC, (long long)c);
    const int64_t total = batch * outC * h * w;
    if (total == 0) return TNH_OK;
    if (indexes) {  // every input element feeds at most one output: the backward scatters
      std::lock_guard<std::mutex> lk(g_pool_mu);
      g_pool_geom[indexes] = PoolRecord{PoolGeom{outC, h, w, h, w, 1, 1, 1, 0}, batch};
    }
    hipLaunchKernelGGL(maxpool_depth_kernel, dim3(grid_for(total)), dim3(kThreads), 0, cx->stream, total, c, outC,
                       h * w, input, output, indexes);
    return launch_status("maxpool_depth_kernel");
  }
  TNH_ARG(outH == (h + padding - kernelSize) / strideY + 1 && outW == (w + padding - kernelSize) / strideX + 1,
          "maxpool_fwd: output dims do not match (h + pad - size)/stride + 1");
  TNH_ARG(outH > 0 && outW > 0, "maxpool_fwd: empty output");
  const int64_t total = batch * outC * outH * outW;
  if (total == 0) return TNH_OK;
  PoolGeom g{c, h, w, outH, outW, kernelSize, strideX, strideY, -padding / 2};
  if (indexes) {
    std::lock_guard<std::mutex> lk(g_pool_mu);
    g_pool_geom[indexes] = PoolRecord{g, batch};
  }
  if (pool2_fast(g, batch, input, output, indexes)) {
    const int tot = static_cast<int>(total / 2);
    if (w % 4 == 0 && al16(input))
      hipLaunchKernelGGL(maxpool2_fwd_kernel<true>, dim3(grid_for(tot)), dim3(kThreads), 0, cx->stream, tot,
                         static_cast<int>(outH), static_cast<int>(outW / 2), static_cast<int>(h), static_cast<int>(w),
                         input, output, indexes);
    else
      hipLaunchKernelGGL(maxpool2_fwd_kernel<false>, dim3(grid_for(tot)), dim3(kThreads), 0, cx->stream, tot,
                         static_cast<int>(outH), static_cast<int>(outW / 2), static_cast<int>(h), static_cast<int>(w),
                         input, output, indexes);
    return launch_status("maxpool2_fwd_kernel");
  }
  hipLaunchKernelGGL(maxpool_fwd_kernel, dim3(grid_for(total)), dim3(kThreads), 0, cx->stream, g, total, input, output,
                     indexes);
  return launch_status("maxpool_fwd_kernel");
}

namespace {

// Backward with a known forward geometry: windows that do not overlap
// (size <= stride both ways) scatter (exact, no ordering needed); overlapping
// ones gather in the serial order.
int maxpool_bwd_known(Context* cx, int64_t batch, const PoolGeom& g, const int64_t* indexes, const float* delta,
                      float* deltaIn) {
  if (g.size <= g.sX && g.size <= g.sY) {
    const int64_t total = batch * g.C * g.OH * g.OW;
    if (total == 0) return TNH_OK;
    hipLaunchKernelGGL(maxpool_scatter_kernel<false>, dim3(grid_for(total)), dim3(kThreads), 0, cx->stream, total,
                       indexes, delta, deltaIn);
    return launch_status("maxpool_scatter_kernel");
  }
  const int64_t total = batch * g.C * g.H * g.W;
  if (total == 0) return TNH_OK;
  hipLaunchKernelGGL(maxpool_bwd_kernel, dim3(grid_for(total)), dim3(kThreads), 0, cx->stream, g, total, indexes,
                     delta, deltaIn);
  return launch_status("maxpool_bwd_kernel");
}

}  // namespace

extern "C" int32_t tnh_maxpool_bwd(int64_t batch, int64_t outC, int64_t outH, int64_t outW, float* output,
                                   const int64_t* indexes, const float* delta) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(batch >= 0 && outC > 0 && outH > 0 && outW > 0, "maxpool_bwd: bad sizes");
  TNH_ARG(indexes && delta && output, "maxpool_bwd: NULL buffer");
  PoolRecord rec{};
  bool known = false;
  {
    std::lock_guard<std::mutex> lk(g_pool_mu);
    auto it = g_pool_geom.find(indexes);
    if (it != g_pool_geom.end()) {
      const PoolGeom& g = it->second.g;
      known = g.C == outC && g.OH == outH && g.OW == outW && it->second.batch == batch;
      rec = it->second;
    }
  }
  if (known) return maxpool_bwd_known(cx, batch, rec.g, indexes, delta, output);
  const int64_t total = batch * outC * outH * outW;
  if (total == 0) return TNH_OK;
  hipLaunchKernelGGL(maxpool_scatter_kernel<true>, dim3(grid_for(total)), dim3(kThreads), 0, cx->stream, total,
                     indexes, delta, output);
  return launch_status("maxpool_scatter_kernel<atomic>");
}

extern "C" int32_t tnh_maxpool_bwd_geom(int64_t batch, int64_t outC, int64_t outH, int64_t outW, float* output,
                                        const int64_t* indexes, const float* delta, int64_t h, int64_t w,
                                        int64_t strideX, int64_t strideY, int64_t padding, int64_t kernelSize) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(batch >= 0 && outC > 0 && h > 0 && w > 0 && kernelSize > 0 && strideX > 0 && strideY > 0 && padding >= 0,
          "maxpool_bwd_geom: bad geometry");
  TNH_ARG(outH == (h + padding - kernelSize) / strideY + 1 && outW == (w + padding - kernelSize) / strideX + 1,
          "maxpool_bwd_geom: output dims do not match the forward geometry");
  TNH_ARG(indexes && delta && output, "maxpool_bwd_geom: NULL buffer");
  const PoolGeom g{outC, h, w, outH, outW, kernelSize, strideX, strideY, -padding / 2};
  return maxpool_bwd_known(cx, batch, g, indexes, delta, output);
}

extern "C" int32_t tnh_upsample(int64_t batch, int64_t channels, int64_t h, int64_t w, float* in, int64_t stride,
                                int32_t isForward, float scale, float* out, int32_t zeroIn) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(batch >= 0 && channels > 0 && h > 0 && w > 0 && stride > 0, "upsample: bad geometry");
  TNH_ARG(in && out, "upsample: NULL buffer");
  const int64_t planes = batch * channels;
  if (planes == 0) return TNH_OK;
  if (isForward) {
    if (stride == 2 && al8(out) && w > 0) {
      const int64_t total = planes * h * w;
      hipLaunchKernelGGL(upsample2_fwd_kernel, dim3(grid_for(total)), dim3(kThreads), 0, cx->stream, total, h, w,
                         scale, in, out);
      return launch_status("upsample2_fwd_kernel");
    }
    const int64_t total = planes * h * w * stride * stride;
    hipLaunchKernelGGL(upsample_fwd_kernel, dim3(grid_for(total)), dim3(kThreads), 0, cx->stream, total, h, w, stride,
                       scale, in, out);
    return launch_status("upsample_fwd_kernel");
  }
  const int64_t total = planes * h * w;
  hipLaunchKernelGGL(upsample_bwd_kernel, dim3(grid_for(total)), dim3(kThreads), 0, cx->stream, total, h, w, stride,
                     scale, in, out, zeroIn);
  return launch_status("upsample_bwd_kernel");
}

extern "C" int32_t tnh_upsample_nhwc(int64_t batch, int64_t channels, int64_t h, int64_t w, int64_t stride,
                                     float scale, const float* in, int64_t inOff, int64_t inPix, float* out,
                                     int64_t outOff, int64_t outPix) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(batch >= 0 && channels > 0 && h > 0 && w > 0 && stride > 0, "upsample_nhwc: bad geometry");
  TNH_ARG(in && out && inOff >= 0 && outOff >= 0, "upsample_nhwc: NULL buffer or negative offset");
  TNH_ARG(inPix >= channels && outPix >= channels, "upsample_nhwc: pixel stride below the channel count");
  const float* src = in + inOff;
  float* dst = out + outOff;
  TNH_ARG(stride <= 64, "upsample_nhwc: stride %lld above 64", (long long)stride);
  const int64_t pixels = batch * h * w;  // input pixels
  if (pixels == 0) return TNH_OK;
  const bool vec = channels % 4 == 0 && inPix % 4 == 0 && outPix % 4 == 0 &&
                   (reinterpret_cast<uintptr_t>(src) & 15) == 0 && (reinterpret_cast<uintptr_t>(dst) & 15) == 0;
  const int64_t total = pixels * (vec ? channels / 4 : channels);
  // 32-bit indices when every index the kernel forms (input elements, rows
  // of output pixels) stays below 2^31
  const bool small = total + kThreads * 65536LL < INT32_MAX && batch * h * stride < INT32_MAX &&
                     w * stride < INT32_MAX;
  auto go = [&](auto vecTag, auto idx) {
    constexpr bool VEC = decltype(vecTag)::value;
    using I = decltype(idx);
    hipLaunchKernelGGL((upsample_nhwc_kernel<VEC, I>), dim3(grid_for(total)), dim3(kThreads), 0, cx->stream,
                       static_cast<I>(total), static_cast<I>(channels), static_cast<I>(h), static_cast<I>(w),
                       static_cast<int>(stride), scale, src, inPix, dst, outPix);
  };
  if (vec)
    small ? go(std::true_type{}, int{}) : go(std::true_type{}, int64_t{});
  else
    small ? go(std::false_type{}, int{}) : go(std::false_type{}, int64_t{});
  return launch_status("upsample_nhwc_kernel");
}

extern "C" int32_t tnh_maxpool_fwd_nhwc(int64_t batch, int64_t channels, int64_t h, int64_t w, int64_t outH,
                                        int64_t outW, int64_t strideX, int64_t strideY, int64_t padding,
                                        int64_t kernelSize, const float* in, int64_t inOff, int64_t inPix, float* out,
                                        int64_t outOff, int64_t outPix) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(batch >= 0 && channels > 0 && h > 0 && w > 0 && kernelSize > 0 && strideX > 0 && strideY > 0 &&
              padding >= 0,
          "maxpool_fwd_nhwc: bad geometry");
  TNH_ARG(outH == (h + padding - kernelSize) / strideY + 1 && outW == (w + padding - kernelSize) / strideX + 1,
          "maxpool_fwd_nhwc: output dims do not match (h + pad - size)/stride + 1");
  TNH_ARG(outH > 0 && outW > 0, "maxpool_fwd_nhwc: empty output");
  TNH_ARG(in && out && inOff >= 0 && outOff >= 0, "maxpool_fwd_nhwc: NULL buffer or negative offset");
  TNH_ARG(inPix >= channels && outPix >= channels, "maxpool_fwd_nhwc: pixel stride below the channel count");
  TNH_ARG(kernelSize <= 64 && padding <= 64 && strideX <= 64 && strideY <= 64,
          "maxpool_fwd_nhwc: size, stride and padding up to 64");
  const float* src = in + inOff;
  float* dst = out + outOff;
  const int64_t pixels = batch * outH * outW;
  if (pixels == 0) return TNH_OK;
  const bool vec = channels % 4 == 0 && inPix % 4 == 0 && outPix % 4 == 0 && al16(src) && al16(dst);
  const int64_t CV = vec ? channels / 4 : channels;
  const int64_t total = pixels * CV;
  // 32-bit pixel arithmetic when every pixel index (input and output, and
  // the grid-stride index) stays below 2^31
  const bool small = total + kThreads * 65536LL < INT32_MAX && batch * h * w < INT32_MAX;
  const int off = static_cast<int>(-padding / 2);
  auto go = [&](auto vecTag, auto idx) {
    constexpr bool VEC = decltype(vecTag)::value;
    using I = decltype(idx);
    hipLaunchKernelGGL((maxpool_nhwc_kernel<VEC, I>), dim3(grid_for(total)), dim3(kThreads), 0, cx->stream,
                       static_cast<I>(total), static_cast<I>(CV), static_cast<I>(h), static_cast<I>(w),
                       static_cast<I>(outH), static_cast<I>(outW), static_cast<int>(kernelSize),
                       static_cast<int>(strideY), static_cast<int>(strideX), off, src, inPix, dst, outPix);
  };
  if (vec)
    small ? go(std::true_type{}, int{}) : go(std::true_type{}, int64_t{});
  else
    small ? go(std::false_type{}, int{}) : go(std::false_type{}, int64_t{});
  return launch_status("maxpool_nhwc_kernel");
}
