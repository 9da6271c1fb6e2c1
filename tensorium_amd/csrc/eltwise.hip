// Bandwidth-bound element-wise kernels: bias / scale epilogues, activations,
// BLAS-1 helpers, route (concat) copies and the batch-norm normalize.  Each
// element is produced by exactly the single fp32 operation the reference CPU
// path applies (bit-exact).  Per-channel passes walk rows (rows.hpp);
// flat passes use 16-byte accesses when the buffers allow.
#include <cfloat>

#include "chanstat.hpp"
#include "common.hpp"
#include "rows.hpp"
#include "yolo_math.hpp"

namespace tnh {
namespace {

constexpr int kThreads = 256;

unsigned grid_for(int64_t n) {
  const int64_t b = (n + kThreads - 1) / kThreads;
  return static_cast<unsigned>(b < 16384 ? (b > 0 ? b : 1) : 16384);
}

#define GRID_STRIDE(i, n) \
  for (int64_t i = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; i < (n); i += int64_t(gridDim.x) * blockDim.x)

bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

template <class Op>
__device__ inline float4 map4(const Op& op, const typename Op::Ch& c, float4 v) {
  return make_float4(op(c, v.x), op(c, v.y), op(c, v.z), op(c, v.w));
}

// x = op(channel constants, x) in place, row by row (rows.hpp)
template <int VW, class Op>
__global__ __launch_bounds__(kThreads) void rows_kernel(Op op, float* __restrict__ x, Rows g) {
  const int t = threadIdx.x, lr = t / g.cpt, lc = t - lr * g.cpt;
  if (lr >= g.rpw) return;
  for (int64_t r = static_cast<int64_t>(blockIdx.x) * g.rpw + lr; r < g.rows;
       r += static_cast<int64_t>(gridDim.x) * g.rpw) {
    const typename Op::Ch c = op.chan(r % g.nb);
    float* row = x + r * g.block;
    for (int64_t k = lc; k < g.cpr; k += g.cpt) {
      if constexpr (VW == 4) {
        float4* p = reinterpret_cast<float4*>(row) + k;
        *p = map4(op, c, *p);
      } else {
        row[k] = op(c, row[k]);
      }
    }
  }
}

// vsAddB (ntensors.pas:4066) / forward_bias: x = bias[f] + x
struct BiasOp {
  const float* b;
  int64_t inc;
  struct Ch { float b; };
  __device__ Ch chan(int64_t f) const { return {b[f * inc]}; }
  __device__ float operator()(const Ch& c, float x) const { return c.b + x; }
};

// vsMulB (ntensors.pas:4112) / forward_scale: x = scale[f] * x
struct ScaleOp {
  const float* s;
  int64_t inc;
  struct Ch { float s; };
  __device__ Ch chan(int64_t f) const { return {s[f * inc]}; }
  __device__ float operator()(const Ch& c, float x) const { return c.s * x; }
};

// forwardScale then forwardBias (nbaselayer.pas:366-367), two roundings:
// x = fl(scale[f] * x) + bias[f]
struct ScaleAddOp {
  const float* s;
  const float* b;
  int64_t inc;
  struct Ch { float s, b; };
  __device__ Ch chan(int64_t f) const { return {s[f * inc], b[f * inc]}; }
  __device__ float operator()(const Ch& c, float x) const { return bn_scale_add(c.s, c.b, x); }
};

// The CPU normalize of TTensor.blockNormalize (ntensors.pas:8693-8718) with
// IEEE division: x = (x - mean[f]) / d with d = max(sqrt(var[f]), 1e-6)
// (_snormblkvv, :4357, blocks of more than one element) or d =
// sqrt(max(var[f], 1e-6)) (_snormvv, :4338, one element per channel).
// Pascal's Max(a, b) = a > b ? a : b, so a NaN variance gives d = 1e-6.
struct NormOp {
  const float* m;
  int64_t ms;
  const float* v;
  int64_t vs;
  int clampVar;
  struct Ch { float m, d; };
  __device__ Ch make(float mean, float var) const { return {mean, bn_norm_d(var, clampVar != 0)}; }
  __device__ Ch chan(int64_t f) const { return make(m[f * ms], v[f * vs]); }
  __device__ float operator()(const Ch& c, float x) const { return bn_norm(x, c.m, c.d); }
};

__device__ inline float act_fwd(float v, int act) { return bn_act(v, act); }


// Batch norm forward of TBaseLayer.batchNorm (nbaselayer.pas:335-368) and
// the layer's activation in one pass: xn = (x - mean) / d (NormOp), out =
// act(fl(scale * xn) + bias); xNorm may be NULL (inference statistics).
// Bit-identical to the reference's separate copy / normalize / copy / scale /
// bias / activate passes.
template <int VW, int ACT>
__global__ __launch_bounds__(kThreads) void bn_fwd_kernel(NormOp norm, ScaleAddOp sa, const float* __restrict__ x,
                                                          float* __restrict__ xNorm, float* __restrict__ out,
                                                          Rows g) {
  const int t = threadIdx.x, lr = t / g.cpt, lc = t - lr * g.cpt;
  if (lr >= g.rpw) return;
  for (int64_t r = static_cast<int64_t>(blockIdx.x) * g.rpw + lr; r < g.rows;
       r += static_cast<int64_t>(gridDim.x) * g.rpw) {
    const int64_t f = r % g.nb;
    const NormOp::Ch cn = norm.chan(f);
    const ScaleAddOp::Ch cs = sa.chan(f);
    const int64_t base = r * g.block;
    for (int64_t k = lc; k < g.cpr; k += g.cpt) {
      if constexpr (VW == 4) {
        const float4 n = map4(norm, cn, reinterpret_cast<const float4*>(x + base)[k]);
        if (xNorm) reinterpret_cast<float4*>(xNorm + base)[k] = n;
        const float4 o = map4(sa, cs, n);
        reinterpret_cast<float4*>(out + base)[k] =
            make_float4(act_fwd(o.x, ACT), act_fwd(o.y, ACT), act_fwd(o.z, ACT), act_fwd(o.w, ACT));
      } else {
        const float n = norm(cn, x[base + k]);
        if (xNorm) xNorm[base + k] = n;
        out[base + k] = act_fwd(sa(cs, n), ACT);
      }
    }
  }
}

// bn_fwd_kernel followed by the 2x2 / stride 2 maxpool of its output in one
// pass (the config-3 blocks: conv, batch norm, leaky, maxpool): a thread
// takes two rows of four pixels of one plane, writes their x_norm and out as
// bn_fwd_kernel does, then the two windows' max and global int64 index
// exactly as the maxpool kernels scan them (rows, then columns, strict '>'
// from -MaxSingle).  W % 4 == 0, H and W even, 16-byte aligned tensors.
// STATS: the batch statistics' final step is taken here (tnh_bn_statistics'
// partials in sp, P <= 64): the workgroup forms the mean and variance of the
// planes its threads touch (at most kStatPlanes; one unit per thread, grid
// = total / kThreads), the one holding a channel's image-0 plane stores
// them.
constexpr int kStatPlanes = 64;
template <int ACT, bool STATS>
__global__ __launch_bounds__(kThreads) void bn_fwd_pool2_kernel(NormOp norm, ScaleAddOp sa, int64_t total, int64_t C,
                                                                int64_t H, int64_t W, const float* __restrict__ x,
                                                                float* __restrict__ xNorm, float* __restrict__ out,
                                                                float* __restrict__ pooled,
                                                                int64_t* __restrict__ idx, StatParts sp) {
  const int64_t OH = H / 2, OW2 = W / 4;
  __shared__ float sM[STATS ? kStatPlanes : 1], sV[STATS ? kStatPlanes : 1];
  int64_t pA = 0;
  if constexpr (STATS) {
    const int64_t u0 = blockIdx.x * int64_t(kThreads);
    const int64_t upp = OH * OW2;  // units per plane
    const int64_t u1 = (u0 + kThreads < total ? u0 + kThreads : total) - 1;
    pA = u0 / upp;
    const int nP = static_cast<int>(u1 / upp - pA + 1);
    // wave w takes planes w, w + 4, ...: the loads of up to four, then
    // their arithmetic
    constexpr int kW = kThreads / 64;
    for (int k0 = threadIdx.x >> 6; k0 < nP; k0 += 4 * kW) {
      float ts[4], tq[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        ts[j] = tq[j] = 0.f;
        const int k = k0 + j * kW;
        if (k < nP) sp.lanes((pA + k) % C, ts[j], tq[j]);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int k = k0 + j * kW;
        if (k < nP) {
          const int64_t plane = pA + k;
          float m, v;
          sp.finish_lanes(plane % C, plane < C, ts[j], tq[j], m, v);
          if ((threadIdx.x & 63) == 0) {
            sM[k] = m;
            sV[k] = v;
          }
        }
      }
    }
    __syncthreads();
  }
  for (int64_t t = blockIdx.x * int64_t(kThreads) + threadIdx.x; t < total; t += int64_t(gridDim.x) * kThreads) {
    const int64_t jp = t % OW2, r = t / OW2;  // r = plane*OH + i
    const int64_t i = r % OH, plane = r / OH;
    const int64_t f = plane % C;
    NormOp::Ch cn;
    if constexpr (STATS)
      cn = norm.make(sM[plane - pA], sV[plane - pA]);
    else
      cn = norm.chan(f);
    const ScaleAddOp::Ch cs = sa.chan(f);
    const int64_t x0 = 4 * jp;
    const int64_t row0 = (plane * H + 2 * i) * W;
    float a[8];
#pragma unroll
    for (int n = 0; n < 2; ++n) {
      const int64_t e = row0 + n * W + x0;
      const float4 nv = map4(norm, cn, *reinterpret_cast<const float4*>(x + e));
      if (xNorm) *reinterpret_cast<float4*>(xNorm + e) = nv;
      const float4 o = map4(sa, cs, nv);
      const float4 y = make_float4(act_fwd(o.x, ACT), act_fwd(o.y, ACT), act_fwd(o.z, ACT), act_fwd(o.w, ACT));
      if (out) *reinterpret_cast<float4*>(out + e) = y;
      a[4 * n] = y.x;
      a[4 * n + 1] = y.y;
      a[4 * n + 2] = y.z;
      a[4 * n + 3] = y.w;
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
            mi = row0 + n * W + x0 + 2 * h + c;
          }
        }
      m[h] = mx;
      k[h] = mi;
    }
    const int64_t o = r * (2 * OW2) + 2 * jp;
    *reinterpret_cast<float2*>(pooled + o) = make_float2(m[0], m[1]);
    if (idx) {
      idx[o] = k[0];
      idx[o + 1] = k[1];
    }
  }
}

// bn_fwd_kernel followed by the average of each output plane (the last
// conv block of a classifier before its average pool): one wave per
// (image, channel) plane of hw <= 64 elements, one element per lane, the
// plane's x_norm and out written as bn_fwd_kernel writes them, then
// avgpool_fwd_kernel's wave tree over the out values.  STATS: each wave
// forms its plane's mean and variance from the statistics' partials (the
// final step, stored by the channel's image-0 plane).
template <int ACT, bool STATS>
__global__ __launch_bounds__(kThreads) void bn_fwd_avg_kernel(NormOp norm, ScaleAddOp sa, int64_t planes, int64_t C,
                                                              int64_t hw, const float* __restrict__ x,
                                                              float* __restrict__ xNorm, float* __restrict__ out,
                                                              float* __restrict__ avg, StatParts sp) {
  const int lane = threadIdx.x & 63;
  const int64_t r = static_cast<int64_t>(blockIdx.x) * (kThreads / 64) + (threadIdx.x >> 6);
  if (r >= planes) return;  // whole waves
  const int64_t f = r % C;
  const float xe = lane < hw ? x[r * hw + lane] : 0.f;
  NormOp::Ch cn;
  if constexpr (STATS) {  // P <= 64
    float ts, tq, m, v;
    sp.lanes(f, ts, tq);
    sp.finish_lanes(f, r < C, ts, tq, m, v);
    cn = norm.make(m, v);
  } else {
    cn = norm.chan(f);
  }
  const ScaleAddOp::Ch cs = sa.chan(f);
  float s = 0.f;
  if (lane < hw) {
    const int64_t e = r * hw + lane;
    const float n = norm(cn, xe);
    if (xNorm) xNorm[e] = n;
    const float o = act_fwd(sa(cs, n), ACT);
    if (out) out[e] = o;
    s = s + o;
  }
  for (int off = 32; off > 0; off >>= 1) s = s + __shfl_down(s, off, 64);
  if (lane == 0) avg[r] = s / static_cast<float>(hw);
}

// Launches op over [groups][nb][block] at dst (n floats).
template <class Op>
int launch_rows(Op op, float* dst, int64_t n, int64_t block, int64_t nb, hipStream_t s, const char* name) {
  if (block % 4 == 0 && al16(dst)) {
    const Rows g = make_rows(n, block, nb, 4);
    hipLaunchKernelGGL((rows_kernel<4, Op>), dim3(grid_rows(g)), dim3(kThreads), 0, s, op, dst, g);
  } else {
    const Rows g = make_rows(n, block, nb, 1);
    hipLaunchKernelGGL((rows_kernel<1, Op>), dim3(grid_rows(g)), dim3(kThreads), 0, s, op, dst, g);
  }
  return launch_status(name);
}

__global__ void activate_kernel(float* x, int64_t n, int act) {
  GRID_STRIDE(i, n) x[i] = act_fwd(x[i], act);
}

// 16 bytes per thread (n4 float4s at a 16-byte aligned base)
template <int ACT>
__global__ void activate4_kernel(float4* x, int64_t n4) {
  GRID_STRIDE(i, n4) {
    const float4 v = x[i];
    x[i] = make_float4(act_fwd(v.x, ACT), act_fwd(v.y, ACT), act_fwd(v.z, ACT), act_fwd(v.w, ACT));
  }
}

__device__ inline float act_grad(float v, int act) {
  if (act == TNH_AC_LEAKY) return v > 0.f ? 1.f : 0.1f;
  if (act == TNH_AC_LOGISTIC) return (1.f - v) * v;
  return 1.f;
}

template <int ACT>
__global__ void derive4_kernel(const float4* x, int64_t n4, float4* delta) {
  GRID_STRIDE(i, n4) {
    const float4 v = x[i];
    const float4 d = delta[i];
    delta[i] = make_float4(d.x * act_grad(v.x, ACT), d.y * act_grad(v.y, ACT), d.z * act_grad(v.z, ACT),
                           d.w * act_grad(v.w, ACT));
  }
}

// gradient_array: leaky_gradient (nactivation.pas:472-476); logistic y(1-y)
__global__ void derive_kernel(const float* x, int64_t n, int act, float* delta) {
  GRID_STRIDE(i, n) delta[i] = delta[i] * act_grad(x[i], act);
}

__global__ void addvv_kernel(int64_t n, const float* a, int64_t ia, const float* b, int64_t ib, float* c, int64_t ic) {
  GRID_STRIDE(i, n) c[i * ic] = a[i * ia] + b[i * ib];
}

// contiguous shortcut add with 16-byte accesses (n % 4 == 0, aligned)
__global__ void addvv4_kernel(int64_t n4, const float4* a, const float4* b, float4* c) {
  GRID_STRIDE(i, n4) {
    const float4 x = a[i], y = b[i];
    c[i] = make_float4(x.x + y.x, x.y + y.y, x.z + y.z, x.w + y.w);
  }
}

// cblas_saxpy -> saxpy_avx2 (ntensors.pas:1308-1436): one fused multiply-add
// per element, y = fma(a, x, y)
__global__ void axpy_kernel(int64_t n, float a, const float* x, int64_t ix, float* y, int64_t iy) {
  GRID_STRIDE(i, n) y[i * iy] = fmaf(a, x[i * ix], y[i * iy]);
}

__global__ void scale_kernel(int64_t n, float a, float* x, int64_t stride) {
  GRID_STRIDE(i, n) x[i * stride] = a * x[i * stride];
}

__global__ void fill_kernel(int64_t n, float* x, float v, int64_t stride) {
  GRID_STRIDE(i, n) x[i * stride] = v;
}

// contiguous, 16-byte aligned, N % 4 == 0: one 16-byte store per element quad
__global__ void fill4_kernel(int64_t n4, float4* x, float v) {
  GRID_STRIDE(i, n4) x[i] = float4{v, v, v, v};
}

__global__ void copy_kernel(int64_t n, const float* s, int64_t is, float* d, int64_t id) {
  GRID_STRIDE(i, n) d[i * id] = s[i * is];
}

__global__ void copy4_kernel(int64_t n4, const float4* s, float4* d) {
  GRID_STRIDE(i, n4) d[i] = s[i];
}

struct RouteArgs {
  const float* src[8];
  int64_t size[8];
  int64_t prefix[9];  // prefix[i] = sum of size[0..i)
  int n;
};

// dst[b][prefix[i] + j] = src_i[b][j]; one grid row per image
__global__ void route_kernel(RouteArgs r, float* dst, int64_t perImage) {
  const int64_t b = blockIdx.y;
  float* d = dst + b * perImage;
  GRID_STRIDE(e, perImage) {
    int i = 0;
    while (i + 1 < r.n && e >= r.prefix[i + 1]) ++i;
    const int64_t j = e - r.prefix[i];
    d[e] = r.src[i][b * r.size[i] + j];
  }
}

__global__ void yolo_kernel(int64_t total, int64_t HW, int64_t entries, const float* in, float* out) {
  GRID_STRIDE(e, total) {
    const int64_t entry = (e / HW) % entries;  // channel within the anchor group
    const float v = in[e];
    out[e] = yolo_entry(v, static_cast<int>(entry));
  }
}

// TYoloLayer.forward on a channels-last head (pixel stride inPix) into the
// NCHW head layout [b][ch][y][x] the detection decoder reads: 32 pixels x 32
// channels per tile through LDS, so the reads run along channels and the
// writes along pixels; per element the same operation as yolo_kernel.
// The four loads of a thread are issued unconditionally (clamped to the
// tensor) before any is used, and the entry index is 32-bit arithmetic
// (HW, CH < 2^31 checked by the host).
__global__ __launch_bounds__(256) void yolo_nhwc_kernel(int HW, int CH, int entries, const float* __restrict__ in,
                                                        int64_t inPix, float* __restrict__ out) {
  __shared__ float tile[32][33];
  const int64_t b = blockIdx.z;
  const int p0 = blockIdx.x * 32, c0 = blockIdx.y * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 8 rows of 32
  const float* src = in + b * HW * inPix;
  float v[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int p = min(p0 + ty + 8 * k, HW - 1), c = min(c0 + tx, CH - 1);
    v[k] = src[static_cast<int64_t>(p) * inPix + c];
  }
#pragma unroll
  for (int k = 0; k < 4; ++k) tile[ty + 8 * k][tx] = v[k];
  __syncthreads();
  float* dst = out + b * CH * HW;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int c = c0 + ty + 8 * k, p = p0 + tx;
    if (c < CH && p < HW) {
      const float x = tile[tx][ty + 8 * k];
      const int entry = c % entries;
      dst[static_cast<int64_t>(c) * HW + p] = yolo_entry(x, entry);
    }
  }
}

// dst[p*dstPix + c] = src[p*srcPix + c] for c < C: a channel slice copied
// between channels-last tensors (a route input that cannot live in place).
__global__ void copy_channels_kernel(int64_t total, int64_t C, const float* src, int64_t srcPix, float* dst,
                                     int64_t dstPix) {
  GRID_STRIDE(e, total) {
    const int64_t p = e / C, c = e - p * C;
    dst[p * dstPix + c] = src[p * srcPix + c];
  }
}

}  // namespace
}  // namespace tnh

using namespace tnh;

extern "C" int32_t tnh_forward_bias(int64_t dstSize, float* dst, int64_t offset, int64_t srcSize, const float* src,
                                    int64_t incb, int64_t batch) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(dstSize >= 0 && srcSize > 0 && batch > 0 && offset >= 0, "forward_bias: bad sizes");
  if (dstSize == 0) return TNH_OK;
  TNH_ARG(dst && src, "forward_bias: NULL buffer");
  const int64_t block = dstSize / (srcSize * batch);
  TNH_ARG(block * srcSize * batch == dstSize, "forward_bias: sizes do not align");
  return launch_rows(BiasOp{src, incb}, dst + offset, dstSize, block, srcSize, cx->stream, "rows_kernel<bias>");
}

extern "C" int32_t tnh_forward_scale(int64_t dstSize, float* dst, int64_t offset, int64_t scaleSize,
                                     const float* scale, int64_t incb, int64_t batch) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(dstSize >= 0 && scaleSize > 0 && batch > 0 && offset >= 0, "forward_scale: bad sizes");
  if (dstSize == 0) return TNH_OK;
  TNH_ARG(dst && scale, "forward_scale: NULL buffer");
  const int64_t block = dstSize / (scaleSize * batch);
  TNH_ARG(block * scaleSize * batch == dstSize, "forward_scale: sizes do not align");
  return launch_rows(ScaleOp{scale, incb}, dst + offset, dstSize, block, scaleSize, cx->stream,
                     "rows_kernel<scale>");
}

extern "C" int32_t tnh_activate(int64_t N, float* x, int64_t offset, int32_t act) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(N >= 0 && offset >= 0, "activate: bad size");
  TNH_ARG(act == TNH_AC_LINEAR || act == TNH_AC_LEAKY || act == TNH_AC_LOGISTIC,
          "activate: unsupported activation %d", act);
  if (N == 0 || act == TNH_AC_LINEAR) return TNH_OK;  // acLINEAR: no launch (nncuda.pas:533)
  TNH_ARG(x != nullptr, "activate: NULL buffer");
  float* p = x + offset;
  if (N % 4 == 0 && al16(p)) {
    float4* p4 = reinterpret_cast<float4*>(p);
    if (act == TNH_AC_LEAKY)
      hipLaunchKernelGGL(activate4_kernel<TNH_AC_LEAKY>, dim3(grid_for(N / 4)), dim3(kThreads), 0, cx->stream, p4,
                         N / 4);
    else
      hipLaunchKernelGGL(activate4_kernel<TNH_AC_LOGISTIC>, dim3(grid_for(N / 4)), dim3(kThreads), 0, cx->stream, p4,
                         N / 4);
    return launch_status("activate4_kernel");
  }
  hipLaunchKernelGGL(activate_kernel, dim3(grid_for(N)), dim3(kThreads), 0, cx->stream, p, N, act);
  return launch_status("activate_kernel");
}

extern "C" int32_t tnh_derive(int64_t N, const float* x, int64_t offset, int32_t act, float* delta) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(N >= 0 && offset >= 0, "derive: bad size");
  TNH_ARG(act == TNH_AC_LINEAR || act == TNH_AC_LEAKY || act == TNH_AC_LOGISTIC, "derive: unsupported activation %d",
          act);
  if (N == 0 || act == TNH_AC_LINEAR) return TNH_OK;
  TNH_ARG(x && delta, "derive: NULL buffer");
  const float* xp = x + offset;
  if (N % 4 == 0 && al16(xp) && al16(delta)) {
    const float4* x4 = reinterpret_cast<const float4*>(xp);
    float4* d4 = reinterpret_cast<float4*>(delta);
    if (act == TNH_AC_LEAKY)
      hipLaunchKernelGGL(derive4_kernel<TNH_AC_LEAKY>, dim3(grid_for(N / 4)), dim3(kThreads), 0, cx->stream, x4, N / 4,
                         d4);
    else
      hipLaunchKernelGGL(derive4_kernel<TNH_AC_LOGISTIC>, dim3(grid_for(N / 4)), dim3(kThreads), 0, cx->stream, x4,
                         N / 4, d4);
    return launch_status("derive4_kernel");
  }
  hipLaunchKernelGGL(derive_kernel, dim3(grid_for(N)), dim3(kThreads), 0, cx->stream, xp, N, act, delta);
  return launch_status("derive_kernel");
}

extern "C" int32_t tnh_addvv(int64_t N, const float* src1, int64_t src1Offset, int64_t inca, const float* src2,
                             int64_t src2Offset, int64_t incb, float* dst, int64_t dstOffset, int64_t incc) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(N >= 0, "addvv: bad size");
  if (N == 0) return TNH_OK;
  TNH_ARG(src1 && src2 && dst, "addvv: NULL buffer");
  const float* a = src1 + src1Offset;
  const float* b = src2 + src2Offset;
  float* c = dst + dstOffset;
  if (inca == 1 && incb == 1 && incc == 1 && N % 4 == 0 && al16(a) && al16(b) && al16(c)) {
    hipLaunchKernelGGL(addvv4_kernel, dim3(grid_for(N / 4)), dim3(kThreads), 0, cx->stream, N / 4,
                       reinterpret_cast<const float4*>(a), reinterpret_cast<const float4*>(b),
                       reinterpret_cast<float4*>(c));
    return launch_status("addvv4_kernel");
  }
  hipLaunchKernelGGL(addvv_kernel, dim3(grid_for(N)), dim3(kThreads), 0, cx->stream, N, a, inca, b, incb, c, incc);
  return launch_status("addvv_kernel");
}

extern "C" int32_t tnh_axpy(int64_t N, float a, const float* x, int64_t xOffset, int64_t incx, float* y,
                            int64_t yOffset, int64_t incy) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(N >= 0, "axpy: bad size");
  if (N == 0) return TNH_OK;
  TNH_ARG(x && y, "axpy: NULL buffer");
  hipLaunchKernelGGL(axpy_kernel, dim3(grid_for(N)), dim3(kThreads), 0, cx->stream, N, a, x + xOffset, incx,
                     y + yOffset, incy);
  return launch_status("axpy_kernel");
}

extern "C" int32_t tnh_scale(int64_t N, float a, float* x, int64_t stride) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(N >= 0, "scale: bad size");
  if (N == 0) return TNH_OK;
  TNH_ARG(x != nullptr, "scale: NULL buffer");
  hipLaunchKernelGGL(scale_kernel, dim3(grid_for(N)), dim3(kThreads), 0, cx->stream, N, a, x, stride);
  return launch_status("scale_kernel");
}

extern "C" int32_t tnh_fill(int64_t N, float* x, int64_t offset, float val, int64_t stride) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(N >= 0 && offset >= 0, "fill: bad size");
  if (N == 0) return TNH_OK;
  TNH_ARG(x != nullptr, "fill: NULL buffer");
  float* d = x + offset;
  if (stride == 1 && N % 4 == 0 && al16(d)) {
    hipLaunchKernelGGL(fill4_kernel, dim3(grid_for(N / 4)), dim3(kThreads), 0, cx->stream, N / 4,
                       reinterpret_cast<float4*>(d), val);
    return launch_status("fill4_kernel");
  }
  hipLaunchKernelGGL(fill_kernel, dim3(grid_for(N)), dim3(kThreads), 0, cx->stream, N, d, val, stride);
  return launch_status("fill_kernel");
}

extern "C" int32_t tnh_copy(int64_t N, const float* src, int64_t srcOffset, int64_t inca, float* dst,
                            int64_t dstOffset, int64_t incb) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(N >= 0, "copy: bad size");
  if (N == 0) return TNH_OK;
  TNH_ARG(src && dst, "copy: NULL buffer");
  const float* s = src + srcOffset;
  float* d = dst + dstOffset;
  if (inca == 1 && incb == 1 && N % 4 == 0 && al16(s) && al16(d)) {
    hipLaunchKernelGGL(copy4_kernel, dim3(grid_for(N / 4)), dim3(kThreads), 0, cx->stream, N / 4,
                       reinterpret_cast<const float4*>(s), reinterpret_cast<float4*>(d));
    return launch_status("copy4_kernel");
  }
  hipLaunchKernelGGL(copy_kernel, dim3(grid_for(N)), dim3(kThreads), 0, cx->stream, N, s, inca, d, incb);
  return launch_status("copy_kernel");
}

extern "C" int32_t tnh_route(int64_t batch, int32_t n, const float* const* srcs, const int64_t* sizes, float* dst) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(batch >= 0 && batch <= 65535 && n >= 1 && n <= 8, "route: bad batch/inputs");
  TNH_ARG(srcs && sizes && dst, "route: NULL argument");
  RouteArgs r{};
  r.n = n;
  r.prefix[0] = 0;
  for (int i = 0; i < n; ++i) {
    TNH_ARG(srcs[i] && sizes[i] > 0, "route: input %d empty", i);
    r.src[i] = srcs[i];
    r.size[i] = sizes[i];
    r.prefix[i + 1] = r.prefix[i] + sizes[i];
  }
  if (batch == 0) return TNH_OK;
  const int64_t per = r.prefix[n];
  hipLaunchKernelGGL(route_kernel, dim3(grid_for(per), (unsigned)batch), dim3(kThreads), 0, cx->stream, r, dst, per);
  return launch_status("route_kernel");
}

extern "C" int32_t tnh_yolo_fwd(int64_t batch, int64_t n, int64_t classes, int64_t h, int64_t w, const float* in,
                                float* out) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(batch >= 0 && n > 0 && classes >= 0 && h > 0 && w > 0, "yolo_fwd: bad sizes");
  TNH_ARG(in && out, "yolo_fwd: NULL buffer");
  const int64_t total = batch * n * (classes + 5) * h * w;
  if (total == 0) return TNH_OK;
  hipLaunchKernelGGL(yolo_kernel, dim3(grid_for(total)), dim3(kThreads), 0, cx->stream, total, h * w, classes + 5, in,
                     out);
  return launch_status("yolo_kernel");
}

extern "C" int32_t tnh_yolo_fwd_nhwc(int64_t batch, int64_t n, int64_t classes, int64_t h, int64_t w,
                                     const float* in, int64_t inOff, int64_t inPix, float* out) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(batch >= 0 && n > 0 && classes >= 0 && h > 0 && w > 0, "yolo_fwd_nhwc: bad sizes");
  TNH_ARG(in && out && inOff >= 0, "yolo_fwd_nhwc: NULL buffer or negative offset");
  const int64_t CH = n * (classes + 5), HW = h * w;
  TNH_ARG(inPix >= CH, "yolo_fwd_nhwc: inPix %lld < %lld channels", (long long)inPix, (long long)CH);
  TNH_ARG(batch < 65536 && HW <= INT32_MAX - 32 && (CH + 31) / 32 < 65536, "yolo_fwd_nhwc: grid too large");
  if (batch == 0) return TNH_OK;
  const dim3 grid(static_cast<unsigned>((HW + 31) / 32), static_cast<unsigned>((CH + 31) / 32),
                  static_cast<unsigned>(batch));
  hipLaunchKernelGGL(yolo_nhwc_kernel, grid, dim3(256), 0, cx->stream, static_cast<int>(HW), static_cast<int>(CH),
                     static_cast<int>(classes + 5), in + inOff, inPix, out);
  return launch_status("yolo_nhwc_kernel");
}

extern "C" int32_t tnh_copy_channels(int64_t pixels, int64_t C, const float* src, int64_t srcOff, int64_t srcPix,
                                     float* dst, int64_t dstOff, int64_t dstPix) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(pixels >= 0 && C >= 0 && srcPix >= C && dstPix >= C && srcOff >= 0 && dstOff >= 0,
          "copy_channels: bad sizes");
  const int64_t total = pixels * C;
  if (total == 0) return TNH_OK;
  TNH_ARG(src && dst, "copy_channels: NULL buffer");
  hipLaunchKernelGGL(copy_channels_kernel, dim3(grid_for(total)), dim3(kThreads), 0, cx->stream, total, C,
                     src + srcOff, srcPix, dst + dstOff, dstPix);
  return launch_status("copy_channels_kernel");
}

extern "C" int32_t tnh_bn_normalize(int64_t dstSize, float* x, int64_t offset, int64_t N, const float* mean,
                                    const float* variance, int64_t batch) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(dstSize >= 0 && N > 0 && batch > 0 && offset >= 0, "bn_normalize: bad sizes");
  if (dstSize == 0) return TNH_OK;
  TNH_ARG(x && mean && variance, "bn_normalize: NULL buffer");
  const int64_t block = dstSize / (N * batch);
  TNH_ARG(block * N * batch == dstSize, "bn_normalize: sizes do not align");
  return launch_rows(NormOp{mean, 1, variance, 1, block == 1}, x + offset, dstSize, block, N, cx->stream,
                     "rows_kernel<normalize>");
}

extern "C" int32_t tnh_normalize(int64_t srcSize, int64_t dstSize, int64_t groups, const float* means,
                                 int64_t meansStride, const float* vars, int64_t varsStride, float* dst,
                                 int64_t dstOffset) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(srcSize > 0 && dstSize >= 0 && groups > 0 && dstOffset >= 0 && meansStride >= 0 && varsStride >= 0,
          "normalize: bad sizes");
  if (dstSize == 0) return TNH_OK;
  TNH_ARG(means && vars && dst, "normalize: NULL buffer");
  const int64_t block = dstSize / (srcSize * groups);
  TNH_ARG(block > 0 && block * srcSize * groups == dstSize, "normalize: sizes do not align");
  return launch_rows(NormOp{means, meansStride, vars, varsStride, block == 1}, dst + dstOffset, dstSize, block,
                     srcSize, cx->stream, "rows_kernel<normalize>");
}

extern "C" int32_t tnh_forward_scale_add(int64_t dstSize, float* dst, int64_t offset, int64_t scaleSize,
                                         const float* scales, const float* biases, int64_t incb, int64_t batch) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(dstSize >= 0 && scaleSize > 0 && batch > 0 && offset >= 0, "forward_scale_add: bad sizes");
  if (dstSize == 0) return TNH_OK;
  TNH_ARG(dst && scales && biases, "forward_scale_add: NULL buffer");
  const int64_t block = dstSize / (scaleSize * batch);
  TNH_ARG(block > 0 && block * scaleSize * batch == dstSize, "forward_scale_add: sizes do not align");
  return launch_rows(ScaleAddOp{scales, biases, incb}, dst + offset, dstSize, block, scaleSize, cx->stream,
                     "rows_kernel<scale_add>");
}

extern "C" int32_t tnh_bn_forward(int64_t dstSize, int64_t N, int64_t batch, const float* x, float* xNorm,
                                  float* out, const float* mean, const float* variance, const float* scales,
                                  const float* biases, int32_t act) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(dstSize >= 0 && N > 0 && batch > 0, "bn_forward: bad sizes");
  TNH_ARG(act == TNH_AC_LINEAR || act == TNH_AC_LEAKY || act == TNH_AC_LOGISTIC, "bn_forward: activation %d", act);
  if (dstSize == 0) return TNH_OK;
  TNH_ARG(x && out && mean && variance && scales && biases, "bn_forward: NULL buffer");
  const int64_t block = dstSize / (N * batch);
  TNH_ARG(block > 0 && block * N * batch == dstSize, "bn_forward: sizes do not align");
  const NormOp norm{mean, 1, variance, 1, block == 1};
  const ScaleAddOp sa{scales, biases, 1};
  const bool v4 = block % 4 == 0 && al16(x) && al16(out) && (!xNorm || al16(xNorm));
  const Rows g = make_rows(dstSize, block, N, v4 ? 4 : 1);
  auto go = [&](auto vw, auto ac) {
    constexpr int VW = decltype(vw)::value, ACT = decltype(ac)::value;
    hipLaunchKernelGGL((bn_fwd_kernel<VW, ACT>), dim3(grid_rows(g)), dim3(kThreads), 0, cx->stream, norm, sa, x,
                       xNorm, out, g);
  };
  using L = std::integral_constant<int, TNH_AC_LEAKY>;
  using G = std::integral_constant<int, TNH_AC_LOGISTIC>;
  using I = std::integral_constant<int, TNH_AC_LINEAR>;
  using V4 = std::integral_constant<int, 4>;
  using V1 = std::integral_constant<int, 1>;
  if (v4) {
    if (act == TNH_AC_LEAKY) go(V4{}, L{}); else if (act == TNH_AC_LOGISTIC) go(V4{}, G{}); else go(V4{}, I{});
  } else {
    if (act == TNH_AC_LEAKY) go(V1{}, L{}); else if (act == TNH_AC_LOGISTIC) go(V1{}, G{}); else go(V1{}, I{});
  }
  return launch_status("bn_fwd_kernel");
}

namespace {

// tnh_bn_forward_maxpool; sp non-NULL: the statistics' final step in the
// same launch (the caller launched their partials)
int bn_forward_maxpool_impl(int64_t batch, int64_t N, int64_t h, int64_t w, const float* x,
                            float* xNorm, float* out, const float* mean, const float* variance, const float* scales,
                            const float* biases, int32_t act, float* pooled, int64_t* indexes, const StatParts* sp) {
  TNH_REQUIRE_CTX(cx);
  const int64_t total = batch * N * (h / 2) * (w / 4);  // (plane, output row, pair of output columns)
  const NormOp norm{mean, 1, variance, 1, h * w == 1};
  const ScaleAddOp sa{scales, biases, 1};
  const int64_t blocks = (total + kThreads - 1) / kThreads;
  const dim3 grid(static_cast<unsigned>(sp ? blocks : (blocks < 65536 ? blocks : 65536)));
  const StatParts none{};
  auto go = [&](auto ac, auto st) {
    constexpr int ACT = decltype(ac)::value;
    constexpr bool ST = decltype(st)::value;
    hipLaunchKernelGGL((bn_fwd_pool2_kernel<ACT, ST>), grid, dim3(kThreads), 0, cx->stream, norm, sa, total, N, h, w,
                       x, xNorm, out, pooled, indexes, sp ? *sp : none);
  };
  using L = std::integral_constant<int, TNH_AC_LEAKY>;
  using G = std::integral_constant<int, TNH_AC_LOGISTIC>;
  using I = std::integral_constant<int, TNH_AC_LINEAR>;
  using Y = std::true_type;
  using Nn = std::false_type;
  if (sp) {
    if (act == TNH_AC_LEAKY) go(L{}, Y{}); else if (act == TNH_AC_LOGISTIC) go(G{}, Y{}); else go(I{}, Y{});
  } else {
    if (act == TNH_AC_LEAKY) go(L{}, Nn{}); else if (act == TNH_AC_LOGISTIC) go(G{}, Nn{}); else go(I{}, Nn{});
  }
  if (indexes) pool_remember_2x2(indexes, batch, N, h, w);
  return launch_status("bn_fwd_pool2_kernel");
}

int bn_forward_avgpool_impl(int64_t batch, int64_t N, int64_t hw, const float* x, float* xNorm, float* out,
                            const float* mean, const float* variance, const float* scales, const float* biases,
                            int32_t act, float* avg, const StatParts* sp) {
  TNH_REQUIRE_CTX(cx);
  const int64_t planes = batch * N;
  const NormOp norm{mean, 1, variance, 1, hw == 1};
  const ScaleAddOp sa{scales, biases, 1};
  const dim3 grid(static_cast<unsigned>((planes + kThreads / 64 - 1) / (kThreads / 64)));
  const StatParts none{};
  auto go = [&](auto ac, auto st) {
    constexpr int ACT = decltype(ac)::value;
    constexpr bool ST = decltype(st)::value;
    hipLaunchKernelGGL((bn_fwd_avg_kernel<ACT, ST>), grid, dim3(kThreads), 0, cx->stream, norm, sa, planes, N, hw, x,
                       xNorm, out, avg, sp ? *sp : none);
  };
  using L = std::integral_constant<int, TNH_AC_LEAKY>;
  using G = std::integral_constant<int, TNH_AC_LOGISTIC>;
  using I = std::integral_constant<int, TNH_AC_LINEAR>;
  using Y = std::true_type;
  using Nn = std::false_type;
  if (sp) {
    if (act == TNH_AC_LEAKY) go(L{}, Y{}); else if (act == TNH_AC_LOGISTIC) go(G{}, Y{}); else go(I{}, Y{});
  } else {
    if (act == TNH_AC_LEAKY) go(L{}, Nn{}); else if (act == TNH_AC_LOGISTIC) go(G{}, Nn{}); else go(I{}, Nn{});
  }
  return launch_status("bn_fwd_avg_kernel");
}

}  // namespace

#define BN_POOL2_CHECKS(who)                                                                                         \
  TNH_ARG(batch > 0 && N > 0 && h > 0 && w > 0, who ": bad sizes");                                                  \
  TNH_ARG(act == TNH_AC_LINEAR || act == TNH_AC_LEAKY || act == TNH_AC_LOGISTIC, who ": activation %d", act);        \
  TNH_ARG(x && mean && variance && scales && biases && pooled, who ": NULL buffer");                                 \
  TNH_ARG(h % 2 == 0 && w % 4 == 0 && al16(x) && (!out || al16(out)) && (!xNorm || al16(xNorm)) &&                  \
              (reinterpret_cast<uintptr_t>(pooled) & 7) == 0 && (!indexes || al16(indexes)),                         \
          who ": needs even h, w %% 4 == 0 and aligned tensors")

#define BN_AVG_CHECKS(who)                                                                                           \
  TNH_ARG(batch > 0 && N > 0 && hw > 0 && hw <= 64, who ": bad sizes (hw <= 64)");                                   \
  TNH_ARG(act == TNH_AC_LINEAR || act == TNH_AC_LEAKY || act == TNH_AC_LOGISTIC, who ": activation %d", act);        \
  TNH_ARG(x && mean && variance && scales && biases && avg, who ": NULL buffer");                                    \
  TNH_ARG(batch * N < (int64_t(1) << 31), who ": too many planes")

extern "C" int32_t tnh_bn_forward_maxpool(int64_t batch, int64_t N, int64_t h, int64_t w, const float* x,
                                          float* xNorm, float* out, const float* mean, const float* variance,
                                          const float* scales, const float* biases, int32_t act, float* pooled,
                                          int64_t* indexes) {
  BN_POOL2_CHECKS("bn_forward_maxpool");
  return bn_forward_maxpool_impl(batch, N, h, w, x, xNorm, out, mean, variance, scales, biases,
                                 act, pooled, indexes, nullptr);
}

extern "C" int32_t tnh_bn_forward_avgpool(int64_t batch, int64_t N, int64_t hw, const float* x, float* xNorm,
                                          float* out, const float* mean, const float* variance, const float* scales,
                                          const float* biases, int32_t act, float* avg) {
  BN_AVG_CHECKS("bn_forward_avgpool");
  return bn_forward_avgpool_impl(batch, N, hw, x, xNorm, out, mean, variance, scales, biases, act, avg, nullptr);
}

extern "C" int32_t tnh_bn_train_forward_maxpool(int64_t batch, int64_t N, int64_t h, int64_t w, const float* x,
                                                float* xNorm, float* out, float* mean, float* variance,
                                                float* rollMean, float* rollVar, float momentum, const float* scales,
                                                const float* biases, int32_t act, float* pooled, int64_t* indexes) {
  BN_POOL2_CHECKS("bn_train_forward_maxpool");
  const int64_t upp = (h / 2) * (w / 4);
  const int64_t blocks = (batch * N * upp + kThreads - 1) / kThreads;
  StatParts sp;
  if (int st = bn_stat_partials(N, h * w, batch, x, mean, variance, rollMean, rollVar, momentum, sp)) return st;
  // the planes one workgroup touches must fit its table
  if ((kThreads + upp - 1) / upp + 1 > kStatPlanes || sp.P > 64 || blocks >= (int64_t(1) << 31)) {
    // ... else the final step in its own launch
    if (int st = bn_stat_final(N, sp)) return st;
    return bn_forward_maxpool_impl(batch, N, h, w, x, xNorm, out, mean, variance, scales,
                                   biases, act, pooled, indexes, nullptr);
  }
  return bn_forward_maxpool_impl(batch, N, h, w, x, xNorm, out, mean, variance, scales,
                                 biases, act, pooled, indexes, &sp);
}

extern "C" int32_t tnh_bn_train_forward_avgpool(int64_t batch, int64_t N, int64_t hw, const float* x, float* xNorm,
                                                float* out, float* mean, float* variance, float* rollMean,
                                                float* rollVar, float momentum, const float* scales,
                                                const float* biases, int32_t act, float* avg) {
  BN_AVG_CHECKS("bn_train_forward_avgpool");
  StatParts sp;
  if (int st = bn_stat_partials(N, hw, batch, x, mean, variance, rollMean, rollVar, momentum, sp)) return st;
  if (sp.P > 64) {  // the final step in its own launch
    if (int st = bn_stat_final(N, sp)) return st;
    return bn_forward_avgpool_impl(batch, N, hw, x, xNorm, out, mean, variance, scales, biases, act, avg, nullptr);
  }
  return bn_forward_avgpool_impl(batch, N, hw, x, xNorm, out, mean, variance, scales, biases, act, avg, &sp);
}
