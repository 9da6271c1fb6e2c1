// Training-direction kernels of the convolution path: batch-norm statistics
// and their deltas, softmax cross-entropy, average pooling, delta clamping,
// the fused SGD update and the weight-gradient GEMM of conv backward.
//
// Channel reductions run several workgroups per channel and add their
// partials in a fixed order (deterministic run to run); element-wise
// formulas follow the reference
// CPU operation order exactly (no contraction: the build uses
// -ffp-contract=off, FMAs are explicit where the reference fuses).
#include <algorithm>
#include <cmath>
#include <initializer_list>
#include <type_traits>

#include "chanstat.hpp"
#include "common.hpp"
#include "gemm_core.hpp"
#include "rows.hpp"

namespace tnh {
namespace {

constexpr int kRed = 256;  // threads per reduction workgroup
constexpr float kEps = 1e-6f;  // sEPSILON (ntensors.pas:95)

#define GRID_STRIDE(i, n) \
  for (int64_t i = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; i < (n); i += int64_t(gridDim.x) * blockDim.x)

unsigned grid_1d(int64_t n) {
  const int64_t b = (n + 255) / 256;
  return static_cast<unsigned>(b < 16384 ? (b > 0 ? b : 1) : 16384);
}

// Sum of one value per thread over a kRed-thread workgroup (fixed order).
__device__ inline float block_sum(float v, float* sh) {
  sh[threadIdx.x] = v;
  __syncthreads();
  for (int w = kRed / 2; w > 0; w >>= 1) {
    if (threadIdx.x < w) sh[threadIdx.x] = sh[threadIdx.x] + sh[threadIdx.x + w];
    __syncthreads();
  }
  const float r = sh[0];
  __syncthreads();
  return r;
}

// ---------------------------------------------------------------------------
// Channel reductions over a [groups][nch][block] view (element (b, i, k) at
// (b*nch + i)*block + k), spread over P workgroups per channel.  A
// channel's groups*block elements are cut into units (one row b, or a chunk
// of cs elements of a long row); workgroup (p, i) takes units
// [p*U/P, (p+1)*U/P) of channel i, each thread adds its elements in order
// (16 bytes at a time when the rows allow) and a fixed tree over the
// workgroup leaves one partial per workgroup in the context's reduction
// buffer.  A second kernel adds a channel's P partials in a fixed order
// (fixed_total).  Every order is fixed, so results do not vary run to run.
// ---------------------------------------------------------------------------
struct ChanSplit {
  int64_t nch, block, groups;
  int64_t cs;     // elements per unit
  int64_t kc;     // units per row
  int64_t units;  // groups * kc
  int P;          // workgroups per channel
};

// nq partial sums per workgroup; about four workgroups per CU over all
// channels, at least ~1024 elements each.  part: the current stream's
// partial-sum buffer (each stream has its own, so reductions forked onto
// several streams do not share one).
int chan_split(ChanSplit& s, float*& part, int64_t nch, int64_t block, int64_t groups, int nq, Context* cx) {
  TNH_ARG(nch * nq <= cx->redFloats, "channel reduction: %lld channels do not fit the partial-sum buffer",
          (long long)nch);
  part = reduction_buffer(cx);
  if (!part)
    return fail(TNH_ERR_OUT_OF_MEMORY,
                "channel reduction: no partial-sum buffer for this stream (the spares are taken and it cannot be "
                "allocated now; run one reduction on the stream before capturing it)");
  s.nch = nch;
  s.block = block;
  s.groups = groups;
  s.cs = block <= 4096 ? block : 4096;
  s.kc = (block + s.cs - 1) / s.cs;
  s.units = groups * s.kc;
  int64_t P = (4 * static_cast<int64_t>(cx->cu_count) + nch - 1) / nch;
  P = std::min<int64_t>(P, std::max<int64_t>(1, groups * block / 1024));
  P = std::min<int64_t>({P, s.units, cx->redFloats / (nq * nch), 4096});  // grid.y holds P
  s.P = static_cast<int>(std::max<int64_t>(P, 1));
  return TNH_OK;
}

// Sum of v[0 .. n) in a fixed order: lane l of the first wave adds v[l],
// v[l + 64], ... in turn, then a fixed tree over the 64 lanes.  Every thread
// of the workgroup calls it and gets the result; the arithmetic does not
// depend on the workgroup size.
__device__ inline float fixed_total(const float* v, int n, float* sh) {
  if (threadIdx.x < 64) {
    float t = 0.f;
    for (int k = threadIdx.x; k < n; k += 64) t = t + v[k];
    sh[threadIdx.x] = t;
  }
  __syncthreads();
  for (int w = 32; w > 0; w >>= 1) {
    if (threadIdx.x < w) sh[threadIdx.x] = sh[threadIdx.x] + sh[threadIdx.x + w];
    __syncthreads();
  }
  const float r = sh[0];
  __syncthreads();
  return r;
}

// Walks workgroup (p, i)'s units, calling op.add(acc, element index) per
// element or op.add4(acc, index of 4 elements) per 16 bytes.  Units of
// fewer than kRed chunks share a pass: thread t takes chunk t % cpt of unit
// t / cpt, so short rows (an 8x8 plane, one element per channel) keep every
// thread busy; a thread's share is fixed, so the sums are too.
template <bool VEC, class Op>
__device__ inline void chan_walk(const ChanSplit& s, int p, int64_t i, const Op& op, float* acc) {
  const int64_t u0 = s.units * p / s.P, u1 = s.units * (p + 1) / s.P;
  constexpr int V = VEC ? 4 : 1;
  const int64_t cpr = (s.cs + V - 1) / V;  // chunks of a full unit
  const int cpt = static_cast<int>(cpr < kRed ? cpr : kRed);
  const int upp = kRed / cpt;  // units per pass
  const int lu = threadIdx.x / cpt, lc = threadIdx.x - lu * cpt;
  if (lu >= upp) return;
  for (int64_t u = u0 + lu; u < u1; u += upp) {
    const int64_t b = u / s.kc, c = u - b * s.kc;
    const int64_t base = (b * s.nch + i) * s.block + c * s.cs;
    const int64_t len = std::min(s.cs, s.block - c * s.cs) / V;
    for (int64_t k = lc; k < len; k += cpt) {
      if constexpr (VEC)
        op.add4(acc, base + 4 * k);
      else
        op.add(acc, base + k);
    }
  }
}

// A reduction without a per-channel final step (the first pass of a
// two-pass statistic).
struct NoFin {
  __device__ void run(int64_t, const ChanSplit&, float*) const {}
};

// grid: (channel, workgroup of the channel); channels in x, which holds up
// to 2^31 - 1 of them.  Each workgroup stores its NQ partials; a second
// launch (chan_final_kernel) runs the channel's final step.  (A final step
// run by the channel's last-arriving workgroup, found with an arrival
// counter, was measured slower on the config-3 step: its chain of
// write-through stores, the atomic and the system-scope loads at the end of
// the launch outlasts a separate 64-thread launch.)
template <int NQ, bool VEC, class Op>
__global__ __launch_bounds__(kRed) void chan_partial_kernel(Op op, ChanSplit s, float* part) {
  __shared__ float sh[kRed];
  const int64_t i = blockIdx.x;
  const int p = blockIdx.y;
  op.begin(i, s, part, sh);
  float acc[NQ];
#pragma unroll
  for (int q = 0; q < NQ; ++q) acc[q] = 0.f;
  chan_walk<VEC>(s, p, i, op, acc);
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    const float r = block_sum(acc[q], sh);
    if (threadIdx.x == 0) part[(q * s.nch + i) * s.P + p] = r;
  }
}

// The second launch of a reduction: one 64-thread workgroup per channel
// runs the final step.
template <class Fin>
__global__ __launch_bounds__(64) void chan_final_kernel(Fin fin, ChanSplit s) {
  __shared__ float sh[64];
  fin.run(blockIdx.x, s, sh);
}

__device__ inline float4 ld4(const float* p) { return *reinterpret_cast<const float4*>(p); }

// MeansAndVars (ntensors.pas:9102-9180), first pass: sum
struct SumOp {
  const float* x;
  __device__ void begin(int64_t, const ChanSplit&, const float*, float*) {}
  __device__ void add(float* a, int64_t e) const { a[0] = a[0] + x[e]; }
  __device__ void add4(float* a, int64_t e) const {
    const float4 v = ld4(x + e);
    a[0] = a[0] + v.x;
    a[0] = a[0] + v.y;
    a[0] = a[0] + v.z;
    a[0] = a[0] + v.w;
  }
};

// second pass: residual sum of squares about the fp32 mean (the mean from
// the first pass's partials, the same fixed sum the final kernel forms)
struct RssOp {
  const float* x;
  const float* sumPart;  // [nch][P]
  float S;
  float m;
  __device__ void begin(int64_t i, const ChanSplit& s, const float*, float* sh) {
    m = fixed_total(sumPart + i * s.P, s.P, sh) / S;
  }
  __device__ void add(float* a, int64_t e) const {
    const float d = x[e] - m;
    a[0] = a[0] + d * d;
  }
  __device__ void add4(float* a, int64_t e) const {
    const float4 v = ld4(x + e);
    float d = v.x - m;
    a[0] = a[0] + d * d;
    d = v.y - m;
    a[0] = a[0] + d * d;
    d = v.z - m;
    a[0] = a[0] + d * d;
    d = v.w - m;
    a[0] = a[0] + d * d;
  }
};

// second pass of tnh_variances: residual sum of squares about the caller's
// means (TNNCuda.variances takes them as an argument, nncuda.pas:1350)
struct RssGivenOp {
  const float* x;
  const float* means;
  float m;
  __device__ void begin(int64_t i, const ChanSplit&, const float*, float*) { m = means[i]; }
  __device__ void add(float* a, int64_t e) const {
    const float d = x[e] - m;
    a[0] = a[0] + d * d;
  }
  __device__ void add4(float* a, int64_t e) const {
    const float4 v = ld4(x + e);
    float d = v.x - m;
    a[0] = a[0] + d * d;
    d = v.y - m;
    a[0] = a[0] + d * d;
    d = v.z - m;
    a[0] = a[0] + d * d;
    d = v.w - m;
    a[0] = a[0] + d * d;
  }
};

// dst[i] = (the channel's fixed-order partial total) / div
// dst[i] = (the channel's fixed-order partial total) / div
struct TotalDivFin {
  const float* part;
  float div;
  float* dst;
  __device__ void run(int64_t i, const ChanSplit& s, float* sh) const {
    const float t = fixed_total(part + i * s.P, s.P, sh);
    if (threadIdx.x == 0) dst[i] = t / div;
  }
};

// mean = sum / S and variance = residual sum / (S - 1), then the rolling
// statistics (part: [2][nch][P], the sums then the residual sums)
struct MeanVarFin {
  const float* part;
  float S;
  float* means;
  float* vars;
  float* rollMean;
  float* rollVar;
  float keep, bm;
  __device__ void run(int64_t i, const ChanSplit& s, float* sh) const {
    const float m = fixed_total(part + i * s.P, s.P, sh) / S;
    const float rss = fixed_total(part + (s.nch + i) * s.P, s.P, sh);
    if (threadIdx.x == 0) {
      const float v = rss / (S - 1.f);
      means[i] = m;
      vars[i] = v;
      if (rollMean) {  // Multiply(1 - momentum), then axpy(momentum, .) (nbaselayer.pas:352-355)
        rollMean[i] = fmaf(bm, m, keep * rollMean[i]);
        rollVar[i] = fmaf(bm, v, keep * rollVar[i]);
      }
    }
  }
};

// sMeanAndVarianceDelta (ntensors.pas:8831-8898): sum(delta) and
// sum(delta * (x - mean))
struct MvdOp {
  const float* delta;
  const float* x;
  const float* mean;
  float mu;
  __device__ void begin(int64_t i, const ChanSplit&, const float*, float*) { mu = mean[i]; }
  __device__ void add(float* a, int64_t e) const {
    const float d = delta[e];
    a[0] = a[0] + d;
    a[1] = a[1] + d * (x[e] - mu);
  }
  __device__ void add4(float* a, int64_t e) const {
    const float4 d = ld4(delta + e), v = ld4(x + e);
    a[0] = a[0] + d.x;
    a[1] = a[1] + d.x * (v.x - mu);
    a[0] = a[0] + d.y;
    a[1] = a[1] + d.y * (v.y - mu);
    a[0] = a[0] + d.z;
    a[1] = a[1] + d.z * (v.z - mu);
    a[0] = a[0] + d.w;
    a[1] = a[1] + d.w * (v.w - mu);
  }
};

struct MvdFin {
  const float* part;
  const float* variance;
  float* mean_delta;
  float* variance_delta;
  __device__ void run(int64_t i, const ChanSplit& s, float* sh) const {
    const float m = fixed_total(part + i * s.P, s.P, sh);
    const float v = fixed_total(part + (s.nch + i) * s.P, s.P, sh);
    if (threadIdx.x == 0) {
      const float vc = fmaxf(variance[i], kEps);
      mean_delta[i] = m * (-1.0f / sqrtf(vc));
      // Power(max(var, eps), -3/2) is evaluated in double and the product stored as single
      variance_delta[i] = static_cast<float>(static_cast<double>(v) * -0.5 * pow(static_cast<double>(vc), -1.5));
    }
  }
};

// The batch-norm backward's two final steps in one launch: the mean / variance
// deltas (MvdFin) and dgamma += the BnBackOp partials' total (AddFin), each
// from its own partials.
struct BnBackFin {
  MvdFin mvd;
  const float* dotPart;
  float* scaleUpdates;
  const double* vpow;  // normalize_delta_fin_kernel: BnBackOpT's Power term
  __device__ void run(int64_t i, const ChanSplit& s, float* sh) const {
    mvd.run(i, s, sh);
    const float t = fixed_total(dotPart + i * s.P, s.P, sh);
    if (threadIdx.x == 0) scaleUpdates[i] = scaleUpdates[i] + t;
  }
};

// addDots (ntensors.pas:7783-7830): sum of a*b
struct DotOp {
  const float* x;
  const float* y;
  __device__ void begin(int64_t, const ChanSplit&, const float*, float*) {}
  __device__ void add(float* a, int64_t e) const { a[0] = a[0] + x[e] * y[e]; }
  __device__ void add4(float* a, int64_t e) const {
    const float4 u = ld4(x + e), v = ld4(y + e);
    a[0] = a[0] + u.x * v.x;
    a[0] = a[0] + u.y * v.y;
    a[0] = a[0] + u.z * v.z;
    a[0] = a[0] + u.w * v.w;
  }
};

// dst[i] += the channel's total (addDots, addSums / backward_bias)
struct AddFin {
  const float* part;
  float* dst;
  __device__ void run(int64_t i, const ChanSplit& s, float* sh) const {
    const float t = fixed_total(part + i * s.P, s.P, sh);
    if (threadIdx.x == 0) dst[i] = dst[i] + t;
  }
};

// Where the layer's incoming delta comes from: the delta buffer itself, or
// the backward of the pool layer above it, formed element by element as
// that backward would leave it in the delta that TNNet zeroes before each
// pass (nnet.pas:287-294), so the buffer need not be zeroed or written first:
//   kFromMaxPool2: the 2x2 stride-2 maxpool scatter (TMaxPoolLayer.backward,
//     delta[index] += poolDelta): 0 + poolDelta[o] at the element window o's
//     index names, +0 at its other three elements;
//   kFromAvgPool: TAvgPoolLayer.backward (navgpoollayer.pas:86-100), 0 +
//     poolDelta[plane] / hw at every element of the plane.
enum DeltaSrc { kFromDelta = 0, kFromMaxPool2 = 1, kFromAvgPool = 2 };

// batchNormBack's first three steps (nbaselayer.pas:372-392) in one pass:
// DeriveArray (delta *= act'(out)), addDots (dgamma += sum x_norm * delta)
// and forwardScale (delta *= gamma), each element visited once with each
// step's own operation, so the deltas and the dot equal the three separate
// passes bit for bit.  MVD: the pass also takes MvdOp's two sums of the new
// delta (a[0], a[1]; the dot in a[2]), element by element in the order
// MvdOp's own pass over the same split adds them, so its partials are the
// same bits and its pass over delta and x is saved.
template <int SRC, bool MVD = false>
struct BnBackOpT {
  float* delta;
  const float* out;
  const float* xn;
  const float* gamma;
  int act;
  float g;
  const int64_t* pidx = nullptr;  // kFromMaxPool2: the pool's indexes
  const float* pdel = nullptr;    // the pool layer's delta
  uint32_t block = 0, w = 0;      // plane size and row width (SRC != kFromDelta)
  // non-NULL: the first workgroup of channel i also stores
  // Power(max(var[i], eps), -3/2) in double for the mean / variance delta
  // step (the one term of it that does not wait for the delta sums)
  const float* var = nullptr;
  double* vpow = nullptr;
  const float* x = nullptr;     // MVD or xn NULL: the pre-normalization input
  const float* mean = nullptr;  // MVD or xn NULL: the forward's means
  const float* varN = nullptr;  // xn NULL: the forward's variances
  bool oneElem = false;         // xn NULL: one element per channel and image
  const float* beta = nullptr;  // out NULL: the biases (out formed from x_norm)
  float mu = 0.f, nd = 1.f, bb = 0.f;
  __device__ void begin(int64_t i, const ChanSplit&, const float*, float*) {
    g = gamma[i];
    if (MVD || !xn) mu = mean[i];
    if (!xn) nd = bn_norm_d(varN[i], oneElem);  // x_norm formed as the forward formed it
    if (!out) bb = beta[i];
    if (vpow && blockIdx.y == 0 && threadIdx.x == 0)
      vpow[i] = pow(static_cast<double>(fmaxf(var[i], kEps)), -1.5);
  }
  // 2x2 window of element e (planes of h x w, h and w even)
  __device__ uint32_t win(uint32_t e) const {
    const uint32_t plane = e / block, r = e - plane * block, y = r / w, x = r - y * w;
    return plane * (block >> 2) + (y >> 1) * (w >> 1) + (x >> 1);
  }
  __device__ float src(int64_t e) const {
    if constexpr (SRC == kFromDelta) {
      return delta[e];
    } else if constexpr (SRC == kFromAvgPool) {
      return 0.f + pdel[static_cast<uint32_t>(e) / block] / static_cast<float>(block);
    } else {
      const uint32_t o = win(static_cast<uint32_t>(e));
      return pidx[o] == e ? 0.f + pdel[o] : 0.f;
    }
  }
  // four consecutive elements (e % 4 == 0; the 16-byte walk must be taken
  // exactly when tnh_bn_backward takes it, which fixes the sums' order)
  __device__ float4 src4(int64_t e) const {
    if constexpr (SRC == kFromDelta) {
      return ld4(delta + e);
    } else if constexpr (SRC == kFromAvgPool) {
      const float v = 0.f + pdel[static_cast<uint32_t>(e) / block] / static_cast<float>(block);
      return make_float4(v, v, v, v);
    } else {
      if (w & 3) return make_float4(src(e), src(e + 1), src(e + 2), src(e + 3));
      // one row, two windows
      const uint32_t o = win(static_cast<uint32_t>(e));
      const int64_t k0 = pidx[o], k1 = pidx[o + 1];
      const float p0 = 0.f + pdel[o], p1 = 0.f + pdel[o + 1];
      return make_float4(k0 == e ? p0 : 0.f, k0 == e + 1 ? p0 : 0.f, k1 == e + 2 ? p1 : 0.f, k1 == e + 3 ? p1 : 0.f);
    }
  }
  __device__ static float grad(float v, int act) {
    if (act == TNH_AC_LEAKY) return v > 0.f ? 1.f : 0.1f;
    if (act == TNH_AC_LOGISTIC) return (1.f - v) * v;
    return 1.f;
  }
  __device__ float one(float* a, float d, float o, float xnv, float xv) const {
    const float d1 = d * grad(o, act);
    constexpr int kDot = MVD ? 2 : 0;
    a[kDot] = a[kDot] + xnv * d1;
    const float r = g * d1;
    if constexpr (MVD) {  // MvdOp::add on the new delta
      a[0] = a[0] + r;
      a[1] = a[1] + r * (xv - mu);
    }
    return r;
  }
  // the forward's output formed again from x_norm (out NULL)
  __device__ float outOf(float xnv) const { return bn_act(bn_scale_add(g, bb, xnv), act); }
  __device__ void add(float* a, int64_t e) const {
    const float xv = (MVD || !xn) ? x[e] : 0.f;
    const float xnv = xn ? xn[e] : bn_norm(xv, mu, nd);
    delta[e] = one(a, src(e), out ? out[e] : outOf(xnv), xnv, xv);
  }
  __device__ void add4(float* a, int64_t e) const {
    const float4 d = src4(e);
    const float4 v = (MVD || !xn) ? ld4(x + e) : make_float4(0.f, 0.f, 0.f, 0.f);
    const float4 xv = xn ? ld4(xn + e)
                         : make_float4(bn_norm(v.x, mu, nd), bn_norm(v.y, mu, nd), bn_norm(v.z, mu, nd),
                                       bn_norm(v.w, mu, nd));
    const float4 o = out ? ld4(out + e) : make_float4(outOf(xv.x), outOf(xv.y), outOf(xv.z), outOf(xv.w));
    float4 r;
    r.x = one(a, d.x, o.x, xv.x, v.x);
    r.y = one(a, d.y, o.y, xv.y, v.y);
    r.z = one(a, d.z, o.z, xv.z, v.z);
    r.w = one(a, d.w, o.w, xv.w, v.w);
    *reinterpret_cast<float4*>(delta + e) = r;
  }
};
using BnBackOp = BnBackOpT<kFromDelta>;

bool al16p(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// Launches a channel reduction (NQ partials per workgroup) and, for a Fin
// other than NoFin, the launch of its per-channel final step.
template <int NQ, class Op, class Fin = NoFin>
int launch_partial(Context* cx, const Op& op, const ChanSplit& s, bool vec, float* part, const char* name,
                   const Fin& fin = Fin{}) {
  const dim3 grid(static_cast<unsigned>(s.nch), static_cast<unsigned>(s.P));
  if (vec)
    hipLaunchKernelGGL((chan_partial_kernel<NQ, true, Op>), grid, dim3(kRed), 0, cx->stream, op, s, part);
  else
    hipLaunchKernelGGL((chan_partial_kernel<NQ, false, Op>), grid, dim3(kRed), 0, cx->stream, op, s, part);
  if (int st = launch_status(name)) return st;
  if (std::is_same<Fin, NoFin>::value) return TNH_OK;
  hipLaunchKernelGGL((chan_final_kernel<Fin>), dim3(static_cast<unsigned>(s.nch)), dim3(64), 0, cx->stream, fin, s);
  return launch_status("chan_final_kernel");
}

// 16-byte loads are legal when every unit starts 16-byte aligned
bool chan_vec(const ChanSplit& s, std::initializer_list<const float*> ptrs) {
  if (s.block % 4 || s.cs % 4) return false;
  for (const float* p : ptrs)
    if (!al16p(p)) return false;
  return true;
}

int means_vars_impl(int64_t srcSize, int64_t dstSize, int64_t groups, const float* src, int64_t offset,
                    float* means, float* vars, float* rollMean, float* rollVar, float momentum) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(dstSize > 0 && groups > 0 && srcSize > 0 && offset >= 0, "means_vars: bad sizes");
  TNH_ARG(src && means && vars, "means_vars: NULL buffer");
  const int64_t block = srcSize / (dstSize * groups);
  TNH_ARG(block * dstSize * groups == srcSize && groups * block > 1, "means_vars: sizes do not align");
  ChanSplit s;
  float* red = nullptr;
  if (int st = chan_split(s, red, dstSize, block, groups, 2, cx)) return st;
  const float* x = src + offset;
  const bool vec = chan_vec(s, {x});
  float* sumPart = red;
  float* rssPart = red + dstSize * s.P;
  const float S = static_cast<float>(groups * block);
  if (int st = launch_partial<1>(cx, SumOp{x}, s, vec, sumPart, "chan_partial_kernel<sum>")) return st;
  const float keep = 1.0f - momentum;
  return launch_partial<1>(cx, RssOp{x, sumPart, S, 0.f}, s, vec, rssPart, "chan_partial_kernel<rss>",
                           MeanVarFin{red, S, means, vars, rollMean, rollVar, keep, momentum});
}

// sNormalizeDelta (ntensors.pas:8900-8960), element order of
// sNormalizeDelta_pas/_avx: d / std + ((x - mean) * vd + md), with the
// channel's md = mean_delta / bs, vd = 2 * variance_delta / bs and
// std = sqrt(max(var, eps)) formed once per row (rows.hpp).
template <int VW>
__global__ __launch_bounds__(kRowThreads) void normalize_delta_kernel(float* __restrict__ delta,
                                                                      const float* __restrict__ x, Rows g,
                                                                      float batchSize, const float* mean,
                                                                      const float* variance, const float* mean_delta,
                                                                      const float* variance_delta) {
  rows_walk(g, [&](int64_t r, int lc) {
    const int64_t i = r % g.nb;
    const float md = mean_delta[i] / batchSize;
    const float vd = (2.0f * variance_delta[i]) / batchSize;
    const float sd = sqrtf(fmaxf(variance[i], kEps));
    const float mu = mean[i];
    auto one = [&](float d, float xv) {
      float t = (xv - mu) * vd;
      t = t + md;
      return d / sd + t;
    };
    float* dr = delta + r * g.block;
    const float* xr = x + r * g.block;
    for (int64_t k = lc; k < g.cpr; k += g.cpt) {
      if constexpr (VW == 4) {
        const float4 d = reinterpret_cast<const float4*>(dr)[k], v = reinterpret_cast<const float4*>(xr)[k];
        reinterpret_cast<float4*>(dr)[k] = make_float4(one(d.x, v.x), one(d.y, v.y), one(d.z, v.z), one(d.w, v.w));
      } else {
        dr[k] = one(dr[k], xr[k]);
      }
    }
  });
}

// The batch-norm backward's last two launches in one: each workgroup first
// forms the mean / variance deltas of its rows' channels from the MvdOp
// partials (MvdFin's arithmetic and wave_total's order = that of
// fixed_total; P <= 64, one partial per lane); the workgroup holding a
// channel's image-0 row also stores them and adds the channel's dgamma total
// (BnBackFin).  Then its rows are normalized as normalize_delta_kernel does.
// One row pass per workgroup (grid = rows / rpw), rpw <= kFinRows.  Each
// thread loads its first chunk of delta and x before the final steps, so
// their latency overlaps.
constexpr int kFinRows = 16;
template <int VW>
__global__ __launch_bounds__(kRowThreads) void normalize_delta_fin_kernel(float* __restrict__ delta,
                                                                          const float* __restrict__ x, Rows g,
                                                                          float batchSize, const float* mean,
                                                                          const float* variance, BnBackFin fin,
                                                                          int P) {
  using V = typename std::conditional<VW == 4, float4, float>::type;
  __shared__ float sMd[kFinRows], sVd[kFinRows];
  const int64_t r0 = static_cast<int64_t>(blockIdx.x) * g.rpw;
  const int lr = threadIdx.x / g.cpt, lc = threadIdx.x - lr * g.cpt;
  const bool live = lr < g.rpw && r0 + lr < g.rows;
  V* dr = reinterpret_cast<V*>(delta + (r0 + lr) * g.block);
  const V* xr = reinterpret_cast<const V*>(x + (r0 + lr) * g.block);
  V d0{}, x0{};
  if (live && lc < g.cpr) {
    d0 = dr[lc];
    x0 = xr[lc];
  }
  // the final steps: wave w takes rows w, w + 4, ... (at most kFinRows / 4)
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  constexpr int kPer = kFinRows / (kRowThreads / 64);
  float pm[kPer], pv[kPer], pd[kPer], vc[kPer];
  double pw[kPer];
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int row = wv + j * (kRowThreads / 64);
    const int64_t r = r0 + row;
    pm[j] = pv[j] = pd[j] = 0.f;
    vc[j] = 1.f;
    pw[j] = 1.0;
    if (row < g.rpw && r < g.rows) {
      const int64_t i = r % g.nb;
      if (lane < P) {
        pm[j] = 0.f + fin.mvd.part[i * P + lane];
        pv[j] = 0.f + fin.mvd.part[(g.nb + i) * P + lane];
        if (r < g.nb) pd[j] = 0.f + fin.dotPart[i * P + lane];
      }
      vc[j] = fmaxf(variance[i], kEps);
      pw[j] = fin.vpow[i];
    }
  }
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int row = wv + j * (kRowThreads / 64);
    const int64_t r = r0 + row;
    if (row < g.rpw && r < g.rows) {  // wave-uniform
      const int64_t i = r % g.nb;
      const float m = lane_total(pm[j]);
      const float v = lane_total(pv[j]);
      const float md = m * (-1.0f / sqrtf(vc[j]));
      // Power(max(var, eps), -3/2) in double, the product stored as single
      const float vd = static_cast<float>(static_cast<double>(v) * -0.5 * pw[j]);
      if (r < g.nb) {  // image 0's row of channel i: once per channel
        const float t = lane_total(pd[j]);
        if (lane == 0) {
          fin.mvd.mean_delta[i] = md;
          fin.mvd.variance_delta[i] = vd;
          fin.scaleUpdates[i] = fin.scaleUpdates[i] + t;
        }
      }
      if (lane == 0) {
        sMd[row] = md;
        sVd[row] = vd;
      }
    }
  }
  __syncthreads();
  if (!live) return;
  const int64_t i = (r0 + lr) % g.nb;
  const float md = sMd[lr] / batchSize;
  const float vd = (2.0f * sVd[lr]) / batchSize;
  const float sd = sqrtf(fmaxf(variance[i], kEps));
  const float mu = mean[i];
  auto one = [&](float d, float xv) {
    float t = (xv - mu) * vd;
    t = t + md;
    return d / sd + t;
  };
  auto put = [&](int64_t k, const V& d, const V& xv) {
    if constexpr (VW == 4)
      dr[k] = make_float4(one(d.x, xv.x), one(d.y, xv.y), one(d.z, xv.z), one(d.w, xv.w));
    else
      dr[k] = one(d, xv);
  };
  if (lc < g.cpr) put(lc, d0, x0);
  for (int64_t k = lc + g.cpt; k < g.cpr; k += g.cpt) put(k, dr[k], xr[k]);
}

// softmax (nsoftmaxlayer.pas:81-105): one thread per (batch, group) row.
__global__ void softmax_kernel(const float* in, float* out, int64_t n, int64_t batch, int64_t batchSize,
                               int64_t groups, int64_t groupSize, int64_t stride, float temp) {
  GRID_STRIDE(r, batch * groups) {
    const int64_t b = r / groups, g = r - b * groups;
    const float* x = in + b * batchSize + g * groupSize;
    float* y = out + b * batchSize + g * groupSize;
    float largest = x[0];
    for (int64_t i = 1; i < n; ++i)
      if (x[i * stride] > largest) largest = x[i * stride];
    float sum = 0.f;
    for (int64_t i = 0; i < n; ++i) {
      // exp() of the reference runs in double; the result is stored as single
      const float e = static_cast<float>(exp(static_cast<double>((x[i * stride] - largest) / temp)));
      sum = sum + e;
      y[i * stride] = e;
    }
    for (int64_t i = 0; i < n; ++i) y[i * stride] = y[i * stride] / sum;
  }
}

// softmaxCrossEntropy (nsoftmaxlayer.pas:123-137).
__global__ void cross_entropy_kernel(int64_t n, const float* pred, const float* truth, float* delta, float* error) {
  GRID_STRIDE(i, n) {
    const float t = truth[i], p = pred[i];
    error[i] = t != 0.f ? static_cast<float>(-log(static_cast<double>(fmaxf(p, kEps)))) : 0.f;
    delta[i] = t - p;
  }
}

__global__ void clamp_kernel(int64_t n, float alpha, const float* src, float* dst, int64_t stride) {
  GRID_STRIDE(i, n) dst[i * stride] = fmaxf(fminf(src[i * stride], alpha), -alpha);
}

// TAvgPoolLayer.forward (navgpoollayer.pas:60-84): one workgroup per (b, c).
// One wave per (image, channel) row: lane l adds elements l, l + 64, ... in
// turn, then a fixed shuffle tree over the lanes (the same order every run).
__global__ __launch_bounds__(256) void avgpool_fwd_kernel(const float* in, int64_t rows, int64_t hw, float* out) {
  const int lane = threadIdx.x & 63;
  const int64_t r = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;  // whole waves: no lane of a live wave leaves early
  const float* p = in + r * hw;
  float s = 0.f;
  for (int64_t k = lane; k < hw; k += 64) s = s + p[k];
  for (int off = 32; off > 0; off >>= 1) s = s + __shfl_down(s, off, 64);
  if (lane == 0) out[r] = s / static_cast<float>(hw);
}

// ---------------------------------------------------------------------------
// The config-3 network's tail as two launches: the average pool, the
// connected layer (logits = avg * W^T + bias), the softmax and the
// cross-entropy forward in one, their backwards in the other.  Each value is
// formed as the reference's CPU sequence forms it: the connected product's
// 8-lane dot (sdot_avx2) for the logits, its saxpy FMA chains (saxpy_avx2)
// for dW (over the batch) and the input delta (over the classes), the
// softmax of softmaxBatch, the delta clamp of TConnectedLayer.backward.
// ---------------------------------------------------------------------------

// sdot_avx2's order (ntensors.pas:1233-1306): eight FMA chains over k = 8q +
// l, masked tail lanes adding fma(0, 0, .), then (acc[l] + acc[l+4]) and two
// pairwise adds.  a is in LDS, b in global memory.
__device__ inline float sdot8_dev(int64_t n, const float* a, const float* b) {
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  int64_t j = 0;
  for (; j + 8 <= n; j += 8)
#pragma unroll
    for (int l = 0; l < 8; ++l) acc[l] = fmaf(a[j + l], b[j + l], acc[l]);
  if (j < n) {
#pragma unroll
    for (int l = 0; l < 8; ++l) {
      const bool in = j + l < n;
      acc[l] = fmaf(in ? a[j + l] : 0.f, in ? b[j + l] : 0.f, acc[l]);
    }
  }
  const float t0 = acc[0] + acc[4], t1 = acc[1] + acc[5], t2 = acc[2] + acc[6], t3 = acc[3] + acc[7];
  return (t0 + t1) + (t2 + t3);
}

// One workgroup per image b after the average pool's launch (dynamic LDS:
// F + classes floats, and the weights when they fit).
__global__ __launch_bounds__(256) void softmax_head_fwd_kernel(int64_t F, int64_t hw, int64_t classes, bool stageW,
                                                               const float* __restrict__ avg,
                                                               const float* __restrict__ W,
                                                               const float* __restrict__ bias,
                                                               const float* __restrict__ truth,
                                                               float* __restrict__ logits, float* __restrict__ prob,
                                                               float* __restrict__ delta, float* __restrict__ error) {
  extern __shared__ float sm[];
  float* sAvg = sm;
  float* sLog = sm + F;
  const int64_t b = blockIdx.x;
  // the image's averages (written by avgpool_fwd_kernel just before) to LDS
  for (int64_t f = threadIdx.x; f < F; f += blockDim.x) sAvg[f] = avg[b * F + f];
  __syncthreads();
  // the weights to LDS when they fit (read once per workgroup, coalesced)
  const float* Wl = W;
  if (stageW) {
    float* sW = sm + F + classes;
    for (int64_t e = threadIdx.x; e < classes * F; e += blockDim.x) sW[e] = W[e];
    __syncthreads();
    Wl = sW;
  }
  // logits = 0 + 1*sdot (gemm NT with beta 0, alpha 1), then + bias (forwardBias)
  for (int64_t c = threadIdx.x; c < classes; c += blockDim.x) {
    const float dot = 1.0f * sdot8_dev(F, sAvg, Wl + c * F);
    const float l = (0.0f + dot) + bias[c];
    sLog[c] = l;
    logits[b * classes + c] = l;
  }
  __syncthreads();
  if (threadIdx.x == 0) {  // softmax_kernel's row (temperature 1), then the cross-entropy
    const float* xl = sLog;
    float largest = xl[0];
    for (int64_t i = 1; i < classes; ++i)
      if (xl[i] > largest) largest = xl[i];
    float sum = 0.f;
    for (int64_t i = 0; i < classes; ++i) {
      const float e = static_cast<float>(exp(static_cast<double>((xl[i] - largest) / 1.0f)));
      sum = sum + e;
      sLog[i] = e;  // each logit is read before its slot is reused
    }
    for (int64_t i = 0; i < classes; ++i) {
      const float pv = sLog[i] / sum;
      const float t = truth[b * classes + i];
      prob[b * classes + i] = pv;
      error[b * classes + i] = t != 0.f ? static_cast<float>(-log(static_cast<double>(fmaxf(pv, kEps)))) : 0.f;
      delta[b * classes + i] = t - pv;
    }
  }
}

// Workgroups [0, batch): image b's connected-layer input delta (a saxpy FMA
// chain over the classes from +0, gemm NN) and its average-pool backward into
// deltaIn; workgroups [batch, batch + classes): class c's weight gradient
// (FMA chain over the images into dW, gemm TN with beta 1) and bias gradient
// (the images' sum, then added: addSums).  Every workgroup reads the softmax
// delta through the clamp, so none waits for another; the image workgroups
// also store the clamped delta.
__global__ __launch_bounds__(256) void softmax_head_bwd_kernel(int64_t batch, int64_t F, int64_t hw,
                                                               int64_t classes, float alpha, float* __restrict__ delta,
                                                               const float* __restrict__ avg,
                                                               const float* __restrict__ W, float* __restrict__ dW,
                                                               float* __restrict__ db, float* __restrict__ avgDelta,
                                                               float* __restrict__ dIn) {
  extern __shared__ float sm[];
  auto clampv = [&](float v) { return fmaxf(fminf(v, alpha), -alpha); };
  if (blockIdx.x < batch) {
    const int64_t b = blockIdx.x;
    float* sDel = sm;
    float* sDA = sm + classes;
    for (int64_t c = threadIdx.x; c < classes; c += blockDim.x) sDel[c] = clampv(delta[b * classes + c]);
    __syncthreads();
    for (int64_t c = threadIdx.x; c < classes; c += blockDim.x) delta[b * classes + c] = sDel[c];
    for (int64_t f = threadIdx.x; f < F; f += blockDim.x) {
      float acc = 0.f;
      for (int64_t c = 0; c < classes; ++c) acc = fmaf(1.0f * sDel[c], W[c * F + f], acc);
      sDA[f] = acc;
      avgDelta[b * F + f] = acc;
    }
    __syncthreads();
    if (dIn) {
      float* d = dIn + b * F * hw;
      for (int64_t e = threadIdx.x; e < F * hw; e += blockDim.x) d[e] = d[e] + sDA[e / hw] / static_cast<float>(hw);
    }
    return;
  }
  const int64_t c = blockIdx.x - batch;
  // the class's clamped deltas to LDS (chunks of the dynamic LDS's F +
  // classes floats), then 32 images' averages in flight per step of the chain
  const int64_t chunk = F + classes;
  float* sD = sm;
  float s = 0.f;  // bias gradient: the images' sum in order (thread 0)
  for (int64_t f0 = 0; f0 < F; f0 += blockDim.x) {
    const int64_t f = f0 + threadIdx.x;
    float acc = f < F ? dW[c * F + f] : 0.f;
    for (int64_t b0 = 0; b0 < batch; b0 += chunk) {
      const int64_t nb = min(chunk, batch - b0);
      __syncthreads();
      for (int64_t j = threadIdx.x; j < nb; j += blockDim.x) sD[j] = clampv(delta[(b0 + j) * classes + c]);
      __syncthreads();
      if (f0 == 0 && threadIdx.x == 0)
        for (int64_t j = 0; j < nb; ++j) s = s + sD[j];
      if (f < F) {
        int64_t j = 0;
        for (; j + 32 <= nb; j += 32) {
          float av[32];
#pragma unroll
          for (int q = 0; q < 32; ++q) av[q] = avg[(b0 + j + q) * F + f];
#pragma unroll
          for (int q = 0; q < 32; ++q) acc = fmaf(1.0f * sD[j + q], av[q], acc);
        }
        for (; j < nb; ++j) acc = fmaf(1.0f * sD[j], avg[(b0 + j) * F + f], acc);
      }
    }
    if (f < F) dW[c * F + f] = acc;
  }
  if (threadIdx.x == 0) db[c] = db[c] + s;
}

// TAvgPoolLayer.backward (navgpoollayer.pas:86-100).
__global__ void avgpool_bwd_kernel(int64_t n, int64_t hw, const float* dOut, float* dIn) {
  GRID_STRIDE(e, n) dIn[e] = dIn[e] + dOut[e / hw] / static_cast<float>(hw);
}

// T*Layer.update (nConvolutionLayer.pas:684-691, nconnectedlayer.pas:344-353):
// wu = fma(-decay*batch, w, wu); w = fma(lr/batch, wu, w); wu *= momentum.
__global__ void sgd_kernel(int64_t n, float aDecay, float aRate, float momentum, float* w, float* wu) {
  GRID_STRIDE(i, n) {
    const float u = fmaf(aDecay, w[i], wu[i]);
    w[i] = fmaf(aRate, u, w[i]);
    wu[i] = u * momentum;
  }
}

// The conv layers of a weight arena whose updated weights also go to their
// tap-major (and, for the data gradient, flipped) copies.
constexpr int kMaxPack = 8;
struct PackSet {
  int n;
  int64_t off[kMaxPack], F[kMaxPack], C[kMaxPack], taps[kMaxPack];
  float* tap[kMaxPack];
  float* flip[kMaxPack];
  // weight-gradient pieces from tnh_conv2d_wgrad_pieces ([nPieces][F][C*taps],
  // nPieces 0: none), added to the layer's weight updates before the step
  const float* pieces[kMaxPack];
  int nPieces[kMaxPack];
};

// weightUpdates[j] + the sum of layer l's pieces at j, with the arithmetic of
// tnh_conv2d_wgrad (alpha = beta = 1): one piece is the accumulator itself;
// several are summed from zero in piece order, kPieceLoads loads issued
// together (wgrad_reduce_kernel's order), then the old value is added.
constexpr int kPieceLoads = 16;
__device__ inline float add_pieces(const PackSet& ps, int l, int64_t j, float wu) {
  const int P = ps.nPieces[l];
  const float* pc = ps.pieces[l];
  const int64_t total = ps.F[l] * ps.C[l] * ps.taps[l];
  float v;
  if (P == 1) {
    v = pc[j];
  } else {
    v = 0.f;
    for (int s = 0; s < P; s += kPieceLoads) {
      float t[kPieceLoads];
#pragma unroll
      for (int q = 0; q < kPieceLoads; ++q) t[q] = s + q < P ? pc[(s + q) * total + j] : 0.f;
#pragma unroll
      for (int q = 0; q < kPieceLoads; ++q)
        if (s + q < P) v = v + t[q];
    }
  }
  return v + wu;
}

// sgd_kernel, then each updated weight of a listed conv layer is also
// written where tnh_conv2d_pack_weights_dgrad would put it; elements n ..
// n + np - 1 of the grid run param_update_kernel's update on p / pu.
__global__ void sgd_pack_kernel(int64_t n, float aDecay, float aRate, float momentum, float* w, float* wu,
                                PackSet ps, int64_t np, float* p, float* pu) {
  GRID_STRIDE(i, n + np) {
    if (i >= n) {
      const int64_t j = i - n;
      p[j] = fmaf(aRate, pu[j], p[j]);
      pu[j] = pu[j] * momentum;
      continue;
    }
    float g = wu[i];
    for (int l = 0; l < ps.n; ++l) {
      const int64_t j = i - ps.off[l];
      if (ps.nPieces[l] > 0 && j >= 0 && j < ps.F[l] * ps.C[l] * ps.taps[l]) g = add_pieces(ps, l, j, g);
    }
    const float u = fmaf(aDecay, w[i], g);
    const float v = fmaf(aRate, u, w[i]);
    w[i] = v;
    wu[i] = u * momentum;
    for (int l = 0; l < ps.n; ++l) {
      const int64_t j = i - ps.off[l];
      const int64_t per = ps.C[l] * ps.taps[l];
      if (j < 0 || j >= ps.F[l] * per) continue;
      const int64_t f = j / per, r = j - f * per;
      const int64_t c = r / ps.taps[l], t = r - c * ps.taps[l];
      ps.tap[l][(f * ps.taps[l] + t) * ps.C[l] + c] = v;
      if (ps.flip[l]) ps.flip[l][(c * ps.taps[l] + (ps.taps[l] - 1 - t)) * ps.F[l] + f] = v;
    }
  }
}

// p = fma(lr/batch, pu, p); pu *= momentum (biases / scales).
__global__ void param_update_kernel(int64_t n, float aRate, float momentum, float* p, float* pu) {
  GRID_STRIDE(i, n) {
    p[i] = fmaf(aRate, pu[i], p[i]);
    pu[i] = pu[i] * momentum;
  }
}

// ---------------------------------------------------------------------------
// Weight-gradient GEMM: C = beta*C + alpha * sum_b A_b * B_b^T with
// A_b = A + b*strideA ([M][L], row stride lda) and B_b = B + b*strideB
// ([N][L], row stride ldb).  The batch is folded into one K axis of length
// batch*L; with L a multiple of the panel depth a panel never straddles two
// images, so the per-panel base offset is uniform: (k0 / L)*stride + k0 % L.
// Both operands are k-contiguous (KC layout).  Split-K over gridDim.y fills
// the GPU (M x N is small for conv weights); partial sums are reduced in
// split order.
// ---------------------------------------------------------------------------
template <bool VEC, int ROWS, int BK, int NT>
struct SegLoader : DenseLoader<true, VEC, ROWS, BK, NT> {
  using Base = DenseLoader<true, VEC, ROWS, BK, NT>;
  int64_t segL, segStride;
  __device__ inline void load(int64_t k0) {
    const int64_t seg = k0 / segL;
    const uint32_t koff = static_cast<uint32_t>((seg * segStride + (k0 - seg * segL)) * 4);
#pragma unroll
    for (int v = 0; v < Base::PER; ++v) {
      const bool ok = Base::rowOk[v] && static_cast<int>(k0) + Base::kIdx[v] < Base::K;
      const uint32_t off = sel_off(ok, Base::off0[v] + koff);
      if constexpr (VEC)
        Base::reg[v] = buf_ld4(Base::rsrc, off);
      else
        Base::reg[v] = buf_ld1(Base::rsrc, off);
    }
  }
};

struct WgradArgs {
  const float* A;
  const float* B;
  float* C;
  float* part;
  int64_t M, N, L, lda, ldb, ldc, strideA, strideB, batch;
  int64_t aBytes, bBytes, kChunk;
  float alpha, beta;
  int tilesM, tilesN, splits;
  int rawPieces;  // store every split's raw sums in part, no reduction (also one split)
};

template <class Cfg, bool VA, bool VB>
__global__ __launch_bounds__(Cfg::NT) void wgrad_kernel(WgradArgs a) {
  using AL = SegLoader<VA, Cfg::BM, Cfg::BK, Cfg::NT>;
  using BL = SegLoader<VB, Cfg::BN, Cfg::BK, Cfg::NT>;
  using Main = GemmMainloop<Cfg, AL, BL>;
  __shared__ __attribute__((aligned(16))) float smem[Main::LDS_FLOATS];
  lds_t* lds = (lds_t*)smem;
  int tm, tn;
  tile_coords(blockIdx.x, a.tilesM, a.tilesN, tm, tn);
  const int64_t m0 = static_cast<int64_t>(tm) * Cfg::BM, n0 = static_cast<int64_t>(tn) * Cfg::BN;
  const int64_t Ktot = a.batch * a.L;
  AL al;
  al.init(a.A, a.aBytes, a.lda, a.M, Ktot, m0, threadIdx.x);
  al.segL = a.L;
  al.segStride = a.strideA;
  BL bl;
  bl.init(a.B, a.bBytes, a.ldb, a.N, Ktot, n0, threadIdx.x);
  bl.segL = a.L;
  bl.segStride = a.strideB;
  f32x16 acc[Cfg::FM][Cfg::FN];
  const int64_t kBegin = blockIdx.y * a.kChunk;
  const int64_t kEnd = min(Ktot, kBegin + a.kChunk);
  Main::exec(al, bl, kBegin, kEnd, lds, acc);
  if (a.splits > 1) {
    float* part = a.part + static_cast<int64_t>(blockIdx.y) * a.M * a.N;
    Main::for_each(acc, [&](int row, int col, float v) {
      const int64_t gr = m0 + row, gc = n0 + col;
      if (gr < a.M && gc < a.N) part[gr * a.N + gc] = v;
    });
    return;
  }
  Main::for_each(acc, [&](int row, int col, float v) {
    const int64_t gr = m0 + row, gc = n0 + col;
    if (gr < a.M && gc < a.N) {
      float* p = a.C + gr * a.ldc + gc;
      float out = a.alpha * v;
      if (a.beta != 0.f) out = out + a.beta * *p;
      *p = out;
    }
  });
}

// The convolution weight gradient with the im2col in the B loader:
// dW[f][n] = sum over (b, oy, ox) of delta_b[f][oy*OW + ox] * x_b[c][iy][ix],
// n = (c*kh + ky)*kw + kx (the reference weight order), iy = oy*sY - pH +
// ky*dY, ix = ox*sX - pW + kx*dX, 0 outside the image: the values im2col
// writes (sim2Col, ntensors.pas:11415), read straight from the input.  The
// reduction axis is wgrad_kernel's (image by image, L = OH*OW pixels each,
// panels of BK pixels inside one image), so the sums equal im2col followed by
// tnh_sgemm_nt_batch_reduce bit for bit.  A panel starts at a multiple of BK
// pixels; with OW | BK or BK | OW the output row and column of a thread's
// pixels are the panel's (uniform) plus a per-thread constant.
struct ColGeom {
  int64_t xBatchStride, xBytes;
  int C, H, W, OW, L, kh, kw, sY, sX, pH, pW, dY, dX;
};

template <int ROWS, int BK, int NT>
struct ColGatherLoader : DenseLoader<true, true, ROWS, BK, NT> {
  // a thread's unit is 4 consecutive pixels of one row n: with OW % 4 == 0
  // they lie in one output row, so one row test and one address serve all
  // four (the input columns are sX apart); the four values go to LDS as one
  // 16-byte store, like a dense 16-byte load's
  using Base = DenseLoader<true, true, ROWS, BK, NT>;
  static constexpr int PER = Base::PER;
  ColGeom g;
  int ky[PER], kx[PER], dy[PER], dx[PER];
  int64_t cOff[PER];  // c*H*W of the unit's row
  __device__ inline void init_col(const float* x, const ColGeom& geom, int64_t rows, int64_t Ktot, int64_t row0,
                                  int tid) {
    g = geom;
    Base::rsrc = make_rsrc(x, geom.xBytes);
    Base::K = static_cast<int>(Ktot);
#pragma unroll
    for (int v = 0; v < PER; ++v) {
      const int idx = tid + v * NT;
      int row, k;
      Base::coords(idx, row, k);
      const int64_t n = row0 + row;
      Base::rowOk[v] = n < rows && (!Base::kPartial || idx < Base::UNITS);
      Base::kIdx[v] = k;
      const int64_t nn = Base::rowOk[v] ? n : 0;
      const int64_t taps = static_cast<int64_t>(g.kh) * g.kw;
      const int64_t c = nn / taps, t = nn - c * taps;
      ky[v] = static_cast<int>(t / g.kw);
      kx[v] = static_cast<int>(t - (t / g.kw) * g.kw);
      cOff[v] = c * g.H * g.W;
      dy[v] = g.OW >= BK ? 0 : k / g.OW;
      dx[v] = g.OW >= BK ? k : k % g.OW;
    }
  }
  __device__ inline void load(int64_t k0) {
    const int64_t b = k0 / g.L;  // uniform: a panel lies inside one image
    const int64_t l0 = k0 - b * g.L;
    const int oy0 = static_cast<int>(l0 / g.OW);
    const int ox0 = static_cast<int>(l0 - static_cast<int64_t>(oy0) * g.OW);
    const int64_t base = b * g.xBatchStride;
#pragma unroll
    for (int v = 0; v < PER; ++v) {
      const int iy = (oy0 + dy[v]) * g.sY - g.pH + ky[v] * g.dY;
      const int ix = (ox0 + dx[v]) * g.sX - g.pW + kx[v] * g.dX;
      const bool rowIn = Base::rowOk[v] && static_cast<unsigned>(iy) < static_cast<unsigned>(g.H);
      const int64_t e = base + cOff[v] + static_cast<int64_t>(iy) * g.W + ix;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const bool ok = rowIn && static_cast<unsigned>(ix + j * g.sX) < static_cast<unsigned>(g.W);
        Base::reg[v][j] = buf_ld1(Base::rsrc, sel_off(ok, static_cast<uint32_t>((e + j * g.sX) * 4)));
      }
    }
  }
};

template <class Cfg, bool VA>
__global__ __launch_bounds__(Cfg::NT) void wgrad_col_kernel(WgradArgs a, ColGeom geom) {
  using AL = SegLoader<VA, Cfg::BM, Cfg::BK, Cfg::NT>;
  using BL = ColGatherLoader<Cfg::BN, Cfg::BK, Cfg::NT>;
  using Main = GemmMainloop<Cfg, AL, BL>;
  __shared__ __attribute__((aligned(16))) float smem[Main::LDS_FLOATS];
  lds_t* lds = (lds_t*)smem;
  int tm, tn;
  tile_coords(blockIdx.x, a.tilesM, a.tilesN, tm, tn);
  const int64_t m0 = static_cast<int64_t>(tm) * Cfg::BM, n0 = static_cast<int64_t>(tn) * Cfg::BN;
  const int64_t Ktot = a.batch * a.L;
  AL al;
  al.init(a.A, a.aBytes, a.lda, a.M, Ktot, m0, threadIdx.x);
  al.segL = a.L;
  al.segStride = a.strideA;
  BL bl;
  bl.init_col(a.B, geom, a.N, Ktot, n0, threadIdx.x);
  f32x16 acc[Cfg::FM][Cfg::FN];
  const int64_t kBegin = blockIdx.y * a.kChunk;
  const int64_t kEnd = min(Ktot, kBegin + a.kChunk);
  Main::exec(al, bl, kBegin, kEnd, lds, acc);
  if (a.splits > 1 || a.rawPieces) {
    float* part = a.part + static_cast<int64_t>(blockIdx.y) * a.M * a.N;
    Main::for_each(acc, [&](int row, int col, float v) {
      const int64_t gr = m0 + row, gc = n0 + col;
      if (gr < a.M && gc < a.N) part[gr * a.N + gc] = v;
    });
    return;
  }
  Main::for_each(acc, [&](int row, int col, float v) {
    const int64_t gr = m0 + row, gc = n0 + col;
    if (gr < a.M && gc < a.N) {
      float* p = a.C + gr * a.ldc + gc;
      float out = a.alpha * v;
      if (a.beta != 0.f) out = out + a.beta * *p;
      *p = out;
    }
  });
}

// Sums the split partials of each output element: one wave per element, lane
// l adds splits l, l + 64, ... in turn (their loads issued together), then a
// fixed tree over the lanes; then alpha and beta.  Fixed order: the result
// does not vary run to run.
__global__ __launch_bounds__(256) void wgrad_reduce_wave_kernel(WgradArgs a) {
  __shared__ float sh[4][64];
  const int64_t total = a.M * a.N;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t e = static_cast<int64_t>(blockIdx.x) * 4 + w;
  float v = 0.f;
  if (e < total)
    for (int s = lane; s < a.splits; s += 64) v = v + a.part[s * total + e];
  sh[w][lane] = v;
  __syncthreads();
  for (int k = 32; k > 0; k >>= 1) {
    if (lane < k) sh[w][lane] = sh[w][lane] + sh[w][lane + k];
    __syncthreads();
  }
  if (lane == 0 && e < total) {
    const int64_t r = e / a.N, c = e - r * a.N;
    float* p = a.C + r * a.ldc + c;
    float out = a.alpha * sh[w][0];
    if (a.beta != 0.f) out = out + a.beta * *p;
    *p = out;
  }
}

// The same sums when there are many output elements: one thread per element
// adds the splits in split order, kReduceLoads loads issued together
// (coalesced along the elements), the last round's too.
constexpr int kReduceLoads = 16;  // 8 and 32 were slower on the config-3 step
__global__ __launch_bounds__(256) void wgrad_reduce_kernel(WgradArgs a) {
  const int64_t total = a.M * a.N;
  GRID_STRIDE(e, total) {
    float v = 0.f;
    for (int s = 0; s < a.splits; s += kReduceLoads) {
      float t[kReduceLoads];
#pragma unroll
      for (int j = 0; j < kReduceLoads; ++j) t[j] = s + j < a.splits ? a.part[(s + j) * total + e] : 0.f;
#pragma unroll
      for (int j = 0; j < kReduceLoads; ++j)
        if (s + j < a.splits) v = v + t[j];  // only the pieces, in split order
    }
    const int64_t r = e / a.N, c = e - r * a.N;
    float* p = a.C + r * a.ldc + c;
    float out = a.alpha * v;
    if (a.beta != 0.f) out = out + a.beta * *p;
    *p = out;
  }
}

using WCfg = TileCfg<64, 64, 32, 2, 2, 2>;

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

int launch_wgrad_reduce(const WgradArgs& a, hipStream_t s);
// weight gradients of fewer elements sum their pieces a wave per element
constexpr int64_t kWaveReduceBelow = 8192;

template <bool VA, bool VB>
int launch_wgrad(WgradArgs a, hipStream_t s) {
  dim3 grid(static_cast<unsigned>(a.tilesM * a.tilesN), static_cast<unsigned>(a.splits));
  hipLaunchKernelGGL((wgrad_kernel<WCfg, VA, VB>), grid, dim3(WCfg::NT), 0, s, a);
  if (int st = launch_status("wgrad_kernel")) return st;
  return launch_wgrad_reduce(a, s);
}

template <bool VA>
int launch_wgrad_col(WgradArgs a, const ColGeom& g, hipStream_t s) {
  dim3 grid(static_cast<unsigned>(a.tilesM * a.tilesN), static_cast<unsigned>(a.splits));
  hipLaunchKernelGGL((wgrad_col_kernel<WCfg, VA>), grid, dim3(WCfg::NT), 0, s, a, g);
  if (int st = launch_status("wgrad_col_kernel")) return st;
  return launch_wgrad_reduce(a, s);
}

int launch_wgrad_reduce(const WgradArgs& a, hipStream_t s) {
  if (a.splits > 1 && !a.rawPieces) {
    // few outputs: a wave per output element spreads the splits over its
    // lanes; many: a thread per element keeps the loads coalesced
    if (a.M * a.N < kWaveReduceBelow) {
      hipLaunchKernelGGL(wgrad_reduce_wave_kernel, dim3(static_cast<unsigned>((a.M * a.N + 3) / 4)), dim3(256), 0, s,
                         a);
      return launch_status("wgrad_reduce_wave_kernel");
    }
    hipLaunchKernelGGL(wgrad_reduce_kernel, dim3(grid_1d(a.M * a.N)), dim3(256), 0, s, a);
    return launch_status("wgrad_reduce_kernel");
  }
  return TNH_OK;
}

}  // namespace

namespace {
__global__ __launch_bounds__(256) void stat_final_kernel(StatParts sp, int64_t C) {
  const int64_t f = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (f >= C) return;  // whole waves
  float m, v;
  sp.finish(f, true, m, v);
}
}  // namespace

int bn_stat_final(int64_t C, const StatParts& sp) {
  TNH_REQUIRE_CTX(cx);
  hipLaunchKernelGGL(stat_final_kernel, dim3(static_cast<unsigned>((C + 3) / 4)), dim3(256), 0, cx->stream, sp, C);
  return launch_status("stat_final_kernel");
}

int bn_stat_partials(int64_t C, int64_t block, int64_t groups, const float* x, float* means, float* vars,
                     float* rollMean, float* rollVar, float momentum, StatParts& sp) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(C > 0 && groups > 0 && block > 0 && groups * block > 1, "bn statistics: bad sizes");
  TNH_ARG(x && means && vars, "bn statistics: NULL buffer");
  TNH_ARG((rollMean == nullptr) == (rollVar == nullptr), "bn statistics: give both rolling buffers or none");
  ChanSplit s;
  float* red = nullptr;
  if (int st = chan_split(s, red, C, block, groups, 2, cx)) return st;
  const bool vec = chan_vec(s, {x});
  const float S = static_cast<float>(groups * block);
  sp = StatParts{red, red + C * s.P, s.P, S, means, vars, rollMean, rollVar, 1.0f - momentum, momentum};
  if (int st = launch_partial<1>(cx, SumOp{x}, s, vec, red, "chan_partial_kernel<sum>")) return st;
  return launch_partial<1>(cx, RssOp{x, red, S, 0.f}, s, vec, red + C * s.P, "chan_partial_kernel<rss>");
}

}  // namespace tnh

using namespace tnh;

extern "C" int32_t tnh_means_vars(int64_t srcSize, int64_t dstSize, int64_t groups, const float* src,
                                  int64_t offset, float* means, float* vars) {
  return means_vars_impl(srcSize, dstSize, groups, src, offset, means, vars, nullptr, nullptr, 0.f);
}

extern "C" int32_t tnh_bn_statistics(int64_t srcSize, int64_t dstSize, int64_t groups, const float* src,
                                     int64_t offset, float* means, float* vars, float* rollingMeans,
                                     float* rollingVars, float momentum) {
  TNH_ARG((rollingMeans == nullptr) == (rollingVars == nullptr), "bn_statistics: give both rolling buffers or none");
  return means_vars_impl(srcSize, dstSize, groups, src, offset, means, vars, rollingMeans, rollingVars, momentum);
}

extern "C" int32_t tnh_means(int64_t srcSize, int64_t dstSize, int64_t groups, const float* src, int64_t offset,
                             float* means) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(dstSize > 0 && groups > 0 && srcSize > 0 && offset >= 0, "means: bad sizes");
  TNH_ARG(src && means, "means: NULL buffer");
  const int64_t block = srcSize / (dstSize * groups);
  TNH_ARG(block * dstSize * groups == srcSize, "means: sizes do not align");
  ChanSplit s;
  float* red = nullptr;
  if (int st = chan_split(s, red, dstSize, block, groups, 1, cx)) return st;
  const float* x = src + offset;
  return launch_partial<1>(cx, SumOp{x}, s, chan_vec(s, {x}), red, "chan_partial_kernel<sum>",
                           TotalDivFin{red, static_cast<float>(groups * block), means});
}

extern "C" int32_t tnh_variances(int64_t srcSize, int64_t dstSize, int64_t groups, const float* src, int64_t offset,
                                 const float* means, float* vars) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(dstSize > 0 && groups > 0 && srcSize > 0 && offset >= 0, "variances: bad sizes");
  TNH_ARG(src && means && vars, "variances: NULL buffer");
  const int64_t block = srcSize / (dstSize * groups);
  TNH_ARG(block * dstSize * groups == srcSize && groups * block > 1, "variances: sizes do not align");
  ChanSplit s;
  float* red = nullptr;
  if (int st = chan_split(s, red, dstSize, block, groups, 1, cx)) return st;
  const float* x = src + offset;
  return launch_partial<1>(cx, RssGivenOp{x, means, 0.f}, s, chan_vec(s, {x}), red, "chan_partial_kernel<rss>",
                           TotalDivFin{red, static_cast<float>(groups * block) - 1.f, vars});
}

extern "C" int32_t tnh_means_vars_delta(int64_t srcSize, int64_t dstSize, int64_t groups, const float* delta,
                                        const float* x, int64_t offset, const float* mean, const float* variance,
                                        float* mean_delta, float* variance_delta) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(dstSize > 0 && groups > 0 && srcSize > 0 && offset >= 0, "means_vars_delta: bad sizes");
  TNH_ARG(delta && x && mean && variance && mean_delta && variance_delta, "means_vars_delta: NULL buffer");
  const int64_t block = srcSize / (dstSize * groups);
  TNH_ARG(block * dstSize * groups == srcSize, "means_vars_delta: sizes do not align");
  ChanSplit s;
  float* red = nullptr;
  if (int st = chan_split(s, red, dstSize, block, groups, 2, cx)) return st;
  const float* d = delta + offset;
  const float* xx = x + offset;
  return launch_partial<2>(cx, MvdOp{d, xx, mean, 0.f}, s, chan_vec(s, {d, xx}), red,
                           "chan_partial_kernel<mean_var_delta>", MvdFin{red, variance, mean_delta, variance_delta});
}

extern "C" int32_t tnh_normalize_delta(int64_t deltaSize, int64_t meanSize, int64_t groups, float* delta,
                                       const float* x, int64_t offset, const float* mean, const float* variance,
                                       const float* mean_delta, const float* variance_delta) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(deltaSize > 0 && meanSize > 0 && groups > 0 && offset >= 0, "normalize_delta: bad sizes");
  TNH_ARG(delta && x && mean && variance && mean_delta && variance_delta, "normalize_delta: NULL buffer");
  const int64_t block = deltaSize / (meanSize * groups);
  TNH_ARG(block * meanSize * groups == deltaSize, "normalize_delta: sizes do not align");
  const float batchSize = static_cast<float>(block * groups);
  float* d = delta + offset;
  const float* xx = x + offset;
  if (block % 4 == 0 && rows_al16(d) && rows_al16(xx)) {
    const Rows g = make_rows(deltaSize, block, meanSize, 4);
    hipLaunchKernelGGL(normalize_delta_kernel<4>, dim3(grid_rows(g)), dim3(kRowThreads), 0, cx->stream, d, xx, g,
                       batchSize, mean, variance, mean_delta, variance_delta);
  } else {
    const Rows g = make_rows(deltaSize, block, meanSize, 1);
    hipLaunchKernelGGL(normalize_delta_kernel<1>, dim3(grid_rows(g)), dim3(kRowThreads), 0, cx->stream, d, xx, g,
                       batchSize, mean, variance, mean_delta, variance_delta);
  }
  return launch_status("normalize_delta_kernel");
}

extern "C" int32_t tnh_add_dots(int64_t N, int64_t dstSize, int64_t groups, const float* src1, const float* src2,
                                int64_t srcOffset, float* dst) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(N > 0 && dstSize > 0 && groups > 0 && srcOffset >= 0, "add_dots: bad sizes");
  TNH_ARG(src1 && src2 && dst, "add_dots: NULL buffer");
  const int64_t block = N / (dstSize * groups);
  TNH_ARG(block * dstSize * groups == N, "add_dots: sizes do not align");
  ChanSplit s;
  float* red = nullptr;
  if (int st = chan_split(s, red, dstSize, block, groups, 1, cx)) return st;
  const float* a = src1 + srcOffset;
  const float* b = src2 + srcOffset;
  return launch_partial<1>(cx, DotOp{a, b}, s, chan_vec(s, {a, b}), red, "chan_partial_kernel<dots>",
                           AddFin{red, dst});
}

extern "C" int32_t tnh_backward_bias(int64_t dstSize, float* dst, int64_t srcSize, const float* src,
                                     int64_t srcOffset, int64_t incb, int64_t batch) {
  (void)incb;
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(dstSize > 0 && srcSize >= 0 && batch > 0 && srcOffset >= 0, "backward_bias: bad sizes");
  TNH_ARG(dst && src, "backward_bias: NULL buffer");
  const int64_t block = srcSize / (dstSize * batch);
  TNH_ARG(block * dstSize * batch == srcSize, "backward_bias: sizes do not align");
  if (srcSize == 0) return TNH_OK;
  ChanSplit s;
  float* red = nullptr;
  if (int st = chan_split(s, red, dstSize, block, batch, 1, cx)) return st;
  const float* x = src + srcOffset;
  return launch_partial<1>(cx, SumOp{x}, s, chan_vec(s, {x}), red, "chan_partial_kernel<sum>", AddFin{red, dst});
}

extern "C" int32_t tnh_bn_backward_scale(int64_t N, int64_t dstSize, int64_t groups, const float* output,
                                         int32_t act, const float* xNorm, const float* scales, float* delta,
                                         float* scaleUpdates) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(N > 0 && dstSize > 0 && groups > 0, "bn_backward_scale: bad sizes");
  TNH_ARG(output && xNorm && scales && delta && scaleUpdates, "bn_backward_scale: NULL buffer");
  TNH_ARG(act == TNH_AC_LINEAR || act == TNH_AC_LEAKY || act == TNH_AC_LOGISTIC, "bn_backward_scale: activation %d",
          act);
  const int64_t block = N / (dstSize * groups);
  TNH_ARG(block * dstSize * groups == N, "bn_backward_scale: sizes do not align");
  ChanSplit s;
  float* red = nullptr;
  if (int st = chan_split(s, red, dstSize, block, groups, 1, cx)) return st;
  return launch_partial<1>(cx, BnBackOp{delta, output, xNorm, scales, act, 0.f}, s,
                           chan_vec(s, {delta, output, xNorm}), red, "chan_partial_kernel<bn_back>",
                           AddFin{red, scaleUpdates});
}

extern "C" int32_t tnh_softmax_batch(int64_t N, const float* input, int64_t iOffset, int64_t batch,
                                     int64_t batchSize, int64_t groups, int64_t groupSize, int64_t stride, float temp,
                                     float* output, int64_t oOffset) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(N > 0 && batch >= 0 && groups > 0 && stride > 0 && iOffset >= 0 && oOffset >= 0,
          "softmax_batch: bad sizes");
  TNH_ARG(input && output, "softmax_batch: NULL buffer");
  if (batch == 0) return TNH_OK;
  hipLaunchKernelGGL(softmax_kernel, dim3(grid_1d(batch * groups)), dim3(256), 0, cx->stream, input + iOffset,
                     output + oOffset, N, batch, batchSize, groups, groupSize, stride, temp);
  return launch_status("softmax_kernel");
}

extern "C" int32_t tnh_cross_entropy_softmax(int64_t N, const float* pred, const float* truth, float* delta,
                                             float* error) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(N >= 0, "cross_entropy_softmax: bad size");
  if (N == 0) return TNH_OK;
  TNH_ARG(pred && truth && delta && error, "cross_entropy_softmax: NULL buffer");
  hipLaunchKernelGGL(cross_entropy_kernel, dim3(grid_1d(N)), dim3(256), 0, cx->stream, N, pred, truth, delta, error);
  return launch_status("cross_entropy_kernel");
}

extern "C" int32_t tnh_clamp(int64_t N, float alpha, const float* src, float* dst, int64_t stride, int64_t offset) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(N >= 0 && stride > 0 && offset >= 0, "clamp: bad arguments");
  if (N == 0) return TNH_OK;
  TNH_ARG(src && dst, "clamp: NULL buffer");
  hipLaunchKernelGGL(clamp_kernel, dim3(grid_1d(N)), dim3(256), 0, cx->stream, N, alpha, src + offset, dst + offset,
                     stride);
  return launch_status("clamp_kernel");
}

extern "C" int32_t tnh_avgpool_fwd(int64_t batch, int64_t c, int64_t h, int64_t w, const float* input,
                                   float* output) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(batch >= 0 && c > 0 && h > 0 && w > 0, "avgpool_fwd: bad sizes");
  if (batch == 0) return TNH_OK;
  TNH_ARG(input && output, "avgpool_fwd: NULL buffer");
  TNH_ARG(batch * c < (int64_t(1) << 31), "avgpool_fwd: too many planes");
  hipLaunchKernelGGL(avgpool_fwd_kernel, dim3(static_cast<unsigned>((batch * c + 3) / 4)), dim3(256), 0, cx->stream,
                     input, batch * c, h * w, output);
  return launch_status("avgpool_fwd_kernel");
}

extern "C" int32_t tnh_avgpool_bwd(int64_t batch, int64_t c, int64_t h, int64_t w, const float* delta,
                                   float* deltaIn) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(batch >= 0 && c > 0 && h > 0 && w > 0, "avgpool_bwd: bad sizes");
  if (batch == 0) return TNH_OK;
  TNH_ARG(delta && deltaIn, "avgpool_bwd: NULL buffer");
  const int64_t n = batch * c * h * w;
  hipLaunchKernelGGL(avgpool_bwd_kernel, dim3(grid_1d(n)), dim3(256), 0, cx->stream, n, h * w, delta, deltaIn);
  return launch_status("avgpool_bwd_kernel");
}

extern "C" int32_t tnh_sgd_update(int64_t N, float learningRate, int64_t batch, float momentum, float decay,
                                  float* weights, float* weightUpdates) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(N >= 0 && batch > 0, "sgd_update: bad arguments");
  if (N == 0) return TNH_OK;
  TNH_ARG(weights && weightUpdates, "sgd_update: NULL buffer");
  const float aDecay = -decay * static_cast<float>(batch);
  const float aRate = learningRate / static_cast<float>(batch);
  hipLaunchKernelGGL(sgd_kernel, dim3(grid_1d(N)), dim3(256), 0, cx->stream, N, aDecay, aRate, momentum, weights,
                     weightUpdates);
  return launch_status("sgd_kernel");
}

extern "C" int32_t tnh_sgd_update_pack_pieces(int64_t N, float learningRate, int64_t batch, float momentum,
                                              float decay, float* weights, float* weightUpdates, int32_t nPack,
                                              const int64_t* packOffset, const int64_t* packF, const int64_t* packC,
                                              const int64_t* packTaps, float* const* packTap, float* const* packFlip,
                                              const float* const* packPieces, const int32_t* packNPieces,
                                              int64_t nParams, float* params, float* paramUpdates) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(N >= 0 && batch > 0 && nParams >= 0, "sgd_update_pack: bad arguments");
  TNH_ARG(nPack >= 0 && nPack <= kMaxPack, "sgd_update_pack: %d layers (at most %d)", nPack, kMaxPack);
  if (N + nParams == 0) return TNH_OK;
  TNH_ARG(N == 0 || (weights && weightUpdates), "sgd_update_pack: NULL buffer");
  TNH_ARG(nParams == 0 || (params && paramUpdates), "sgd_update_pack: NULL parameter buffer");
  TNH_ARG(nPack == 0 || (packOffset && packF && packC && packTaps && packTap && packFlip),
          "sgd_update_pack: NULL layer table");
  PackSet ps{};
  ps.n = nPack;
  for (int l = 0; l < nPack; ++l) {
    TNH_ARG(packF[l] > 0 && packC[l] > 0 && packTaps[l] > 0 && packOffset[l] >= 0 &&
                packOffset[l] + packF[l] * packC[l] * packTaps[l] <= N && packTap[l],
            "sgd_update_pack: layer %d outside the arena", l);
    TNH_ARG(packTap[l] != weights && packFlip[l] != weights, "sgd_update_pack: a copy aliases the weights");
    ps.off[l] = packOffset[l];
    ps.F[l] = packF[l];
    ps.C[l] = packC[l];
    ps.taps[l] = packTaps[l];
    ps.tap[l] = packTap[l];
    ps.flip[l] = packFlip[l];
    ps.pieces[l] = nullptr;
    ps.nPieces[l] = 0;
    if (packNPieces && packNPieces[l] != 0) {
      TNH_ARG(packNPieces[l] > 0 && packPieces && packPieces[l], "sgd_update_pack: layer %d: bad pieces", l);
      TNH_ARG(packPieces[l] != weights && packPieces[l] != weightUpdates, "sgd_update_pack: pieces alias the arena");
      ps.pieces[l] = packPieces[l];
      ps.nPieces[l] = packNPieces[l];
    }
  }
  const float aDecay = -decay * static_cast<float>(batch);
  const float aRate = learningRate / static_cast<float>(batch);
  hipLaunchKernelGGL(sgd_pack_kernel, dim3(grid_1d(N + nParams)), dim3(256), 0, cx->stream, N, aDecay, aRate, momentum,
                     weights, weightUpdates, ps, nParams, params, paramUpdates);
  return launch_status("sgd_pack_kernel");
}

extern "C" int32_t tnh_sgd_update_pack(int64_t N, float learningRate, int64_t batch, float momentum, float decay,
                                       float* weights, float* weightUpdates, int32_t nPack, const int64_t* packOffset,
                                       const int64_t* packF, const int64_t* packC, const int64_t* packTaps,
                                       float* const* packTap, float* const* packFlip, int64_t nParams, float* params,
                                       float* paramUpdates) {
  return tnh_sgd_update_pack_pieces(N, learningRate, batch, momentum, decay, weights, weightUpdates, nPack,
                                    packOffset, packF, packC, packTaps, packTap, packFlip, nullptr, nullptr, nParams,
                                    params, paramUpdates);
}

extern "C" int32_t tnh_param_update(int64_t N, float learningRate, int64_t batch, float momentum, float* params,
                                    float* paramUpdates) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(N >= 0 && batch > 0, "param_update: bad arguments");
  if (N == 0) return TNH_OK;
  TNH_ARG(params && paramUpdates, "param_update: NULL buffer");
  const float aRate = learningRate / static_cast<float>(batch);
  hipLaunchKernelGGL(param_update_kernel, dim3(grid_1d(N)), dim3(256), 0, cx->stream, N, aRate, momentum, params,
                     paramUpdates);
  return launch_status("param_update_kernel");
}

namespace tnh {
namespace {
// Tiles and the split of the batch-folded K axis: about two workgroups per
// CU over the weight tiles, at least four panels per split, the partials in
// the stream's workspace (whole K when there is none, e.g. under capture
// before any eager call).
// measured on the config-3 step: 1 or 4 workgroups per CU, or at least 16
// panels per split, were 1.5-3.5% slower per step
constexpr int64_t kWgradWgPerCu = 2, kWgradMinPanels = 4;

// With rawPieces the caller's memory takes the pieces (a.part, set after the
// split is known), so the split never falls back to whole K.
int wgrad_split(Context* cx, WgradArgs& a, const char* who) {
  a.tilesM = static_cast<int>((a.M + WCfg::BM - 1) / WCfg::BM);
  a.tilesN = static_cast<int>((a.N + WCfg::BN - 1) / WCfg::BN);
  const int64_t tiles = static_cast<int64_t>(a.tilesM) * a.tilesN;
  TNH_ARG(tiles < (int64_t(1) << 31), "%s: grid too large", who);
  const int64_t Ktot = a.batch * a.L;
  const int64_t panels = Ktot / WCfg::BK;
  int64_t splits = (kWgradWgPerCu * cx->cu_count + tiles - 1) / tiles;
  splits = std::max<int64_t>(1, std::min<int64_t>({splits, panels / kWgradMinPanels, 1024}));
  a.kChunk = (panels + splits - 1) / splits * WCfg::BK;
  a.splits = static_cast<int>((Ktot + a.kChunk - 1) / a.kChunk);
  if (a.rawPieces) return TNH_OK;
  if (a.splits > 1) {
    a.part = static_cast<float*>(workspace(cx, static_cast<size_t>(a.splits) * a.M * a.N * 4));
    if (!a.part) {
      a.splits = 1;
      a.kChunk = Ktot;
    }
  }
  return TNH_OK;
}
}  // namespace
}  // namespace tnh

extern "C" int32_t tnh_sgemm_nt_batch_reduce(int64_t M, int64_t N, int64_t L, float alpha, const float* A,
                                             int64_t aOff, int64_t lda, int64_t strideA, const float* B,
                                             int64_t bOff, int64_t ldb, int64_t strideB, float beta, float* C,
                                             int64_t cOff, int64_t ldc, int64_t batch) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(M >= 0 && N >= 0 && L >= 0 && batch >= 0, "sgemm_nt_batch_reduce: negative size");
  if (M == 0 || N == 0) return TNH_OK;
  TNH_ARG(C != nullptr && ldc >= N && cOff >= 0, "sgemm_nt_batch_reduce: bad C");
  if (L == 0 || batch == 0) {  // empty sum: C = beta*C
    return tnh_sgemm(0, 1, M, N, 0, alpha, A, 0, 1, B, 0, 1, beta, C, cOff, ldc);
  }
  TNH_ARG(A && B && lda >= L && ldb >= L && aOff >= 0 && bOff >= 0, "sgemm_nt_batch_reduce: bad A/B");
  TNH_ARG(strideA >= 0 && strideB >= 0, "sgemm_nt_batch_reduce: negative stride");
  const int64_t aElems = (batch - 1) * strideA + (M - 1) * lda + L;
  const int64_t bElems = (batch - 1) * strideB + (N - 1) * ldb + L;
  TNH_ARG(aElems * 4 <= kMaxBufBytes && bElems * 4 <= kMaxBufBytes && batch * L < (int64_t(1) << 31),
          "sgemm_nt_batch_reduce: operands span more than 2 GiB (split the batch)");
  if (L % WCfg::BK != 0) {
    // a panel would straddle two images: accumulate image by image
    for (int64_t b = 0; b < batch; ++b) {
      if (int st = tnh_sgemm(0, 1, M, N, L, alpha, A, aOff + b * strideA, lda, B, bOff + b * strideB, ldb,
                             b == 0 ? beta : 1.0f, C, cOff, ldc))
        return st;
    }
    return TNH_OK;
  }
  WgradArgs a{};
  a.A = A + aOff;
  a.B = B + bOff;
  a.C = C + cOff;
  a.M = M; a.N = N; a.L = L; a.lda = lda; a.ldb = ldb; a.ldc = ldc;
  a.strideA = strideA; a.strideB = strideB; a.batch = batch;
  a.aBytes = aElems * 4;
  a.bBytes = bElems * 4;
  a.alpha = alpha;
  a.beta = beta;
  if (int st = wgrad_split(cx, a, "sgemm_nt_batch_reduce")) return st;
  const bool va = aligned16(a.A) && lda % 4 == 0 && strideA % 4 == 0 && L % 4 == 0;
  const bool vb = aligned16(a.B) && ldb % 4 == 0 && strideB % 4 == 0 && L % 4 == 0;
  if (va && vb) return launch_wgrad<true, true>(a, cx->stream);
  if (va) return launch_wgrad<true, false>(a, cx->stream);
  if (vb) return launch_wgrad<false, true>(a, cx->stream);
  return launch_wgrad<false, false>(a, cx->stream);
}

namespace tnh {
namespace {
// tnh_conv2d_wgrad, or with pieces / nPieces (tnh_conv2d_wgrad_pieces) the
// split's raw sums written to the caller's memory instead of reduced into dW.
int32_t conv2d_wgrad_impl(int64_t batch, int64_t C, int64_t H, int64_t W, int64_t F, int64_t kh, int64_t kw,
                          int64_t padH, int64_t padW, int64_t strideY, int64_t strideX, int64_t dilY, int64_t dilX,
                          const float* x, int64_t xBatchStride, const float* delta, int64_t deltaBatchStride,
                          float alpha, float beta, float* dW, bool piecesMode, float* pieces, int64_t piecesFloats,
                          int32_t* nPieces) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(batch >= 0 && C > 0 && H > 0 && W > 0 && F > 0 && kh > 0 && kw > 0 && padH >= 0 && padW >= 0 &&
              strideY > 0 && strideX > 0 && dilY > 0 && dilX > 0,
          "conv2d_wgrad: bad geometry");
  TNH_ARG(x && delta && (piecesMode || dW), "conv2d_wgrad: NULL buffer");
  TNH_ARG(!piecesMode || nPieces, "conv2d_wgrad_pieces: NULL nPieces");
  const int64_t OH = (H + 2 * padH - dilY * (kh - 1) - 1) / strideY + 1;
  const int64_t OW = (W + 2 * padW - dilX * (kw - 1) - 1) / strideX + 1;
  TNH_ARG(OH > 0 && OW > 0, "conv2d_wgrad: empty output");
  const int64_t L = OH * OW, K = C * kh * kw;
  TNH_ARG(xBatchStride >= C * H * W && deltaBatchStride >= F * L, "conv2d_wgrad: batch strides too small");
  TNH_ARG(!piecesMode || batch > 0, "conv2d_wgrad_pieces: empty batch");
  if (batch == 0) return tnh_sgemm(0, 1, F, K, 0, alpha, x, 0, 1, x, 0, 1, beta, dW, 0, K);
  const int64_t xElems = (batch - 1) * xBatchStride + C * H * W;
  const int64_t dElems = (batch - 1) * deltaBatchStride + F * L;
  TNH_ARG(xElems * 4 <= kMaxBufBytes && dElems * 4 <= kMaxBufBytes && batch * L < (int64_t(1) << 31) &&
              K * F < (int64_t(1) << 31),
          "conv2d_wgrad: operands span more than 2 GiB (split the batch)");
  constexpr int BK = WCfg::BK;
  const bool fused = L % BK == 0 && OW % 4 == 0 && (OW % BK == 0 || BK % OW == 0);
  if (!fused && piecesMode)
    return fail(TNH_ERR_UNSUPPORTED, "conv2d_wgrad_pieces: needs OH*OW %% 32 == 0, OW %% 4 == 0 and OW | 32 or 32 | OW");
  if (!fused) {
    // the gather's panel geometry does not hold: im2col image by image into
    // the stream's workspace, then the NT product accumulated over images
    float* col = static_cast<float*>(workspace(cx, static_cast<size_t>(K * L) * 4));
    if (!col) return fail(TNH_ERR_OUT_OF_MEMORY, "conv2d_wgrad: no workspace for the column matrix");
    for (int64_t b = 0; b < batch; ++b) {
      if (int st = tnh_im2col(C, H, W, kh, kw, padH, padW, strideY, strideX, dilY, dilX, x, b * xBatchStride, col,
                              0))
        return st;
      if (int st = tnh_sgemm(0, 1, F, K, L, alpha, delta, b * deltaBatchStride, L, col, 0, L, b == 0 ? beta : 1.0f,
                             dW, 0, K))
        return st;
    }
    return TNH_OK;
  }
  WgradArgs a{};
  a.A = delta;
  a.B = x;
  a.C = dW;
  a.M = F; a.N = K; a.L = L; a.lda = L; a.ldb = 0; a.ldc = K;
  a.strideA = deltaBatchStride; a.strideB = xBatchStride; a.batch = batch;
  a.aBytes = dElems * 4;
  a.bBytes = xElems * 4;
  a.alpha = alpha;
  a.beta = beta;
  a.rawPieces = piecesMode ? 1 : 0;
  if (int st = wgrad_split(cx, a, "conv2d_wgrad")) return st;
  if (piecesMode) {
    // the update's pass sums a weight's pieces in one thread, in the order of
    // the thread-per-element reduction; the wave-per-element order of small
    // gradients is not reproduced there
    if (a.splits > 1 && F * K < kWaveReduceBelow)
      return fail(TNH_ERR_UNSUPPORTED, "conv2d_wgrad_pieces: %lld weights (below %lld) sum their pieces a wave each",
                  static_cast<long long>(F * K), static_cast<long long>(kWaveReduceBelow));
    *nPieces = a.splits;
    if (!pieces) return TNH_OK;  // the query: the number of pieces only
    TNH_ARG(piecesFloats >= static_cast<int64_t>(a.splits) * F * K,
            "conv2d_wgrad_pieces: %lld floats hold fewer than %d pieces of %lld", static_cast<long long>(piecesFloats),
            a.splits, static_cast<long long>(F * K));
    a.part = pieces;
  }
  ColGeom g{};
  g.xBatchStride = xBatchStride;
  g.xBytes = xElems * 4;
  g.C = static_cast<int>(C); g.H = static_cast<int>(H); g.W = static_cast<int>(W);
  g.OW = static_cast<int>(OW); g.L = static_cast<int>(L);
  g.kh = static_cast<int>(kh); g.kw = static_cast<int>(kw);
  g.sY = static_cast<int>(strideY); g.sX = static_cast<int>(strideX);
  g.pH = static_cast<int>(padH); g.pW = static_cast<int>(padW);
  g.dY = static_cast<int>(dilY); g.dX = static_cast<int>(dilX);
  const bool va = aligned16(delta) && L % 4 == 0 && deltaBatchStride % 4 == 0;
  if (va) return launch_wgrad_col<true>(a, g, cx->stream);
  return launch_wgrad_col<false>(a, g, cx->stream);
}
}  // namespace
}  // namespace tnh

extern "C" int32_t tnh_conv2d_wgrad(int64_t batch, int64_t C, int64_t H, int64_t W, int64_t F, int64_t kh,
                                    int64_t kw, int64_t padH, int64_t padW, int64_t strideY, int64_t strideX,
                                    int64_t dilY, int64_t dilX, const float* x, int64_t xBatchStride,
                                    const float* delta, int64_t deltaBatchStride, float alpha, float beta,
                                    float* dW) {
  return tnh::conv2d_wgrad_impl(batch, C, H, W, F, kh, kw, padH, padW, strideY, strideX, dilY, dilX, x, xBatchStride,
                                delta, deltaBatchStride, alpha, beta, dW, false, nullptr, 0, nullptr);
}

extern "C" int32_t tnh_conv2d_wgrad_pieces(int64_t batch, int64_t C, int64_t H, int64_t W, int64_t F, int64_t kh,
                                           int64_t kw, int64_t padH, int64_t padW, int64_t strideY, int64_t strideX,
                                           int64_t dilY, int64_t dilX, const float* x, int64_t xBatchStride,
                                           const float* delta, int64_t deltaBatchStride, float* pieces,
                                           int64_t piecesFloats, int32_t* nPieces) {
  return tnh::conv2d_wgrad_impl(batch, C, H, W, F, kh, kw, padH, padW, strideY, strideX, dilY, dilX, x, xBatchStride,
                                delta, deltaBatchStride, 1.0f, 1.0f, nullptr, true, pieces, piecesFloats, nPieces);
}

namespace {

// normalize_delta_fin_kernel over [groups][dstSize][block] (rows per
// workgroup <= kFinRows, checked by the caller)
int launch_normalize_fin(Context* cx, int64_t N, int64_t block, int64_t dstSize, int64_t groups, float* delta,
                         const float* x, const float* mean, const float* variance, const BnBackFin& fin, int P) {
  const bool v4 = block % 4 == 0 && rows_al16(delta) && rows_al16(x);
  const Rows g = make_rows(N, block, dstSize, v4 ? 4 : 1);
  const int64_t wgs = (g.rows + g.rpw - 1) / g.rpw;
  const float batchSize = static_cast<float>(block * groups);
  if (v4)
    hipLaunchKernelGGL(normalize_delta_fin_kernel<4>, dim3(static_cast<unsigned>(wgs)), dim3(kRowThreads), 0,
                       cx->stream, delta, x, g, batchSize, mean, variance, fin, P);
  else
    hipLaunchKernelGGL(normalize_delta_fin_kernel<1>, dim3(static_cast<unsigned>(wgs)), dim3(kRowThreads), 0,
                       cx->stream, delta, x, g, batchSize, mean, variance, fin, P);
  return launch_status("normalize_delta_fin_kernel");
}

// tnh_bn_backward with the layer's incoming delta taken from SRC (see
// BnBackOpT); w is the row width for kFromMaxPool2.
template <int SRC>
int bn_backward_impl(const char* who, int64_t N, int64_t dstSize, int64_t groups, int64_t w, const int64_t* pidx,
                     const float* pdel, const float* output, int32_t act, const float* xNorm, const float* x,
                     const float* scales, const float* mean, const float* variance, float* delta,
                     float* scaleUpdates, float* mean_delta, float* variance_delta, const float* biases) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(N > 0 && dstSize > 0 && groups > 0, "%s: bad sizes", who);
  // xNorm NULL: x_norm is formed from x, mean and variance in the first
  // pass; output NULL: the activation's output from x_norm, scales, biases
  TNH_ARG(x && scales && mean && variance && delta && scaleUpdates && mean_delta && variance_delta,
          "%s: NULL buffer", who);
  TNH_ARG(output || biases, "%s: give the output or the biases it is formed from", who);
  TNH_ARG(act == TNH_AC_LINEAR || act == TNH_AC_LEAKY || act == TNH_AC_LOGISTIC, "%s: activation %d", who, act);
  const int64_t block = N / (dstSize * groups);
  TNH_ARG(block * dstSize * groups == N, "%s: sizes do not align", who);
  ChanSplit s;
  float* red = nullptr;
  // three partials per workgroup slot: the dgamma dots after the two
  // mean / variance delta sums; then (8-byte aligned) a double per channel
  if (int st = chan_split(s, red, dstSize, block, groups, 6, cx)) return st;
  float* dotPart = red + 2 * dstSize * s.P;
  double* vpow = reinterpret_cast<double*>(red + ((3 * dstSize * s.P + 1) & ~int64_t(1)));
  const BnBackFin fin{MvdFin{red, variance, mean_delta, variance_delta}, dotPart, scaleUpdates, vpow};
  const bool v4 = block % 4 == 0 && rows_al16(delta) && rows_al16(x);
  const Rows g = make_rows(N, block, dstSize, v4 ? 4 : 1);
  const int64_t wgs = (g.rows + g.rpw - 1) / g.rpw;
  // many short rows (or P > 64): the finals in their own launch
  const bool fused = g.rpw <= kFinRows && s.P <= 64 && wgs < (int64_t(1) << 31);
  const bool vec = chan_vec(s, {delta, output ? output : x, xNorm ? xNorm : x});
  auto norm_in_pass = [&](auto& o) {  // x_norm from x, mean and variance; out from it
    if (!xNorm) {
      o.x = x;
      o.mean = mean;
      o.varN = variance;
      o.oneElem = block == 1;
    }
    if (!output) o.beta = biases;
  };
  if (fused && vec == chan_vec(s, {delta, x})) {
    // one pass: the first pass's dot and MvdOp's two sums (the same walk as
    // MvdOp's own pass, so the same partials), then the finals + normalize
    BnBackOpT<SRC, true> op{delta, output, xNorm, scales, act, 0.f};
    op.pidx = pidx;
    op.pdel = pdel;
    op.block = static_cast<uint32_t>(block);
    op.w = static_cast<uint32_t>(w);
    op.var = variance;
    op.vpow = vpow;
    op.x = x;
    op.mean = mean;
    norm_in_pass(op);
    if (int st = launch_partial<3>(cx, op, s, vec, red, "chan_partial_kernel<bn_back_mvd>")) return st;
    return launch_normalize_fin(cx, N, block, dstSize, groups, delta, x, mean, variance, fin, s.P);
  }
  BnBackOpT<SRC> op{delta, output, xNorm, scales, act, 0.f};
  op.pidx = pidx;
  op.pdel = pdel;
  op.block = static_cast<uint32_t>(block);
  op.w = static_cast<uint32_t>(w);
  norm_in_pass(op);
  if (fused) {
    op.var = variance;
    op.vpow = vpow;
  }
  if (int st = launch_partial<1>(cx, op, s, vec, dotPart, "chan_partial_kernel<bn_back>")) return st;
  if (!fused) {
    if (int st = launch_partial<2>(cx, MvdOp{delta, x, mean, 0.f}, s, chan_vec(s, {delta, x}), red,
                                   "chan_partial_kernel<mean_var_delta>", fin))
      return st;
    return tnh_normalize_delta(N, dstSize, groups, delta, x, 0, mean, variance, mean_delta, variance_delta);
  }
  if (int st = launch_partial<2>(cx, MvdOp{delta, x, mean, 0.f}, s, chan_vec(s, {delta, x}), red,
                                 "chan_partial_kernel<mean_var_delta>"))
    return st;
  return launch_normalize_fin(cx, N, block, dstSize, groups, delta, x, mean, variance, fin, s.P);
}

}  // namespace

extern "C" int32_t tnh_bn_backward(int64_t N, int64_t dstSize, int64_t groups, const float* output, int32_t act,
                                   const float* xNorm, const float* x, const float* scales, const float* mean,
                                   const float* variance, float* delta, float* scaleUpdates, float* mean_delta,
                                   float* variance_delta, const float* biases) {
  return bn_backward_impl<kFromDelta>("bn_backward", N, dstSize, groups, 0, nullptr, nullptr, output, act, xNorm, x,
                                      scales, mean, variance, delta, scaleUpdates, mean_delta, variance_delta,
                                      biases);
}

extern "C" int32_t tnh_bn_backward_maxpool(int64_t N, int64_t dstSize, int64_t groups, int64_t h, int64_t w,
                                           const int64_t* poolIndexes, const float* poolDelta, const float* output,
                                           int32_t act, const float* xNorm, const float* x, const float* scales,
                                           const float* mean, const float* variance, float* delta,
                                           float* scaleUpdates, float* mean_delta, float* variance_delta,
                                           const float* biases) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(h > 0 && w > 0 && h % 2 == 0 && w % 2 == 0 && groups > 0 && dstSize > 0 && N == groups * dstSize * h * w &&
              N < (int64_t(1) << 31),
          "bn_backward_maxpool: sizes (even h and w, N = groups * dstSize * h * w < 2^31)");
  TNH_ARG(poolIndexes && poolDelta, "bn_backward_maxpool: NULL buffer");
  // each index must name an element of its own window: only indexes that
  // a 2x2 stride-2 pool over exactly this input wrote qualify
  TNH_ARG(pool_is_2x2(poolIndexes, groups, dstSize, h, w),
          "bn_backward_maxpool: the indexes were not written by a 2x2 stride-2 maxpool of this geometry");
  return bn_backward_impl<kFromMaxPool2>("bn_backward_maxpool", N, dstSize, groups, w, poolIndexes, poolDelta, output,
                                         act, xNorm, x, scales, mean, variance, delta, scaleUpdates, mean_delta,
                                         variance_delta, biases);
}

extern "C" int32_t tnh_bn_backward_avgpool(int64_t N, int64_t dstSize, int64_t groups, const float* avgDelta,
                                           const float* output, int32_t act, const float* xNorm, const float* x,
                                           const float* scales, const float* mean, const float* variance,
                                           float* delta, float* scaleUpdates, float* mean_delta,
                                           float* variance_delta, const float* biases) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(N > 0 && N < (int64_t(1) << 31), "bn_backward_avgpool: 0 < N < 2^31");
  TNH_ARG(avgDelta, "bn_backward_avgpool: NULL buffer");
  return bn_backward_impl<kFromAvgPool>("bn_backward_avgpool", N, dstSize, groups, 0, nullptr, avgDelta, output, act,
                                        xNorm, x, scales, mean, variance, delta, scaleUpdates, mean_delta,
                                        variance_delta, biases);
}

extern "C" int32_t tnh_softmax_head_forward(int64_t batch, int64_t F, int64_t hw, int64_t classes, const float* x,
                                            float* avg, const float* weights, const float* biases,
                                            const float* truth, float* logits, float* prob, float* delta,
                                            float* error) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(batch > 0 && F > 0 && hw > 0 && classes > 0 && F <= 8192 && classes <= 1024 && batch < (int64_t(1) << 31),
          "softmax_head_forward: bad sizes");
  TNH_ARG(avg && weights && biases && truth && logits && prob && delta && error, "softmax_head_forward: NULL buffer");
  // the average pool as tnh_avgpool_fwd runs it (a wave per plane: more
  // parallel than a workgroup per image), then the rest per image; x NULL:
  // avg holds the averages already (tnh_bn_forward_avgpool)
  if (x) {
    hipLaunchKernelGGL(avgpool_fwd_kernel, dim3(static_cast<unsigned>((batch * F + 3) / 4)), dim3(256), 0,
                       cx->stream, x, batch * F, hw, avg);
    if (int st = launch_status("avgpool_fwd_kernel")) return st;
  }
  const bool stageW = classes * F <= 8192;  // up to 32 KB of weights in LDS
  const size_t lds = static_cast<size_t>(F + classes + (stageW ? classes * F : 0)) * 4;
  hipLaunchKernelGGL(softmax_head_fwd_kernel, dim3(static_cast<unsigned>(batch)), dim3(256), lds, cx->stream, F, hw,
                     classes, stageW, avg, weights, biases, truth, logits, prob, delta, error);
  return launch_status("softmax_head_fwd_kernel");
}

extern "C" int32_t tnh_softmax_head_backward(int64_t batch, int64_t F, int64_t hw, int64_t classes, float clampAlpha,
                                             float* delta, const float* avg, const float* weights,
                                             float* weightUpdates, float* biasUpdates, float* avgDelta,
                                             float* deltaIn) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(batch > 0 && F > 0 && hw > 0 && classes > 0 && F <= 8192 && classes <= 1024 &&
              batch + classes < (int64_t(1) << 31),
          "softmax_head_backward: bad sizes");
  TNH_ARG(delta && avg && weights && weightUpdates && biasUpdates && avgDelta, "softmax_head_backward: NULL buffer");
  const size_t lds = static_cast<size_t>(F + classes) * 4;
  hipLaunchKernelGGL(softmax_head_bwd_kernel, dim3(static_cast<unsigned>(batch + classes)), dim3(256), lds,
                     cx->stream, batch, F, hw, classes, clampAlpha, delta, avg, weights, weightUpdates, biasUpdates,
                     avgDelta, deltaIn);
  return launch_status("softmax_head_bwd_kernel");
}
