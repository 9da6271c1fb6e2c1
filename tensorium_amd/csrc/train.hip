// Training-direction kernels of the convolution path: batch-norm statistics
// and their deltas, softmax cross-entropy, average pooling, delta clamping,
// the fused SGD update and the weight-gradient GEMM of conv backward.
//
// Channel reductions run one workgroup per channel with a fixed-order tree
// (deterministic run to run); element-wise formulas follow the reference
// CPU operation order exactly (no contraction: the build uses
// -ffp-contract=off, FMAs are explicit where the reference fuses).
#include <algorithm>
#include <cmath>

#include "common.hpp"
#include "gemm_core.hpp"

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

// Element (b, i, k) of a [groups][nch][block] view lives at (b*nch + i)*block + k.
// MeansAndVars (ntensors.pas:9102-9180): mean over groups*block values, then
// the residual sum of squares about the fp32 mean divided by (S - 1).
__global__ __launch_bounds__(kRed) void means_vars_kernel(const float* src, int64_t nch, int64_t block,
                                                          int64_t groups, float* means, float* vars) {
  __shared__ float sh[kRed];
  const int64_t i = blockIdx.x;
  float s = 0.f;
  for (int64_t b = 0; b < groups; ++b) {
    const float* p = src + (b * nch + i) * block;
    for (int64_t k = threadIdx.x; k < block; k += kRed) s = s + p[k];
  }
  const float S = static_cast<float>(groups * block);
  const float m = block_sum(s, sh) / S;
  float v = 0.f;
  for (int64_t b = 0; b < groups; ++b) {
    const float* p = src + (b * nch + i) * block;
    for (int64_t k = threadIdx.x; k < block; k += kRed) {
      const float d = p[k] - m;
      v = v + d * d;
    }
  }
  const float rss = block_sum(v, sh);
  if (threadIdx.x == 0) {
    means[i] = m;
    vars[i] = rss / static_cast<float>(groups * block - 1);
  }
}

// sMeanAndVarianceDelta (ntensors.pas:8831-8898).
__global__ __launch_bounds__(kRed) void means_vars_delta_kernel(const float* delta, const float* x, int64_t nch,
                                                                int64_t block, int64_t groups, const float* mean,
                                                                const float* variance, float* mean_delta,
                                                                float* variance_delta) {
  __shared__ float sh[kRed];
  const int64_t i = blockIdx.x;
  const float mu = mean[i];
  float sm = 0.f, sv = 0.f;
  for (int64_t b = 0; b < groups; ++b) {
    const int64_t base = (b * nch + i) * block;
    for (int64_t k = threadIdx.x; k < block; k += kRed) {
      const float d = delta[base + k];
      sm = sm + d;
      sv = sv + d * (x[base + k] - mu);
    }
  }
  const float m = block_sum(sm, sh);
  const float v = block_sum(sv, sh);
  if (threadIdx.x == 0) {
    const float vc = fmaxf(variance[i], kEps);
    mean_delta[i] = m * (-1.0f / sqrtf(vc));
    // Power(max(var, eps), -3/2) is evaluated in double and the product stored as single
    variance_delta[i] = static_cast<float>(static_cast<double>(v) * -0.5 * pow(static_cast<double>(vc), -1.5));
  }
}

// sNormalizeDelta (ntensors.pas:8900-8960), element order of
// sNormalizeDelta_pas/_avx: d / std + ((x - mean) * vd + md).
__global__ void normalize_delta_kernel(float* delta, const float* x, int64_t n, int64_t nch, int64_t block,
                                       float batchSize, const float* mean, const float* variance,
                                       const float* mean_delta, const float* variance_delta) {
  GRID_STRIDE(e, n) {
    const int64_t i = (e / block) % nch;
    const float md = mean_delta[i] / batchSize;
    const float vd = (2.0f * variance_delta[i]) / batchSize;
    const float sd = sqrtf(fmaxf(variance[i], kEps));
    float t = (x[e] - mean[i]) * vd;
    t = t + md;
    delta[e] = delta[e] / sd + t;
  }
}

// addDots (ntensors.pas:7783-7830): dst[i] += sum over (b, k) of a*b.
__global__ __launch_bounds__(kRed) void add_dots_kernel(const float* a, const float* b, int64_t nch, int64_t block,
                                                        int64_t groups, float* dst) {
  __shared__ float sh[kRed];
  const int64_t i = blockIdx.x;
  float s = 0.f;
  for (int64_t g = 0; g < groups; ++g) {
    const int64_t base = (g * nch + i) * block;
    for (int64_t k = threadIdx.x; k < block; k += kRed) s = s + a[base + k] * b[base + k];
  }
  const float t = block_sum(s, sh);
  if (threadIdx.x == 0) dst[i] = dst[i] + t;
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
__global__ __launch_bounds__(kRed) void avgpool_fwd_kernel(const float* in, int64_t hw, float* out) {
  __shared__ float sh[kRed];
  const int64_t r = blockIdx.x;
  const float* p = in + r * hw;
  float s = 0.f;
  for (int64_t k = threadIdx.x; k < hw; k += kRed) s = s + p[k];
  const float t = block_sum(s, sh);
  if (threadIdx.x == 0) out[r] = t / static_cast<float>(hw);
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

__global__ void wgrad_reduce_kernel(WgradArgs a) {
  const int64_t total = a.M * a.N;
  GRID_STRIDE(e, total) {
    float v = a.part[e];
    for (int s = 1; s < a.splits; ++s) v = v + a.part[s * total + e];
    const int64_t r = e / a.N, c = e - r * a.N;
    float* p = a.C + r * a.ldc + c;
    float out = a.alpha * v;
    if (a.beta != 0.f) out = out + a.beta * *p;
    *p = out;
  }
}

using WCfg = TileCfg<64, 64, 32, 2, 2, 2>;

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

template <bool VA, bool VB>
int launch_wgrad(WgradArgs a, hipStream_t s) {
  dim3 grid(static_cast<unsigned>(a.tilesM * a.tilesN), static_cast<unsigned>(a.splits));
  hipLaunchKernelGGL((wgrad_kernel<WCfg, VA, VB>), grid, dim3(WCfg::NT), 0, s, a);
  if (int st = launch_status("wgrad_kernel")) return st;
  if (a.splits > 1) {
    hipLaunchKernelGGL(wgrad_reduce_kernel, dim3(grid_1d(a.M * a.N)), dim3(256), 0, s, a);
    return launch_status("wgrad_reduce_kernel");
  }
  return TNH_OK;
}

}  // namespace
}  // namespace tnh

using namespace tnh;

extern "C" int32_t tnh_means_vars(int64_t srcSize, int64_t dstSize, int64_t groups, const float* src,
                                  int64_t offset, float* means, float* vars) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(dstSize > 0 && groups > 0 && srcSize > 0 && offset >= 0, "means_vars: bad sizes");
  TNH_ARG(src && means && vars, "means_vars: NULL buffer");
  const int64_t block = srcSize / (dstSize * groups);
  TNH_ARG(block * dstSize * groups == srcSize && groups * block > 1, "means_vars: sizes do not align");
  hipLaunchKernelGGL(means_vars_kernel, dim3(static_cast<unsigned>(dstSize)), dim3(kRed), 0, cx->stream,
                     src + offset, dstSize, block, groups, means, vars);
  return launch_status("means_vars_kernel");
}

extern "C" int32_t tnh_means_vars_delta(int64_t srcSize, int64_t dstSize, int64_t groups, const float* delta,
                                        const float* x, int64_t offset, const float* mean, const float* variance,
                                        float* mean_delta, float* variance_delta) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(dstSize > 0 && groups > 0 && srcSize > 0 && offset >= 0, "means_vars_delta: bad sizes");
  TNH_ARG(delta && x && mean && variance && mean_delta && variance_delta, "means_vars_delta: NULL buffer");
  const int64_t block = srcSize / (dstSize * groups);
  TNH_ARG(block * dstSize * groups == srcSize, "means_vars_delta: sizes do not align");
  hipLaunchKernelGGL(means_vars_delta_kernel, dim3(static_cast<unsigned>(dstSize)), dim3(kRed), 0, cx->stream,
                     delta + offset, x + offset, dstSize, block, groups, mean, variance, mean_delta, variance_delta);
  return launch_status("means_vars_delta_kernel");
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
  hipLaunchKernelGGL(normalize_delta_kernel, dim3(grid_1d(deltaSize)), dim3(256), 0, cx->stream, delta + offset,
                     x + offset, deltaSize, meanSize, block, batchSize, mean, variance, mean_delta, variance_delta);
  return launch_status("normalize_delta_kernel");
}

extern "C" int32_t tnh_add_dots(int64_t N, int64_t dstSize, int64_t groups, const float* src1, const float* src2,
                                int64_t srcOffset, float* dst) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(N > 0 && dstSize > 0 && groups > 0 && srcOffset >= 0, "add_dots: bad sizes");
  TNH_ARG(src1 && src2 && dst, "add_dots: NULL buffer");
  const int64_t block = N / (dstSize * groups);
  TNH_ARG(block * dstSize * groups == N, "add_dots: sizes do not align");
  hipLaunchKernelGGL(add_dots_kernel, dim3(static_cast<unsigned>(dstSize)), dim3(kRed), 0, cx->stream,
                     src1 + srcOffset, src2 + srcOffset, dstSize, block, groups, dst);
  return launch_status("add_dots_kernel");
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
  hipLaunchKernelGGL(avgpool_fwd_kernel, dim3(static_cast<unsigned>(batch * c)), dim3(kRed), 0, cx->stream, input,
                     h * w, output);
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
  a.tilesM = static_cast<int>((M + WCfg::BM - 1) / WCfg::BM);
  a.tilesN = static_cast<int>((N + WCfg::BN - 1) / WCfg::BN);
  const int64_t tiles = static_cast<int64_t>(a.tilesM) * a.tilesN;
  TNH_ARG(tiles < (int64_t(1) << 31), "sgemm_nt_batch_reduce: grid too large");
  const int64_t panels = batch * L / WCfg::BK;
  int64_t splits = (2 * cx->cu_count + tiles - 1) / tiles;
  splits = std::max<int64_t>(1, std::min<int64_t>({splits, panels / 4, 1024}));
  a.kChunk = (panels + splits - 1) / splits * WCfg::BK;
  a.splits = static_cast<int>((batch * L + a.kChunk - 1) / a.kChunk);
  if (a.splits > 1) {
    a.part = static_cast<float*>(workspace(cx, static_cast<size_t>(a.splits) * M * N * 4));
    if (!a.part) {  // no scratch (e.g. under graph capture without a prior eager call)
      a.splits = 1;
      a.kChunk = batch * L;
    }
  }
  const bool va = aligned16(a.A) && lda % 4 == 0 && strideA % 4 == 0 && L % 4 == 0;
  const bool vb = aligned16(a.B) && ldb % 4 == 0 && strideB % 4 == 0 && L % 4 == 0;
  if (va && vb) return launch_wgrad<true, true>(a, cx->stream);
  if (va) return launch_wgrad<true, false>(a, cx->stream);
  if (vb) return launch_wgrad<false, true>(a, cx->stream);
  return launch_wgrad<false, false>(a, cx->stream);
}
