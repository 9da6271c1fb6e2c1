// The element-wise methods of TNNCuda<T> that serve layers around the
// convolution path (the LRN, logistic-cost, L2-cost, dropout, swish and
// scaled-yolo layers), one grid-stride kernel each.  Each element is the
// operation sequence the reference's CPU code (or, where the CPU code is a
// vendor library, TNNCuda's kernel) applies, in fp32 with no contraction
// (-ffp-contract=off): a*b + c is a multiply then an add.
#include <cmath>

#include "common.hpp"

namespace tnh {
namespace {

constexpr int kThreads = 256;
constexpr float kEps = 1e-6f;  // sEPSILON (ntensors.pas:95)

unsigned grid_for(int64_t n) {
  const int64_t b = (n + kThreads - 1) / kThreads;
  return static_cast<unsigned>(b < 16384 ? (b > 0 ? b : 1) : 16384);
}

#define GRID_STRIDE(i, n) \
  for (int64_t i = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; i < (n); i += int64_t(gridDim.x) * blockDim.x)

// dst[i*incc] = src1[i*inca] op src2[i*incb] (subv / mulv, cuda_sgemm.cu:789, 1664)
template <int OP>
__global__ void vv_kernel(int64_t n, const float* a, int64_t ia, const float* b, int64_t ib, float* c, int64_t ic) {
  GRID_STRIDE(i, n) {
    const float x = a[i * ia], y = b[i * ib];
    c[i * ic] = OP == 0 ? x - y : x * y;
  }
}

// dst = src1 * src2 + src3, a multiply then an add
__global__ void fmavv_kernel(int64_t n, const float* a, int64_t ia, const float* b, int64_t ib, const float* c,
                             int64_t ic, float* d, int64_t id) {
  GRID_STRIDE(i, n) {
    const float p = a[i * ia] * b[i * ib];
    d[i * id] = p + c[i * ic];
  }
}

// y = x^a: TTensor.power evaluates Math.Power in double (ntensors.pas:8507-8530)
__global__ void power_kernel(int64_t n, const float* x, int64_t ix, float a, float* y, int64_t iy) {
  GRID_STRIDE(i, n) y[i * iy] = static_cast<float>(pow(static_cast<double>(x[i * ix]), static_cast<double>(a)));
}

// FusedMultiplyAdd -> sfmavss (ntensors.pas:3355-3368): x * scale + bias,
// a multiply then an add
__global__ void fmavss_kernel(int64_t n, const float* src, float scalar, float bias, float* dst) {
  GRID_STRIDE(i, n) {
    const float p = src[i] * scalar;
    dst[i] = p + bias;
  }
}

// logistic cost (cuda_sgemm.cu:814-828), in single precision:
// error = -t log(max(p, eps)) - (1 - t) log(max(1 - p, eps)), delta = t - p
__global__ void ce_logistic_kernel(int64_t n, const float* pred, const float* truth, float* delta, float* error) {
  GRID_STRIDE(i, n) {
    const float t = truth[i], p = pred[i];
    const float a = -t * logf(fmaxf(p, kEps));
    const float b = (1.f - t) * logf(fmaxf(1.f - p, kEps));
    error[i] = a - b;
    delta[i] = t - p;
  }
}

// L2 cost (cuda_sgemm.cu:1655-1662): r = truth - pred, delta = r, error = r*r
__global__ void cost_l2_kernel(int64_t n, const float* pred, const float* truth, float* delta, float* error) {
  GRID_STRIDE(i, n) {
    const float r = truth[i] - pred[i];
    delta[i] = r;
    error[i] = r * r;
  }
}

// dst = 1 / sqrt(max(src, eps)) at stride and offset (cuda_sgemm.cu:1811-1817)
__global__ void inverse_sqrt_kernel(int64_t n, const float* src, float* dst, int64_t stride, int64_t offset) {
  GRID_STRIDE(i, n) {
    const int64_t e = i * stride + offset;
    dst[e] = 1.f / sqrtf(fmaxf(src[e], kEps));
  }
}

// SWISH (array_activate_swish, cuda_sgemm.cu:512-522; swishMP's Pascal loop,
// nactivation.pas:719-750): s = 1 / (1 + exp(-x)), outSigmoid = s, out = x*s
__global__ void swish_kernel(int64_t n, const float* x, float* outSigmoid, float* out) {
  GRID_STRIDE(i, n) {
    const float v = x[i];
    const float s = 1.f / (1.f + expf(-v));
    outSigmoid[i] = s;
    out[i] = v * s;
  }
}

// Dropout's uniform draw: element i of a call with seed s takes the top 24
// bits of splitmix64(s + i) (a counter-based hash, so any grid gives the same
// numbers), u = bits * 2^-24 in [0, 1).
__device__ inline float dropout_uniform(uint64_t seed, int64_t i) {
  uint64_t z = seed + static_cast<uint64_t>(i) * 0x9E3779B97F4A7C15ull + 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  z = z ^ (z >> 31);
  return static_cast<float>(z >> 40) * (1.f / 16777216.f);
}

// forward_dropout (cuda_sgemm.cu:1634-1645): rnd = u, dst = rnd < p ? 0 : src*scale
__global__ void dropout_fwd_kernel(int64_t n, uint64_t seed, float p, float scale, const float* src, float* rnd,
                                   float* dst) {
  GRID_STRIDE(i, n) {
    const float u = dropout_uniform(seed, i);
    rnd[i] = u;
    dst[i] = u < p ? 0.f : src[i] * scale;
  }
}

// backward_dropout (cuda_sgemm.cu:1647-1653): dst = rnd < p ? 0 : src*scale
__global__ void dropout_bwd_kernel(int64_t n, float p, float scale, const float* src, const float* rnd, float* dst) {
  GRID_STRIDE(i, n) dst[i] = rnd[i] < p ? 0.f : src[i] * scale;
}

}  // namespace
}  // namespace tnh

using namespace tnh;

namespace {

int vv(int op, int64_t N, const float* src1, int64_t o1, int64_t inca, const float* src2, int64_t o2, int64_t incb,
       float* dst, int64_t od, int64_t incc, const char* what) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(N >= 0 && o1 >= 0 && o2 >= 0 && od >= 0, "%s: bad sizes", what);
  if (N == 0) return TNH_OK;
  TNH_ARG(src1 && src2 && dst, "%s: NULL buffer", what);
  if (op == 0)
    hipLaunchKernelGGL(vv_kernel<0>, dim3(grid_for(N)), dim3(kThreads), 0, cx->stream, N, src1 + o1, inca, src2 + o2,
                       incb, dst + od, incc);
  else
    hipLaunchKernelGGL(vv_kernel<1>, dim3(grid_for(N)), dim3(kThreads), 0, cx->stream, N, src1 + o1, inca, src2 + o2,
                       incb, dst + od, incc);
  return launch_status(what);
}

}  // namespace

extern "C" int32_t tnh_subvv(int64_t N, const float* src1, int64_t src1Offset, int64_t inca, const float* src2,
                             int64_t src2Offset, int64_t incb, float* dst, int64_t dstOffset, int64_t incc) {
  return vv(0, N, src1, src1Offset, inca, src2, src2Offset, incb, dst, dstOffset, incc, "subvv");
}

extern "C" int32_t tnh_mulvv(int64_t N, const float* src1, int64_t src1Offset, int64_t inca, const float* src2,
                             int64_t src2Offset, int64_t incb, float* dst, int64_t dstOffset, int64_t incc) {
  return vv(1, N, src1, src1Offset, inca, src2, src2Offset, incb, dst, dstOffset, incc, "mulvv");
}

extern "C" int32_t tnh_fmavv(int64_t N, const float* src1, int64_t src1Offset, int64_t inca, const float* src2,
                             int64_t src2Offset, int64_t incb, const float* src3, int64_t src3Offset, int64_t incc,
                             float* dst, int64_t dstOffset, int64_t incd) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(N >= 0 && src1Offset >= 0 && src2Offset >= 0 && src3Offset >= 0 && dstOffset >= 0, "fmavv: bad sizes");
  if (N == 0) return TNH_OK;
  TNH_ARG(src1 && src2 && src3 && dst, "fmavv: NULL buffer");
  hipLaunchKernelGGL(fmavv_kernel, dim3(grid_for(N)), dim3(kThreads), 0, cx->stream, N, src1 + src1Offset, inca,
                     src2 + src2Offset, incb, src3 + src3Offset, incc, dst + dstOffset, incd);
  return launch_status("fmavv_kernel");
}

extern "C" int32_t tnh_power(int64_t N, const float* x, int64_t xOffset, int64_t incx, float a, float* y,
                             int64_t yOffset, int64_t incy) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(N >= 0 && xOffset >= 0 && yOffset >= 0, "power: bad sizes");
  if (N == 0) return TNH_OK;
  TNH_ARG(x && y, "power: NULL buffer");
  hipLaunchKernelGGL(power_kernel, dim3(grid_for(N)), dim3(kThreads), 0, cx->stream, N, x + xOffset, incx, a,
                     y + yOffset, incy);
  return launch_status("power_kernel");
}

extern "C" int32_t tnh_fmavss(int64_t N, const float* src, int64_t offset, float scalar, float bias, float* dst) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(N >= 0 && offset >= 0, "fmavss: bad sizes");
  if (N == 0) return TNH_OK;
  TNH_ARG(src && dst, "fmavss: NULL buffer");
  hipLaunchKernelGGL(fmavss_kernel, dim3(grid_for(N)), dim3(kThreads), 0, cx->stream, N, src + offset, scalar, bias,
                     dst + offset);
  return launch_status("fmavss_kernel");
}

extern "C" int32_t tnh_cross_entropy_logistic(int64_t N, const float* pred, const float* truth, float* delta,
                                              float* error) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(N >= 0, "cross_entropy_logistic: bad size");
  if (N == 0) return TNH_OK;
  TNH_ARG(pred && truth && delta && error, "cross_entropy_logistic: NULL buffer");
  hipLaunchKernelGGL(ce_logistic_kernel, dim3(grid_for(N)), dim3(kThreads), 0, cx->stream, N, pred, truth, delta,
                     error);
  return launch_status("ce_logistic_kernel");
}

extern "C" int32_t tnh_cost_l2(int64_t N, const float* pred, const float* truth, float* delta, float* error) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(N >= 0, "cost_l2: bad size");
  if (N == 0) return TNH_OK;
  TNH_ARG(pred && truth && delta && error, "cost_l2: NULL buffer");
  hipLaunchKernelGGL(cost_l2_kernel, dim3(grid_for(N)), dim3(kThreads), 0, cx->stream, N, pred, truth, delta, error);
  return launch_status("cost_l2_kernel");
}

extern "C" int32_t tnh_inverse_sqrt(int64_t N, float alpha, const float* src, float* dst, int64_t stride,
                                    int64_t offset) {
  (void)alpha;  // TNNCuda passes it and its kernel ignores it (nncuda.pas:1563-1573)
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(N >= 0 && stride >= 1 && offset >= 0, "inverse_sqrt: bad sizes");
  if (N == 0) return TNH_OK;
  TNH_ARG(src && dst, "inverse_sqrt: NULL buffer");
  hipLaunchKernelGGL(inverse_sqrt_kernel, dim3(grid_for(N)), dim3(kThreads), 0, cx->stream, N, src, dst, stride,
                     offset);
  return launch_status("inverse_sqrt_kernel");
}

extern "C" int32_t tnh_activate_swish(int64_t N, const float* x, int64_t offset, float* outSigmoid, float* out) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(N >= 0 && offset >= 0, "activate_swish: bad sizes");
  if (N == 0) return TNH_OK;
  TNH_ARG(x && outSigmoid && out, "activate_swish: NULL buffer");
  hipLaunchKernelGGL(swish_kernel, dim3(grid_for(N)), dim3(kThreads), 0, cx->stream, N, x + offset,
                     outSigmoid + offset, out + offset);
  return launch_status("swish_kernel");
}

extern "C" int32_t tnh_dropout_fwd(int64_t N, const float* src, float probability, float scale, int64_t seed,
                                   float* rnd, float* dst) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(N >= 0, "dropout_fwd: bad size");
  if (N == 0) return TNH_OK;
  TNH_ARG(src && rnd && dst, "dropout_fwd: NULL buffer");
  hipLaunchKernelGGL(dropout_fwd_kernel, dim3(grid_for(N)), dim3(kThreads), 0, cx->stream, N,
                     static_cast<uint64_t>(seed), probability, scale, src, rnd, dst);
  return launch_status("dropout_fwd_kernel");
}

extern "C" int32_t tnh_dropout_bwd(int64_t N, const float* src, float probability, float scale, const float* rnd,
                                   float* dst) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(N >= 0, "dropout_bwd: bad size");
  if (N == 0) return TNH_OK;
  TNH_ARG(src && rnd && dst, "dropout_bwd: NULL buffer");
  hipLaunchKernelGGL(dropout_bwd_kernel, dim3(grid_for(N)), dim3(kThreads), 0, cx->stream, N, probability, scale,
                     src, rnd, dst);
  return launch_status("dropout_bwd_kernel");
}
