// Bandwidth-bound element-wise kernels: bias / scale epilogues, activations,
// BLAS-1 helpers, route (concat) copies and the unfused BN normalize.  Each
// element is produced by exactly the single fp32 operation the reference CPU
// path applies (bit-exact), with grid-stride loops over 64-bit indices.
#include "common.hpp"

namespace tnh {
namespace {

constexpr int kThreads = 256;

unsigned grid_for(int64_t n) {
  const int64_t b = (n + kThreads - 1) / kThreads;
  return static_cast<unsigned>(b < 16384 ? (b > 0 ? b : 1) : 16384);
}

#define GRID_STRIDE(i, n) \
  for (int64_t i = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; i < (n); i += int64_t(gridDim.x) * blockDim.x)

// vsAddB (ntensors.pas:4066) / forward_bias: x += bias[(i / block) % nb]
__global__ void bias_kernel(float* x, int64_t n, int64_t block, int64_t nb, const float* b, int64_t incb) {
  GRID_STRIDE(i, n) {
    const int64_t f = (i / block) % nb;
    x[i] = b[f * incb] + x[i];
  }
}

__global__ void scale_blk_kernel(float* x, int64_t n, int64_t block, int64_t nb, const float* s, int64_t incb) {
  GRID_STRIDE(i, n) {
    const int64_t f = (i / block) % nb;
    x[i] = s[f * incb] * x[i];
  }
}

// backward_bias: dst[f] += sum over (b, j) of src[(b*nb + f)*block + j];
// one workgroup per filter, deterministic tree reduction.
__global__ __launch_bounds__(256) void backward_bias_kernel(float* dst, int64_t nb, int64_t block, const float* src,
                                                             int64_t batch) {
  __shared__ float part[256];
  const int64_t f = blockIdx.x;
  float s = 0.f;
  for (int64_t b = 0; b < batch; ++b) {
    const float* p = src + (b * nb + f) * block;
    for (int64_t j = threadIdx.x; j < block; j += blockDim.x) s = s + p[j];
  }
  part[threadIdx.x] = s;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if (threadIdx.x < w) part[threadIdx.x] = part[threadIdx.x] + part[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) dst[f] = dst[f] + part[0];
}

__device__ inline float act_fwd(float v, int act) {
  if (act == TNH_AC_LEAKY) return 0.f > v ? 0.1f * v : v;  // leaky_array (nactivation.pas:234-268)
  if (act == TNH_AC_LOGISTIC) return 1.f / (1.f + expf(-v));
  return v;
}

__global__ void activate_kernel(float* x, int64_t n, int act) {
  GRID_STRIDE(i, n) x[i] = act_fwd(x[i], act);
}

// gradient_array: leaky_gradient (nactivation.pas:472-476); logistic y(1-y)
__global__ void derive_kernel(const float* x, int64_t n, int act, float* delta) {
  GRID_STRIDE(i, n) {
    const float v = x[i];
    float g = 1.f;
    if (act == TNH_AC_LEAKY) g = v > 0.f ? 1.f : 0.1f;
    if (act == TNH_AC_LOGISTIC) g = (1.f - v) * v;
    delta[i] = delta[i] * g;
  }
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

// _snormblkvv with IEEE division (ntensors.pas:4357, snormvss :4315):
// x = (x - m) / max(sqrt(v), 1e-6)
__global__ void bn_norm_kernel(float* x, int64_t n, int64_t block, int64_t nb, const float* mean, const float* var) {
  GRID_STRIDE(i, n) {
    const int64_t f = (i / block) % nb;
    float d = sqrtf(var[f]);
    d = d > 1e-6f ? d : 1e-6f;
    const float t = x[i] - mean[f];
    x[i] = t / d;
  }
}

// logistic_array's exp approximation (nactivation.pas:36-127), IEEE reciprocal
__device__ inline float logistic_poly(float x) {
  const float l2e = 1.442695041f, c0 = 1.00172476f, c1 = 0.657636276f, c2 = 0.3371894346f;
  const float mx = 8.872283E+001f, mn = -8.733654E+001f;
  float t = 0.f - x;
  if (t >= mx) t = mx;
  if (t <= mn) t = mn;
  t = l2e * t;
  const float fi = floorf(t);
  const float f = t - fi;
  const int i = static_cast<int>(fi);
  float p = __builtin_fmaf(f, c2, c1);
  p = __builtin_fmaf(p, f, c0);
  const float e = __int_as_float(__float_as_int(p) + static_cast<int>(static_cast<unsigned>(i) << 23));
  const float d = e + 1.f;
  return 1.f / d;
}

__global__ void yolo_kernel(int64_t total, int64_t HW, int64_t entries, const float* in, float* out) {
  GRID_STRIDE(e, total) {
    const int64_t entry = (e / HW) % entries;  // channel within the anchor group
    const float v = in[e];
    out[e] = (entry == 2 || entry == 3) ? v : logistic_poly(v);
  }
}

bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

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
      dst[static_cast<int64_t>(c) * HW + p] = (entry == 2 || entry == 3) ? x : logistic_poly(x);
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
  hipLaunchKernelGGL(bias_kernel, dim3(grid_for(dstSize)), dim3(kThreads), 0, cx->stream, dst + offset, dstSize, block,
                     srcSize, src, incb);
  return launch_status("bias_kernel");
}

extern "C" int32_t tnh_forward_scale(int64_t dstSize, float* dst, int64_t offset, int64_t scaleSize,
                                     const float* scale, int64_t incb, int64_t batch) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(dstSize >= 0 && scaleSize > 0 && batch > 0 && offset >= 0, "forward_scale: bad sizes");
  if (dstSize == 0) return TNH_OK;
  TNH_ARG(dst && scale, "forward_scale: NULL buffer");
  const int64_t block = dstSize / (scaleSize * batch);
  TNH_ARG(block * scaleSize * batch == dstSize, "forward_scale: sizes do not align");
  hipLaunchKernelGGL(scale_blk_kernel, dim3(grid_for(dstSize)), dim3(kThreads), 0, cx->stream, dst + offset, dstSize,
                     block, scaleSize, scale, incb);
  return launch_status("scale_blk_kernel");
}

extern "C" int32_t tnh_backward_bias(int64_t dstSize, float* dst, int64_t srcSize, const float* src, int64_t srcOffset,
                                     int64_t incb, int64_t batch) {
  (void)incb;
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(dstSize > 0 && srcSize >= 0 && batch > 0 && srcOffset >= 0, "backward_bias: bad sizes");
  TNH_ARG(dst && src, "backward_bias: NULL buffer");
  const int64_t block = srcSize / (dstSize * batch);
  TNH_ARG(block * dstSize * batch == srcSize, "backward_bias: sizes do not align");
  TNH_ARG(dstSize <= INT32_MAX, "backward_bias: too many filters");
  hipLaunchKernelGGL(backward_bias_kernel, dim3((unsigned)dstSize), dim3(256), 0, cx->stream, dst, dstSize, block,
                     src + srcOffset, batch);
  return launch_status("backward_bias_kernel");
}

extern "C" int32_t tnh_activate(int64_t N, float* x, int64_t offset, int32_t act) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(N >= 0 && offset >= 0, "activate: bad size");
  TNH_ARG(act == TNH_AC_LINEAR || act == TNH_AC_LEAKY || act == TNH_AC_LOGISTIC,
          "activate: unsupported activation %d", act);
  if (N == 0 || act == TNH_AC_LINEAR) return TNH_OK;  // acLINEAR: no launch (nncuda.pas:533)
  TNH_ARG(x != nullptr, "activate: NULL buffer");
  hipLaunchKernelGGL(activate_kernel, dim3(grid_for(N)), dim3(kThreads), 0, cx->stream, x + offset, N, act);
  return launch_status("activate_kernel");
}

extern "C" int32_t tnh_derive(int64_t N, const float* x, int64_t offset, int32_t act, float* delta) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(N >= 0 && offset >= 0, "derive: bad size");
  TNH_ARG(act == TNH_AC_LINEAR || act == TNH_AC_LEAKY || act == TNH_AC_LOGISTIC, "derive: unsupported activation %d",
          act);
  if (N == 0 || act == TNH_AC_LINEAR) return TNH_OK;
  TNH_ARG(x && delta, "derive: NULL buffer");
  hipLaunchKernelGGL(derive_kernel, dim3(grid_for(N)), dim3(kThreads), 0, cx->stream, x + offset, N, act, delta);
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
  hipLaunchKernelGGL(fill_kernel, dim3(grid_for(N)), dim3(kThreads), 0, cx->stream, N, x + offset, val, stride);
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
  hipLaunchKernelGGL(bn_norm_kernel, dim3(grid_for(dstSize)), dim3(kThreads), 0, cx->stream, x + offset, dstSize,
                     block, N, mean, variance);
  return launch_status("bn_norm_kernel");
}
