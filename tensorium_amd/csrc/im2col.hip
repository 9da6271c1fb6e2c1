// Standalone im2col / col2im (bit-exact data movement).
//
// im2col: one thread per (channel, output pixel), writing the kh*kw rows of
//   its channel (coalesced along each row); formula of sim2Col
//   (ntensors.pas:11425-11463).
// col2im: a gather, one thread per image pixel.  The reference scatters
//   (c2i, ntensors.pas:11650-11715: rows i = (c*kh + ky)*kw + kx ascending,
//   each adding its value into im).  For a fixed pixel every row contributes
//   at most once, so the serial result is
//     im[c][y][x] + col[row(ky=0,kx=0)] + col[row(0,1)] + ...  (ky, kx ascending)
//   and a per-pixel loop in that order is bit-identical, with no atomics.
#include "common.hpp"

namespace tnh {
namespace {

struct Geom {
  int64_t C, H, W, kh, kw, pH, pW, sY, sX, dY, dX, OH, OW;
};

// One thread per (channel, output pixel): it reads the kh*kw window taps of
// its pixel and writes them to the kh*kw rows of the channel, so the stores
// of a wave are consecutive along each row and the index arithmetic is paid
// once per thread, not per element.  I is the index type (32-bit when every
// index fits).
template <class I>
__global__ __launch_bounds__(256) void im2col_kernel(Geom g, const float* __restrict__ im, int64_t imStride,
                                                     float* __restrict__ col, int64_t colStride, I total) {
  const int64_t b = blockIdx.y;
  const float* src = im + b * imStride;
  float* dst = col + b * colStride;
  const I OW = static_cast<I>(g.OW), OHW = static_cast<I>(g.OH * g.OW), H = static_cast<I>(g.H),
          W = static_cast<I>(g.W);
  const I kh = static_cast<I>(g.kh), kw = static_cast<I>(g.kw);
  for (I e = static_cast<I>(blockIdx.x) * 256 + threadIdx.x; e < total; e += static_cast<I>(gridDim.x) * 256) {
    const I c = e / OHW, p = e - c * OHW;
    const I oy = p / OW, ox = p - oy * OW;
    const I y0 = oy * static_cast<I>(g.sY) - static_cast<I>(g.pH);
    const I x0 = ox * static_cast<I>(g.sX) - static_cast<I>(g.pW);
    const float* plane = src + static_cast<int64_t>(c) * H * W;
    float* out = dst + static_cast<int64_t>(c) * kh * kw * OHW + p;
    for (I ky = 0; ky < kh; ++ky) {
      const I iy = y0 + ky * static_cast<I>(g.dY);
      const bool rowOk = iy >= 0 && iy < H;
      for (I kx = 0; kx < kw; ++kx) {
        const I ix = x0 + kx * static_cast<I>(g.dX);
        float v = 0.f;
        if (rowOk && ix >= 0 && ix < W) v = plane[static_cast<int64_t>(iy) * W + ix];
        out[static_cast<int64_t>(ky * kw + kx) * OHW] = v;
      }
    }
  }
}

template <class I>
__global__ __launch_bounds__(256) void col2im_kernel(Geom g, const float* __restrict__ col, int64_t colStride,
                                                     float* __restrict__ im, int64_t imStride, I total) {
  const int64_t b = blockIdx.y;
  const float* src = col + b * colStride;
  float* dst = im + b * imStride;
  const I HW = static_cast<I>(g.H * g.W), W = static_cast<I>(g.W), OHW = static_cast<I>(g.OH * g.OW);
  const I OW = static_cast<I>(g.OW), OH = static_cast<I>(g.OH), sY = static_cast<I>(g.sY), sX = static_cast<I>(g.sX);
  const I kh = static_cast<I>(g.kh), kw = static_cast<I>(g.kw);
  for (I e = static_cast<I>(blockIdx.x) * 256 + threadIdx.x; e < total; e += static_cast<I>(gridDim.x) * 256) {
    const I c = e / HW, p = e - c * HW;
    const I y = p / W, x = p - y * W;
    float v = dst[e];
    const float* rows = src + static_cast<int64_t>(c) * kh * kw * OHW;
    for (I ky = 0; ky < kh; ++ky) {
      // c2i: iy = (ky - pH)*dY + oy*sY  ->  oy = (y - (ky - pH)*dY) / sY
      const I ty = y - (ky - static_cast<I>(g.pH)) * static_cast<I>(g.dY);
      if (ty < 0) continue;
      const I oy = sY == 1 ? ty : ty / sY;
      if (oy * sY != ty || oy >= OH) continue;
      for (I kx = 0; kx < kw; ++kx) {
        const I tx = x - (kx - static_cast<I>(g.pW)) * static_cast<I>(g.dX);
        if (tx < 0) continue;
        const I ox = sX == 1 ? tx : tx / sX;
        if (ox * sX != tx || ox >= OW) continue;
        v = v + rows[static_cast<int64_t>(ky * kw + kx) * OHW + oy * OW + ox];
      }
    }
    dst[e] = v;
  }
}

int make_geom(Geom& g, int64_t C, int64_t H, int64_t W, int64_t kh, int64_t kw, int64_t pH, int64_t pW, int64_t sY,
              int64_t sX, int64_t dY, int64_t dX, const char* who) {
  TNH_ARG(C > 0 && H > 0 && W > 0 && kh > 0 && kw > 0, "%s: bad sizes", who);
  TNH_ARG(pH >= 0 && pW >= 0 && sY > 0 && sX > 0 && dY > 0 && dX > 0, "%s: bad pad/stride/dilation", who);
  g = Geom{C, H, W, kh, kw, pH, pW, sY, sX, dY, dX,
           (H + 2 * pH - (dY * (kh - 1) + 1)) / sY + 1, (W + 2 * pW - (dX * (kw - 1) + 1)) / sX + 1};
  TNH_ARG(g.OH > 0 && g.OW > 0, "%s: empty output", who);
  return TNH_OK;
}

unsigned blocks_for(int64_t total) {
  const int64_t b = (total + 255) / 256;
  return static_cast<unsigned>(b < 65536 ? b : 65536);
}

}  // namespace
}  // namespace tnh

extern "C" int32_t tnh_im2col_batched(int64_t C, int64_t H, int64_t W, int64_t kh, int64_t kw, int64_t pH, int64_t pW,
                                      int64_t sY, int64_t sX, int64_t dY, int64_t dX, const float* im, int64_t imOff,
                                      int64_t imStride, float* col, int64_t colOff, int64_t colStride,
                                      int64_t batch) {
  using namespace tnh;
  TNH_REQUIRE_CTX(cx);
  Geom g;
  if (int st = make_geom(g, C, H, W, kh, kw, pH, pW, sY, sX, dY, dX, "im2col")) return st;
  TNH_ARG(batch >= 0 && batch <= 65535, "im2col: batch %lld", (long long)batch);
  TNH_ARG(im && col && imOff >= 0 && colOff >= 0, "im2col: bad buffers");
  if (batch == 0) return TNH_OK;
  const int64_t total = C * g.OH * g.OW;  // (channel, output pixel) pairs
  const bool small = C * kh * kw * g.OH * g.OW + 256LL * 65536 < INT32_MAX && C * H * W < INT32_MAX;
  if (small)
    hipLaunchKernelGGL(im2col_kernel<int>, dim3(blocks_for(total), (unsigned)batch), dim3(256), 0, cx->stream, g,
                       im + imOff, imStride, col + colOff, colStride, static_cast<int>(total));
  else
    hipLaunchKernelGGL(im2col_kernel<int64_t>, dim3(blocks_for(total), (unsigned)batch), dim3(256), 0, cx->stream, g,
                       im + imOff, imStride, col + colOff, colStride, total);
  return launch_status("im2col_kernel");
}

extern "C" int32_t tnh_im2col(int64_t C, int64_t H, int64_t W, int64_t kh, int64_t kw, int64_t pH, int64_t pW,
                              int64_t sY, int64_t sX, int64_t dY, int64_t dX, const float* im, int64_t imOff,
                              float* col, int64_t colOff) {
  return tnh_im2col_batched(C, H, W, kh, kw, pH, pW, sY, sX, dY, dX, im, imOff, 0, col, colOff, 0, 1);
}

extern "C" int32_t tnh_col2im_batched(int64_t C, int64_t H, int64_t W, int64_t kh, int64_t kw, int64_t pH, int64_t pW,
                                      int64_t sY, int64_t sX, int64_t dY, int64_t dX, const float* col,
                                      int64_t colOff, int64_t colStride, float* im, int64_t imOff, int64_t imStride,
                                      int64_t batch) {
  using namespace tnh;
  TNH_REQUIRE_CTX(cx);
  Geom g;
  if (int st = make_geom(g, C, H, W, kh, kw, pH, pW, sY, sX, dY, dX, "col2im")) return st;
  TNH_ARG(batch >= 0 && batch <= 65535, "col2im: batch %lld", (long long)batch);
  TNH_ARG(im && col && imOff >= 0 && colOff >= 0, "col2im: bad buffers");
  if (batch == 0) return TNH_OK;
  const int64_t total = C * H * W;
  const bool small = C * kh * kw * g.OH * g.OW < INT32_MAX && total + 256LL * 65536 < INT32_MAX;
  if (small)
    hipLaunchKernelGGL(col2im_kernel<int>, dim3(blocks_for(total), (unsigned)batch), dim3(256), 0, cx->stream, g,
                       col + colOff, colStride, im + imOff, imStride, static_cast<int>(total));
  else
    hipLaunchKernelGGL(col2im_kernel<int64_t>, dim3(blocks_for(total), (unsigned)batch), dim3(256), 0, cx->stream, g,
                       col + colOff, colStride, im + imOff, imStride, total);
  return launch_status("col2im_kernel");
}

extern "C" int32_t tnh_col2im(int64_t C, int64_t H, int64_t W, int64_t kh, int64_t kw, int64_t pH, int64_t pW,
                              int64_t sY, int64_t sX, int64_t dY, int64_t dX, const float* col, int64_t colOff,
                              float* im, int64_t imOff) {
  return tnh_col2im_batched(C, H, W, kh, kw, pH, pW, sY, sX, dY, dX, col, colOff, 0, im, imOff, 0, 1);
}
