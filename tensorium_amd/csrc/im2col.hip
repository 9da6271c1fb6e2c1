// Standalone im2col / col2im (bit-exact data movement).
//
// im2col: one thread per column element, writes fully coalesced rows of col;
//   formula of sim2Col (ntensors.pas:11425-11463).
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

__global__ __launch_bounds__(256) void im2col_kernel(Geom g, const float* __restrict__ im, int64_t imStride,
                                                     float* __restrict__ col, int64_t colStride, int64_t total) {
  const int64_t b = blockIdx.y;
  const float* src = im + b * imStride;
  float* dst = col + b * colStride;
  const int64_t OHW = g.OH * g.OW;
  for (int64_t e = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; e < total; e += int64_t(gridDim.x) * blockDim.x) {
    const int64_t row = e / OHW, p = e - row * OHW;
    const int64_t oy = p / g.OW, ox = p - oy * g.OW;
    const int64_t c = row / (g.kh * g.kw), r = row - c * (g.kh * g.kw);
    const int64_t ky = r / g.kw, kx = r - ky * g.kw;
    const int64_t iy = -g.pH + ky * g.dY + oy * g.sY;
    const int64_t ix = -g.pW + kx * g.dX + ox * g.sX;
    float v = 0.f;
    if (static_cast<uint64_t>(iy) < static_cast<uint64_t>(g.H) && static_cast<uint64_t>(ix) < static_cast<uint64_t>(g.W))
      v = src[(c * g.H + iy) * g.W + ix];
    dst[e] = v;
  }
}

__global__ __launch_bounds__(256) void col2im_kernel(Geom g, const float* __restrict__ col, int64_t colStride,
                                                     float* __restrict__ im, int64_t imStride, int64_t total) {
  const int64_t b = blockIdx.y;
  const float* src = col + b * colStride;
  float* dst = im + b * imStride;
  const int64_t HW = g.H * g.W, OHW = g.OH * g.OW;
  for (int64_t e = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; e < total; e += int64_t(gridDim.x) * blockDim.x) {
    const int64_t c = e / HW, p = e - c * HW;
    const int64_t y = p / g.W, x = p - y * g.W;
    float v = dst[e];
    for (int64_t ky = 0; ky < g.kh; ++ky) {
      // c2i: iy = (ky - pH)*dY + oy*sY  ->  oy = (y - (ky - pH)*dY) / sY
      const int64_t ty = y - (ky - g.pH) * g.dY;
      if (ty < 0 || ty % g.sY) continue;
      const int64_t oy = ty / g.sY;
      if (oy >= g.OH) continue;
      for (int64_t kx = 0; kx < g.kw; ++kx) {
        const int64_t tx = x - (kx - g.pW) * g.dX;
        if (tx < 0 || tx % g.sX) continue;
        const int64_t ox = tx / g.sX;
        if (ox >= g.OW) continue;
        v = v + src[((c * g.kh + ky) * g.kw + kx) * OHW + oy * g.OW + ox];
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
  const int64_t total = C * kh * kw * g.OH * g.OW;
  hipLaunchKernelGGL(im2col_kernel, dim3(blocks_for(total), (unsigned)batch), dim3(256), 0, cx->stream, g,
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
  hipLaunchKernelGGL(col2im_kernel, dim3(blocks_for(total), (unsigned)batch), dim3(256), 0, cx->stream, g,
                     col + colOff, colStride, im + imOff, imStride, total);
  return launch_status("col2im_kernel");
}

extern "C" int32_t tnh_col2im(int64_t C, int64_t H, int64_t W, int64_t kh, int64_t kw, int64_t pH, int64_t pW,
                              int64_t sY, int64_t sX, int64_t dY, int64_t dX, const float* col, int64_t colOff,
                              float* im, int64_t imOff) {
  return tnh_col2im_batched(C, H, W, kh, kw, pH, pW, sY, sX, dY, dX, col, colOff, 0, im, imOff, 0, 1);
}
