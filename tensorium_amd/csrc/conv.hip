// Fused convolution forward: implicit-GEMM (im2col gathered straight into
// LDS) on MFMA with the bias + activation (+ shortcut) epilogue applied to
// the accumulators before the single write of the output.
//
// GEMM view (Conv2D, ntensors.pas:8252-8345, batch merged into N):
//   M = F filters, N = batch*OH*OW, K = C*kh*kw
//   A = weights [F][K] row-major (filter-major, nConvolutionLayer.pas:206)
//   B = im2col(x) gathered on the fly
// Epilogue per element (reference order, nConvolutionLayer.pas:508-545 and
// naddlayer.pas:698):  v = acc + bias[f];  v = act(v);  v = v + residual.
#include "common.hpp"
#include "gemm_core.hpp"

namespace tnh {
namespace {

struct ConvArgs {
  const float* x;
  int64_t xBatchStride;
  const float* w;
  const float* bias;
  const float* res;
  int64_t rBatchStride;
  float* out;
  int64_t outBatchStride;
  int64_t F, N, K;
  int C, H, W, OW, OHW;
  int sY, sX, pH, pW;
  int act;
  int tilesM, tilesN;
};

__device__ inline float apply_act(float v, int act) {
  if (act == TNH_AC_LEAKY) return v < 0.f ? 0.1f * v : v;  // leaky_array (nactivation.pas:234)
  if (act == TNH_AC_LOGISTIC) return 1.f / (1.f + expf(-v));
  return v;
}

template <class Cfg, int KH, int KW, bool VA>
__global__ __launch_bounds__(Cfg::NT) void conv_gather_kernel(ConvArgs a) {
  using AL = DenseLoader<true, VA, Cfg::BM, Cfg::NT>;
  using BL = ConvGatherLoader<KH, KW, Cfg::BN, Cfg::NT>;
  using Main = GemmMainloop<Cfg, AL, BL>;
  __shared__ __attribute__((aligned(16))) float lds[Main::LDS_FLOATS];

  int tm, tn;
  tile_coords(blockIdx.x, a.tilesM, a.tilesN, tm, tn);
  const int64_t m0 = static_cast<int64_t>(tm) * Cfg::BM, n0 = static_cast<int64_t>(tn) * Cfg::BN;

  AL al;
  al.base = a.w;
  al.ld = a.K;
  al.rows = a.F;
  al.K = a.K;
  BL bl;
  bl.x = a.x;
  bl.xBatchStride = a.xBatchStride;
  bl.H = a.H; bl.W = a.W; bl.OW = a.OW; bl.OHW = a.OHW;
  bl.sY = a.sY; bl.sX = a.sX; bl.pH = a.pH; bl.pW = a.pW;
  bl.N = a.N; bl.K = a.K;
  bl.init_col(n0, threadIdx.x);

  f32x16 acc[Cfg::FM][Cfg::FN];
  Main::run(al, bl, m0, n0, 0, a.K, lds, acc);

  Main::for_each(acc, [&](int row, int col, float v) {
    const int64_t f = m0 + row, n = n0 + col;
    if (f < a.F && n < a.N) {
      const int64_t b = n / a.OHW, p = n - b * a.OHW;
      if (a.bias) v = v + a.bias[f];
      v = apply_act(v, a.act);
      if (a.res) v = v + a.res[b * a.rBatchStride + f * a.OHW + p];
      a.out[b * a.outBatchStride + f * a.OHW + p] = v;
    }
  });
}

template <class Cfg, bool VA, bool VB>
__global__ __launch_bounds__(Cfg::NT) void conv1x1_kernel(ConvArgs a) {
  using AL = DenseLoader<true, VA, Cfg::BM, Cfg::NT>;
  using BL = Conv1x1Loader<VB, Cfg::BN, Cfg::NT>;
  using Main = GemmMainloop<Cfg, AL, BL>;
  __shared__ __attribute__((aligned(16))) float lds[Main::LDS_FLOATS];

  int tm, tn;
  tile_coords(blockIdx.x, a.tilesM, a.tilesN, tm, tn);
  const int64_t m0 = static_cast<int64_t>(tm) * Cfg::BM, n0 = static_cast<int64_t>(tn) * Cfg::BN;

  AL al;
  al.base = a.w;
  al.ld = a.K;
  al.rows = a.F;
  al.K = a.K;
  BL bl;
  bl.x = a.x;
  bl.xBatchStride = a.xBatchStride;
  bl.HW = a.OHW;
  bl.N = a.N;
  bl.K = a.K;
  bl.init_col(n0, threadIdx.x);

  f32x16 acc[Cfg::FM][Cfg::FN];
  Main::run(al, bl, m0, n0, 0, a.K, lds, acc);

  Main::for_each(acc, [&](int row, int col, float v) {
    const int64_t f = m0 + row, n = n0 + col;
    if (f < a.F && n < a.N) {
      const int64_t b = n / a.OHW, p = n - b * a.OHW;
      if (a.bias) v = v + a.bias[f];
      v = apply_act(v, a.act);
      if (a.res) v = v + a.res[b * a.rBatchStride + f * a.OHW + p];
      a.out[b * a.outBatchStride + f * a.OHW + p] = v;
    }
  });
}

using Cfg128 = TileCfg<128, 128, 2, 2>;
using Cfg64 = TileCfg<64, 64, 2, 2>;
using Cfg64x128 = TileCfg<64, 128, 2, 2>;

template <class Cfg>
int grid_for(ConvArgs& a, dim3& grid) {
  const int64_t tm = (a.F + Cfg::BM - 1) / Cfg::BM, tn = (a.N + Cfg::BN - 1) / Cfg::BN;
  if (tm * tn > INT32_MAX) return fail(TNH_ERR_UNSUPPORTED, "conv2d: grid too large");
  a.tilesM = static_cast<int>(tm);
  a.tilesN = static_cast<int>(tn);
  grid = dim3(static_cast<unsigned>(tm * tn));
  return TNH_OK;
}

template <class Cfg, int KH, int KW>
int launch_gather(ConvArgs a, bool va, hipStream_t s) {
  dim3 grid;
  if (int st = grid_for<Cfg>(a, grid)) return st;
  if (va)
    hipLaunchKernelGGL((conv_gather_kernel<Cfg, KH, KW, true>), grid, dim3(Cfg::NT), 0, s, a);
  else
    hipLaunchKernelGGL((conv_gather_kernel<Cfg, KH, KW, false>), grid, dim3(Cfg::NT), 0, s, a);
  return launch_status("conv_gather_kernel");
}

template <class Cfg>
int launch_1x1(ConvArgs a, bool va, bool vb, hipStream_t s) {
  dim3 grid;
  if (int st = grid_for<Cfg>(a, grid)) return st;
  if (va && vb)
    hipLaunchKernelGGL((conv1x1_kernel<Cfg, true, true>), grid, dim3(Cfg::NT), 0, s, a);
  else if (va)
    hipLaunchKernelGGL((conv1x1_kernel<Cfg, true, false>), grid, dim3(Cfg::NT), 0, s, a);
  else if (vb)
    hipLaunchKernelGGL((conv1x1_kernel<Cfg, false, true>), grid, dim3(Cfg::NT), 0, s, a);
  else
    hipLaunchKernelGGL((conv1x1_kernel<Cfg, false, false>), grid, dim3(Cfg::NT), 0, s, a);
  return launch_status("conv1x1_kernel");
}

template <class Cfg>
int launch_any(const ConvArgs& a, int k, bool is1x1, bool va, bool vb, hipStream_t s) {
  if (is1x1) return launch_1x1<Cfg>(a, va, vb, s);
  if (k == 3) return launch_gather<Cfg, 3, 3>(a, va, s);
  if (k == 1) return launch_gather<Cfg, 1, 1>(a, va, s);
  return fail(TNH_ERR_UNSUPPORTED, "conv2d: kernel size %d not supported (1 or 3)", k);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace
}  // namespace tnh

extern "C" int32_t tnh_conv2d_out_dims(int64_t H, int64_t W, int64_t kh, int64_t kw, int64_t pH, int64_t pW,
                                       int64_t sY, int64_t sX, int64_t* OH, int64_t* OW) {
  TNH_ARG(OH && OW, "conv2d_out_dims: NULL output");
  TNH_ARG(kh > 0 && kw > 0 && sY > 0 && sX > 0 && pH >= 0 && pW >= 0, "conv2d_out_dims: bad geometry");
  *OH = (H + 2 * pH - kh) / sY + 1;
  *OW = (W + 2 * pW - kw) / sX + 1;
  return TNH_OK;
}

extern "C" int32_t tnh_conv2d_fwd(int64_t batch, int64_t C, int64_t H, int64_t W, int64_t F, int64_t kh,
                                  int64_t kw, int64_t pH, int64_t pW, int64_t sY, int64_t sX, const float* x,
                                  int64_t xOff, int64_t xBatchStride, const float* weights, int64_t wOff,
                                  const float* bias, int64_t biasOff, int32_t act, const float* residual,
                                  int64_t rOff, int64_t rBatchStride, float* out, int64_t outOff,
                                  int64_t outBatchStride, float* workspace, int64_t workspaceBytes) {
  using namespace tnh;
  (void)workspace;
  (void)workspaceBytes;
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(batch >= 0 && C > 0 && H > 0 && W > 0 && F > 0, "conv2d: bad sizes");
  TNH_ARG(kh == kw && (kh == 1 || kh == 3), "conv2d: only square 1x1 / 3x3 kernels are supported");
  TNH_ARG(sY > 0 && sX > 0 && pH >= 0 && pW >= 0, "conv2d: bad stride/pad");
  TNH_ARG(x && weights && out, "conv2d: NULL x/weights/out");
  TNH_ARG(act == TNH_AC_LINEAR || act == TNH_AC_LEAKY || act == TNH_AC_LOGISTIC, "conv2d: activation %d", act);
  TNH_ARG(xOff >= 0 && wOff >= 0 && outOff >= 0 && biasOff >= 0 && rOff >= 0, "conv2d: negative offset");
  const int64_t OH = (H + 2 * pH - kh) / sY + 1, OW = (W + 2 * pW - kw) / sX + 1;
  TNH_ARG(OH > 0 && OW > 0, "conv2d: empty output");
  TNH_ARG(xBatchStride >= C * H * W || batch <= 1, "conv2d: xBatchStride too small");
  TNH_ARG(outBatchStride >= F * OH * OW || batch <= 1, "conv2d: outBatchStride too small");
  TNH_ARG(!residual || rBatchStride >= F * OH * OW || batch <= 1, "conv2d: rBatchStride too small");
  if (batch == 0) return TNH_OK;
  const int64_t K = C * kh * kw, N = batch * OH * OW;
  TNH_ARG(K < (int64_t(1) << 30) && H * W < (int64_t(1) << 31) && OH * OW < (int64_t(1) << 31),
          "conv2d: tensor too large");

  ConvArgs a{};
  a.x = x + xOff;
  a.xBatchStride = xBatchStride;
  a.w = weights + wOff;
  a.bias = bias ? bias + biasOff : nullptr;
  a.res = residual ? residual + rOff : nullptr;
  a.rBatchStride = rBatchStride;
  a.out = out + outOff;
  a.outBatchStride = outBatchStride;
  a.F = F; a.N = N; a.K = K;
  a.C = (int)C; a.H = (int)H; a.W = (int)W; a.OW = (int)OW; a.OHW = (int)(OH * OW);
  a.sY = (int)sY; a.sX = (int)sX; a.pH = (int)pH; a.pW = (int)pW;
  a.act = act;

  const bool is1x1 = kh == 1 && sY == 1 && sX == 1 && pH == 0 && pW == 0;
  const bool va = aligned16(a.w) && K % 4 == 0;
  const bool vb = is1x1 && aligned16(a.x) && (OH * OW) % 4 == 0 && (batch == 1 || xBatchStride % 4 == 0);
  const int64_t tiles128 = ((F + 127) / 128) * ((N + 127) / 128);
  if (F <= 64) return launch_any<Cfg64x128>(a, (int)kh, is1x1, va, vb, cx->stream);
  if (tiles128 >= 2 * cx->cu_count) return launch_any<Cfg128>(a, (int)kh, is1x1, va, vb, cx->stream);
  return launch_any<Cfg64>(a, (int)kh, is1x1, va, vb, cx->stream);
}
