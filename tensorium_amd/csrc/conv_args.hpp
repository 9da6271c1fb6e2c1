// Arguments and the shared epilogue of the fused convolution kernels
// (conv.hip, conv_lean.hpp).
//
// Epilogue per element, in the reference order (nConvolutionLayer.pas:508-545
// then the shortcut add of naddlayer.pas:698):
//   v = acc + bias[f];  v = act(v);  v = v + residual.
#pragma once
#include "common.hpp"
#include "gemm_core.hpp"

namespace tnh {
namespace conv {

struct ConvArgs {
  ConvGeom g;
  const float* w;
  int64_t wBytes;
  const float* bias;
  const float* res;
  int64_t rBatchStride;
  float* out;
  int64_t outBatchStride;
  int64_t F;
  int act;
  int tilesM, tilesN;
  int splits;       // split-K factor (gridDim.y)
  int64_t kChunk;   // K range per split (multiple of BK)
  float* part;      // splits > 1: partial sums [splits][F][N]
};

// K walk / B operand of a convolution kernel
enum Mode { kGatherRef3 = 0, kGatherTap3 = 1, kGatherRef1 = 2, kTap3 = 3, k1x1 = 4 };

__device__ inline float apply_act(float v, int act) {
  if (act == TNH_AC_LEAKY) return v < 0.f ? 0.1f * v : v;  // leaky_array (nactivation.pas:234)
  if (act == TNH_AC_LOGISTIC) return 1.f / (1.f + expf(-v));
  return v;
}

// Writes one wave's FM x FN accumulator blocks whose top-left output element
// is (row m0w, column n0w): raw partial sums into the split's slice of
// a.part when a.splits > 1 (conv_splitk_reduce applies the epilogue), else
// the epilogue in the reference order.  Each lane owns FN output columns;
// their image / pixel split is computed once.
template <int FM, int FN>
__device__ inline void conv_store(const ConvArgs& a, const f32x16 (&acc)[FM][FN], int64_t m0w, int64_t n0w,
                                  int lane) {
  const int h = lane >> 5;
  if (a.splits > 1) {
    float* part = a.part + static_cast<int64_t>(blockIdx.y) * a.F * a.g.N;
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int64_t n = n0w + j * 32 + (lane & 31);
      if (n >= a.g.N) continue;
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int64_t f = m0w + i * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
          if (f < a.F) part[f * a.g.N + n] = acc[i][j][r];
        }
    }
    return;
  }
  const int64_t OHW = a.g.OHW;
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    const int64_t n = n0w + j * 32 + (lane & 31);
    if (n >= a.g.N) continue;
    const int64_t b = n / OHW, p = n - b * OHW;
    float* out = a.out + b * a.outBatchStride + p;
    const float* res = a.res ? a.res + b * a.rBatchStride + p : nullptr;
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t f = m0w + i * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
        if (f >= a.F) continue;
        float v = acc[i][j][r];
        if (a.bias) v = v + a.bias[f];
        v = apply_act(v, a.act);
        if (res) v = v + res[f * OHW];
        out[f * OHW] = v;
      }
  }
}

}  // namespace conv
}  // namespace tnh
