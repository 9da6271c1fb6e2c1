// TYoloLayer.forward's per-element transform (nyololayer.pas:786-830), shared
// by the yolo kernels (eltwise.hip) and the convolution epilogue that writes
// a yolo head directly (conv_args.hpp).
#pragma once
#include <hip/hip_runtime.h>

namespace tnh {

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

// Entry `entry` (channel within its anchor's 5 + classes group) of a yolo
// head: x, y, objectness and the class scores go through the logistic, the
// box width and height (entries 2 and 3) stay raw.
__device__ inline float yolo_entry(float v, int entry) { return (entry == 2 || entry == 3) ? v : logistic_poly(v); }

}  // namespace tnh
