// Convolution with K split over the waves of a workgroup (conv_wsplit.hip):
// the tile shapes and the launch entries the tuner in conv.hip calls.
#pragma once
#include "conv_args.hpp"

namespace tnh {
namespace conv {

// One workgroup computes a (32*FM) x (32*FN) tile (channels-last: pixels x
// filters; NCHW: filters x pixels) with W
// waves; wave w accumulates panels [w*P/W, (w+1)*P/W) of the P = K/32
// panels of 32 k through its own LDS panel, then the W partial tiles are
// summed through LDS in wave order.
template <int FM_, int FN_, int W_>
struct WsCfg {
  static constexpr int FM = FM_, FN = FN_, W = W_;
  static constexpr int NT = W * 64;
  static constexpr int BM = 32 * FM, BN = 32 * FN, BK = 32;
  static constexpr int UNITS = FM * FN * 4;  // 16-byte register quads of one wave's partial tile
  static constexpr int RED_FLOATS = W * UNITS * 64 * 4;
  static constexpr int PANEL_FLOATS = W * (BM + BN) * 32;  // one panel per wave
  static_assert(W == 2 || W == 4 || W == 8 || W == 16, "waves per workgroup");
  static_assert(RED_FLOATS <= 16384 && PANEL_FLOATS <= 16384, "LDS above 64 KiB");
};

// A 16-pixel x (16*BLK)-filter tile on v_mfma_f32_16x16x4_f32 (same MFMA
// rate as the 32x32x2 form, smaller tiles): a layer of 352 tiles of 32 x 32
// (YOLOv3's 26x26 layers at batch 1) puts two tiles on 96 of 256 CUs; as 688
// tiles of 16 x 32 the busiest CU does three halves, a quarter less.  A
// 13x13 layer (192 tiles of 32 x 32 for 256 CUs) needs 16 x 16 tiles for
// the same.
template <int BLK_, int W_>
struct Ws16Cfg {
  static constexpr int BLK = BLK_, W = W_;  // BLK: 16x16 accumulator blocks per wave
  static constexpr int NT = W * 64;
  static constexpr int BM = 16, BN = 16 * BLK, BK = 32;
  static constexpr int UNITS = BLK;  // 16-byte register quads of one wave's partial tile
  static constexpr int RED_FLOATS = W * UNITS * 64 * 4;
  static constexpr int PANEL_FLOATS = W * (BM + BN) * 32;
  static_assert(W == 2 || W == 4 || W == 8 || W == 16, "waves per workgroup");
  static_assert(RED_FLOATS <= 16384 && PANEL_FLOATS <= 16384, "LDS above 64 KiB");
};

// Tile shapes (index into kWsCfgs; the tuner's configurations kWsFirst + i),
// the ones that won a YOLOv3 layer shape in timed sweeps of (FM, FN, W) in
// {1, 2} x {1, 2} x {2, 4, 8}: 32x32 with 4 or 8 waves, 32x64 with 4; then
// the Ws16Cfg tiles 16x32 and 16x16 with 4 or 8 waves.
struct WsInfo {
  int rows, cols, W;
};
constexpr int kNumWs = 7;
constexpr WsInfo kWsCfgs[kNumWs] = {{32, 32, 4}, {32, 32, 8}, {32, 64, 4}, {16, 32, 4},
                                    {16, 32, 8}, {16, 16, 4}, {16, 16, 8}};

// Launches tile shape `ws` (0 .. kNumWs-1) for a channels-last convolution
// whose ConvArgs are filled as for conv_nhwc_kernel (mode kTap3 or k1x1;
// C % 32 == 0; out and residual within 2 GiB).
int launch_wsplit_nhwc(int ws, ConvArgs a, int mode, hipStream_t s);

// The same tiles for an NCHW convolution whose ConvArgs are filled as for
// conv_lean_kernel (mode kTap3 with tap-major weights, or k1x1; C % 32 == 0;
// out and residual within 2 GiB); vb: the 1x1 input may be read as 16-byte
// pixel vectors (16-byte aligned, HW and the batch stride multiples of 4).
int launch_wsplit_nchw(int ws, ConvArgs a, int mode, bool vb, hipStream_t s);

}  // namespace conv
}  // namespace tnh
