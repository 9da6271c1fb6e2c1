// Convolution for layers too small to fill the GPU with whole-K tiles (a
// YOLOv3 layer at batch 1 has 169 to 2 704 output pixels against 256 CUs):
// the K dimension of one output tile is split over the W waves of its
// workgroup instead of over workgroups, so no partial sums leave the CU and
// no second launch reduces them.
//
// GEMM view, channels-last (as conv_nhwc_kernel): rows m = output pixels,
// columns n = filters; NCHW (as conv_lean_kernel): rows = filters, columns =
// output pixels; k = tap*C + c over tap-major weights [F][kh][kw][C].
//   * Each wave walks its own K range [w*P/W, (w+1)*P/W) of the P = K/32
//     panels of 32 k.  A panel's k-contiguous rows are fetched with
//     coalesced 16-byte loads (8 lanes per 128-byte row), NCHW pixels as 4
//     channels per lane (conv_lean.hpp's loaders), into two register sets in
//     rotation, written to the wave's private LDS panel (16-byte chunks
//     XOR-swizzled as in conv_lean.hpp) and read back in the MFMA operand
//     layout.  A wave only ever reads what it wrote itself and LDS executes
//     one wave's accesses in order, so the K loop has no barrier and the
//     waves never wait for each other.
//   * Everything that varies along K is wave-uniform (tap, channel offset)
//     and rides in the buffer instruction's scalar offset; the 3x3 padding
//     test is a per-row 9-bit tap mask computed once (a tap in the padding
//     gets offset kOOB, which reads 0).
//   * The W partial tiles then go to LDS and every element is summed in wave
//     order 0, 1, .., W-1 (fixed, so every run gives the same bits), then
//     bias + activation + residual in the reference order and one store.
#include "common.hpp"
#include "conv_lean.hpp"
#include "conv_wsplit.hpp"
#include "gemm_core.hpp"
#include "wave_panels.hpp"

namespace tnh {
namespace conv {
namespace {

__device__ inline void st1(__amdgpu_buffer_rsrc_t r, float v, uint32_t voff) {
  __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), r, voff, 0, kStoreThrough);
}

// One wave's channels-last 3x3 tap gather rows (output pixels m0 ..
// m0 + ROWS - 1): row r at k = tap*C + c reads input pixel (iy0 + ky,
// ix0 + kx) of its image, channels c0 .. c0 + 31 of the panel (C % 32 == 0,
// so a panel lies inside one tap).  rowOff is the byte offset of the row's
// pixel at tap (0, 0) plus the lane's chunk, modulo 2^32 (it may point
// before the image at the border; in-range taps add back to the exact
// offset).
template <int ROWS>
struct WaveTapRows {
  static constexpr int PER = ROWS / 8;
  using L = SwzPanel<ROWS, 32>;
  static constexpr int SIZE = L::SIZE;
  __amdgpu_buffer_rsrc_t rsrc;
  uint32_t rowOff[PER], tapMask[PER];
  uint32_t pix4, rowPix4;
  int C;
  int ldsOff[PER];
  f32x4 reg[PER];
  __device__ inline void init(const ConvArgs& a, int64_t m0, int lane) {
    const ConvGeom& g = a.g;
    rsrc = make_rsrc(g.x, g.xBytes);
    C = g.C;
    pix4 = static_cast<uint32_t>(a.xPix) * 4u;
    rowPix4 = static_cast<uint32_t>(g.W) * pix4;
#pragma unroll
    for (int v = 0; v < PER; ++v) {
      const int row = lane / 8 + 8 * v, q = lane % 8;
      const int64_t n = m0 + row;
      const bool ok = n < g.N;
      const int64_t nn = ok ? n : 0;
      const int64_t b = nn / g.OHW;
      const int p = static_cast<int>(nn - b * g.OHW);
      const int oy = p / g.OW, ox = p - (p / g.OW) * g.OW;
      const int iy0 = oy * g.sY - g.pH, ix0 = ox * g.sX - g.pW;
      rowOff[v] = static_cast<uint32_t>(((b * g.H + iy0) * g.W + ix0) * a.xPix * 4 + q * 16);
      uint32_t mk = 0;
#pragma unroll
      for (int ky = 0; ky < 3; ++ky)
#pragma unroll
        for (int kx = 0; kx < 3; ++kx) {
          const bool in = static_cast<unsigned>(iy0 + ky) < static_cast<unsigned>(g.H) &&
                          static_cast<unsigned>(ix0 + kx) < static_cast<unsigned>(g.W);
          mk |= (ok && in ? 1u : 0u) << (ky * 3 + kx);
        }
      tapMask[v] = mk;
      ldsOff[v] = L::chunk(row, q);
    }
  }
  __device__ inline void load(int k0) {
    const int tap = k0 / C;  // uniform
    const int c0 = k0 - tap * C;
    const int ky = tap / 3, kx = tap - (tap / 3) * 3;
    const uint32_t tapOff = static_cast<uint32_t>(ky) * rowPix4 + static_cast<uint32_t>(kx) * pix4;
#pragma unroll
    for (int v = 0; v < PER; ++v)
      reg[v] = buf_ld4s(rsrc, sel_off((tapMask[v] >> tap) & 1u, rowOff[v] + tapOff), static_cast<uint32_t>(c0) * 4u);
  }
  __device__ inline void store(lds_t* panel) const {
#pragma unroll
    for (int v = 0; v < PER; ++v) *reinterpret_cast<lds_f4*>(panel + ldsOff[v]) = reg[v];
  }
};

template <class Cfg, int MODE>
__global__ __launch_bounds__(Cfg::NT) void conv_wsplit_nhwc_kernel(ConvArgs a) {
  constexpr int FM = Cfg::FM, FN = Cfg::FN, W = Cfg::W, UNITS = Cfg::UNITS;
  using AL = typename std::conditional<MODE == kTap3, WaveTapRows<32 * FM>, WaveRowsK<32 * FM>>::type;
  using BL = WaveRowsK<32 * FN>;
  using Pan = LeanCfg<32 * FM, 32 * FN, 32, 1, 1, 1>;  // one wave's panel: two 16-deep chunks
  using Loop = LeanLoop<Pan, AL, BL>;
  constexpr int STAGE = AL::SIZE + BL::SIZE;
  constexpr int LDS = W * STAGE > Cfg::RED_FLOATS ? W * STAGE : Cfg::RED_FLOATS;
  __shared__ __attribute__((aligned(16))) float smem[LDS];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: K bounds stay scalar
  const int r = lane & 31, h = lane >> 5;
  int tm, tn;
  tile_coords(blockIdx.x, a.tilesM, a.tilesN, tm, tn);
  const int64_t m0 = static_cast<int64_t>(tm) * Cfg::BM, n0 = static_cast<int64_t>(tn) * Cfg::BN;
  const int64_t M = a.g.N, K = a.g.K;

  // two register sets of each operand in rotation (identical bindings)
  AL a0, a1;
  BL b0, b1;
  if constexpr (MODE == kTap3) {
    a0.init(a, m0, lane);
    a1.init(a, m0, lane);
  } else {
    a0.init(a.g.x, a.g.xBytes, a.xPix, M, m0, lane);
    a1.init(a.g.x, a.g.xBytes, a.xPix, M, m0, lane);
  }
  b0.init(a.w, a.wBytes, K, a.F, n0, lane);
  b1.init(a.w, a.wBytes, K, a.F, n0, lane);

  // MFMA operand offsets inside a panel (blocks start at multiples of 32
  // rows, so a row's swizzle is that of lane % 32)
  typename Loop::Lanes LN;
#pragma unroll
  for (int c = 0; c < 2; ++c)
#pragma unroll
    for (int e = 0; e < 2; ++e) LN.lo[c][e] = SwzPanel<32, 32>::chunk(r, 4 * c + 2 * h + e);
  LN.aRow = 0;
  LN.bRow = 0;

  f32x16 acc[FM][FN];
  Loop::zero(acc);
  lds_t* panel = (lds_t*)smem + wave * STAGE;
  const int P = static_cast<int>(K / 32);
  const int p0 = wave * P / W, np = (wave + 1) * P / W - p0;
  // K offset of the wave's panel i, clamped to its last panel: the loop
  // issues its loads unconditionally (a conditional load makes the compiler
  // wait for every load in flight), the surplus fetches are never used
  auto kOf = [&](int i) { return 32 * (p0 + min(i, np - 1)); };
  auto multiply = [&]() {
    typename Loop::Frag f0, f1;
    Loop::read(panel, 0, LN, f0);
    Loop::read(panel, 1, LN, f1);
    Loop::mma(f0, acc);
    Loop::mma(f1, acc);
  };
  // Two register sets in rotation: panel i is written to LDS and multiplied
  // while panels i+1 and i+2 are in flight.  The panel is rewritten only
  // after the reads of the previous one were issued (in-order LDS).
  if (np > 0) {
    a0.load(kOf(0));
    b0.load(kOf(0));
    a1.load(kOf(1));
    b1.load(kOf(1));
    for (int i = 0; i < np; i += 2) {
      a0.store(panel);
      b0.store(panel + AL::SIZE);
      a0.load(kOf(i + 2));
      b0.load(kOf(i + 2));
      multiply();
      if (i + 1 < np) {
        a1.store(panel);
        b1.store(panel + AL::SIZE);
      }
      a1.load(kOf(i + 3));
      b1.load(kOf(i + 3));
      if (i + 1 < np) multiply();
    }
  }
  __syncthreads();  // every wave is done with its panel: the LDS now holds the partial tiles

  // Partial tiles to LDS: quad u = (i*FN + j)*4 + q of wave w (registers
  // 4q .. 4q+3 of block (i, j)) at red[(w*UNITS + u)*64 + lane] as 16 bytes,
  // so each store and load is 64 consecutive 16-byte chunks.
  lds_f4* R = (lds_f4*)smem;
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q)
        R[(wave * UNITS + (i * FN + j) * 4 + q) * 64 + lane] =
            f32x4{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
  __syncthreads();

  const __amdgpu_buffer_rsrc_t outR = make_rsrc(a.out, a.outBytes);
  const __amdgpu_buffer_rsrc_t resR = make_rsrc(a.res, a.resBytes);
  const uint32_t op4 = static_cast<uint32_t>(a.outPix) * 4u, rp4 = static_cast<uint32_t>(a.resPix) * 4u;
  for (int u = wave; u < UNITS; u += W) {
    const int i = u / (FN * 4), j = (u / 4) % FN, q = u % 4;
    // every partial's loads first, then the sum in wave order
    f32x4 p[W];
#pragma unroll
    for (int w = 0; w < W; ++w) p[w] = R[(w * UNITS + u) * 64 + lane];
    f32x4 s = p[0];
#pragma unroll
    for (int w = 1; w < W; ++w) s = s + p[w];
    // lane owns filter f; register e of the quad is pixel m0 + 32i + 8q + 4h + e
    const int64_t f = n0 + 32 * j + r;
    const bool okF = f < a.F;
    const float bias = a.bias && okF ? a.bias[f] : -0.f;  // -0.0: the exact additive identity
    const int64_t mBase = m0 + 32 * i + 8 * q + 4 * h;
    uint32_t vo[4], vr[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const bool ok = okF && mBase + e < M;
      vo[e] = sel_off(ok, static_cast<uint32_t>(mBase + e) * op4 + static_cast<uint32_t>(f) * 4u);
      vr[e] = sel_off(ok, static_cast<uint32_t>(mBase + e) * rp4 + static_cast<uint32_t>(f) * 4u);
    }
    float rv[4] = {0.f, 0.f, 0.f, 0.f};
    if (a.res) {
#pragma unroll
      for (int e = 0; e < 4; ++e) rv[e] = buf_ld1s(resR, vr[e], 0);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float v = s[e] + bias;  // nConvolutionLayer.pas:524 (forwardBias)
      if (a.act == TNH_AC_LEAKY)
        v = v < 0.f ? 0.1f * v : v;  // leaky_array (nactivation.pas:234)
      else if (a.act == TNH_AC_LOGISTIC)
        v = 1.f / (1.f + expf(-v));
      if (a.res) v = v + rv[e];  // the fused shortcut (naddlayer.pas:698)
      if (a.upS > 0 || a.yolo) {   // epilogue variants (upsampled / yolo head)
        if (okF && mBase + e < M) store_nhwc_variant(a, outR, mBase + e, f, v);
      } else {
        st1(outR, v, vo[e]);
      }
    }
  }
}

// The 16-row tile (Ws16Cfg): as conv_wsplit_nhwc_kernel with 16x16x4
// MFMAs.  Operand layouts of v_mfma_f32_16x16x4_f32: lane l supplies
// A[i = l % 16][k = l / 16] and B[k = l / 16][j = l % 16]; accumulator
// register r of lane l is D[i = 4*(l / 16) + r][j = l % 16].  A lane reads 16
// bytes (4 consecutive k) of its row per 16-deep chunk and uses element e at
// MFMA step e: step e pairs k = 16c + 4*(l/16) + e of A and B alike, so every
// k of the chunk is summed once (in MFMA order).
template <class Cfg, int MODE>
__global__ __launch_bounds__(Cfg::NT) void conv_wsplit16_nhwc_kernel(ConvArgs a) {
  constexpr int W = Cfg::W, BLK = Cfg::BLK, UNITS = Cfg::UNITS;
  using AL = typename std::conditional<MODE == kTap3, WaveTapRows<16>, WaveRowsK<16>>::type;
  using BL = WaveRowsK<Cfg::BN>;
  constexpr int STAGE = AL::SIZE + BL::SIZE;
  constexpr int LDS = W * STAGE > Cfg::RED_FLOATS ? W * STAGE : Cfg::RED_FLOATS;
  __shared__ __attribute__((aligned(16))) float smem[LDS];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r16 = lane & 15, g = lane >> 4;
  int tm, tn;
  tile_coords(blockIdx.x, a.tilesM, a.tilesN, tm, tn);
  const int64_t m0 = static_cast<int64_t>(tm) * Cfg::BM, n0 = static_cast<int64_t>(tn) * Cfg::BN;
  const int64_t M = a.g.N, K = a.g.K;

  AL a0, a1;
  BL b0, b1;
  if constexpr (MODE == kTap3) {
    a0.init(a, m0, lane);
    a1.init(a, m0, lane);
  } else {
    a0.init(a.g.x, a.g.xBytes, a.xPix, M, m0, lane);
    a1.init(a.g.x, a.g.xBytes, a.xPix, M, m0, lane);
  }
  b0.init(a.w, a.wBytes, K, a.F, n0, lane);
  b1.init(a.w, a.wBytes, K, a.F, n0, lane);

  // LDS offsets of this lane's 16-byte operand reads, chunk c: A row r16,
  // B rows 16*jj + r16, quad 4c + g
  int aOff[2], bOff[2][BLK];
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    aOff[c] = SwzPanel<16, 32>::chunk(r16, 4 * c + g);
#pragma unroll
    for (int jj = 0; jj < BLK; ++jj) bOff[c][jj] = AL::SIZE + SwzPanel<Cfg::BN, 32>::chunk(16 * jj + r16, 4 * c + g);
  }
  f32x4 acc[BLK];
#pragma unroll
  for (int jj = 0; jj < BLK; ++jj) acc[jj] = f32x4{0.f, 0.f, 0.f, 0.f};
  lds_t* panel = (lds_t*)smem + wave * STAGE;
  const int P = static_cast<int>(K / 32);
  const int p0 = wave * P / W, np = (wave + 1) * P / W - p0;
  auto kOf = [&](int i) { return 32 * (p0 + min(i, np - 1)); };
  auto multiply = [&]() {
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const f32x4 fa = *reinterpret_cast<const lds_f4*>(panel + aOff[c]);
      f32x4 fb[BLK];
#pragma unroll
      for (int jj = 0; jj < BLK; ++jj) fb[jj] = *reinterpret_cast<const lds_f4*>(panel + bOff[c][jj]);
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int jj = 0; jj < BLK; ++jj) acc[jj] = __builtin_amdgcn_mfma_f32_16x16x4f32(fa[e], fb[jj][e], acc[jj], 0, 0, 0);
    }
  };
  if (np > 0) {
    a0.load(kOf(0));
    b0.load(kOf(0));
    a1.load(kOf(1));
    b1.load(kOf(1));
    for (int i = 0; i < np; i += 2) {
      a0.store(panel);
      b0.store(panel + AL::SIZE);
      a0.load(kOf(i + 2));
      b0.load(kOf(i + 2));
      multiply();
      if (i + 1 < np) {
        a1.store(panel);
        b1.store(panel + AL::SIZE);
      }
      a1.load(kOf(i + 3));
      b1.load(kOf(i + 3));
      if (i + 1 < np) multiply();
    }
  }
  __syncthreads();

  // partial tiles to LDS: quad jj of wave w at red[(w*UNITS + jj)*64 + lane]
  lds_f4* R = (lds_f4*)smem;
#pragma unroll
  for (int jj = 0; jj < BLK; ++jj) R[(wave * UNITS + jj) * 64 + lane] = acc[jj];
  __syncthreads();

  const __amdgpu_buffer_rsrc_t outR = make_rsrc(a.out, a.outBytes);
  const __amdgpu_buffer_rsrc_t resR = make_rsrc(a.res, a.resBytes);
  const uint32_t op4 = static_cast<uint32_t>(a.outPix) * 4u, rp4 = static_cast<uint32_t>(a.resPix) * 4u;
  for (int u = wave; u < UNITS; u += W) {
    f32x4 p[W];
#pragma unroll
    for (int w = 0; w < W; ++w) p[w] = R[(w * UNITS + u) * 64 + lane];
    f32x4 s = p[0];
#pragma unroll
    for (int w = 1; w < W; ++w) s = s + p[w];
    // lane owns filter f = n0 + 16u + r16; register e is pixel m0 + 4g + e
    const int64_t f = n0 + 16 * u + r16;
    const bool okF = f < a.F;
    const float bias = a.bias && okF ? a.bias[f] : -0.f;
    const int64_t mBase = m0 + 4 * g;
    uint32_t vo[4], vr[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const bool ok = okF && mBase + e < M;
      vo[e] = sel_off(ok, static_cast<uint32_t>(mBase + e) * op4 + static_cast<uint32_t>(f) * 4u);
      vr[e] = sel_off(ok, static_cast<uint32_t>(mBase + e) * rp4 + static_cast<uint32_t>(f) * 4u);
    }
    float rv[4] = {0.f, 0.f, 0.f, 0.f};
    if (a.res) {
#pragma unroll
      for (int e = 0; e < 4; ++e) rv[e] = buf_ld1s(resR, vr[e], 0);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float v = s[e] + bias;  // nConvolutionLayer.pas:524 (forwardBias)
      if (a.act == TNH_AC_LEAKY)
        v = v < 0.f ? 0.1f * v : v;  // leaky_array (nactivation.pas:234)
      else if (a.act == TNH_AC_LOGISTIC)
        v = 1.f / (1.f + expf(-v));
      if (a.res) v = v + rv[e];  // the fused shortcut (naddlayer.pas:698)
      if (a.upS > 0 || a.yolo) {
        if (okF && mBase + e < M) store_nhwc_variant(a, outR, mBase + e, f, v);
      } else {
        st1(outR, v, vo[e]);
      }
    }
  }
}

// ---- NCHW (tnh_conv2d_fwd) forms of the two kernels above.  They repeat
// the K loop instead of sharing a templated body with the channels-last
// kernels: a shared body compiled the channels-last epilogue to a schedule
// that waited on the bias load before computing its store offsets, 5-7%
// slower for the 16-row tiles.

// One wave as the workgroup of conv_lean.hpp's NCHW pixel loaders (LeanTapB,
// Lean1x1B): a COLS-pixel x 32-k panel, the same swizzled [COLS][32] layout
// as a WaveRowsK panel.
template <int COLS>
struct WavePan {
  static constexpr int BK = 32, BN = COLS, NT = 64;
};

// Operands of an NCHW wave-split tile: rows = filters (the tap-major
// weights [F][K], k-contiguous), columns = output pixels, gathered as 4
// channels of one pixel per lane (loads HW floats apart, coalesced over the
// pixels of a lane group) and one 16-byte LDS write; VB: the 1x1 input read
// as 4x4 blocks (16-byte loads along pixels, HW % 4 == 0), which needs a
// panel of 32 or more pixels.
template <int ROWS, int COLS, int MODE, bool VB>
struct NchwOps {
  static constexpr bool kVec = VB && COLS >= 32;
  using AL = WaveRowsK<ROWS>;
  using BL = typename std::conditional<MODE == kTap3, LeanTapB<WavePan<COLS>, 3, 3>,
                                       Lean1x1B<WavePan<COLS>, kVec>>::type;
  static __device__ inline void initA(const ConvArgs& a, int64_t m0, int lane, AL& al) {
    al.init(a.w, a.wBytes, a.g.K, a.F, m0, lane);
  }
  static __device__ inline void initB(const ConvArgs& a, int64_t n0, int lane, BL& bl) { bl.init(a.g, n0, lane); }
};

// NCHW epilogue of a wave-split tile: the finished sums s[e] of filters
// f0 + e (e = 0..3) at output pixel n: bias, activation and residual in the
// reference order, then one store each to out[b * outBatchStride + f * OHW +
// p] (residual likewise with rBatchStride).  Out-of-range elements get kOOB
// (their loads read 0, their stores drop).
__device__ inline void ws_finish_nchw(const ConvArgs& a, __amdgpu_buffer_rsrc_t outR, __amdgpu_buffer_rsrc_t resR,
                                      f32x4 s, int64_t f0, int64_t n) {
  const bool okN = n < a.g.N;
  const uint32_t OHW = static_cast<uint32_t>(a.g.OHW);
  const uint32_t nn = okN ? static_cast<uint32_t>(n) : 0u;
  const uint32_t b = nn / OHW, p = nn - b * OHW;
  const uint32_t ob = b * static_cast<uint32_t>(a.outBatchStride) + p;
  const uint32_t rb = b * static_cast<uint32_t>(a.rBatchStride) + p;
  uint32_t vo[4], vr[4];
  float bias[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int64_t f = f0 + e;
    const bool ok = okN && f < a.F;
    vo[e] = sel_off(ok, (ob + static_cast<uint32_t>(f) * OHW) * 4u);
    vr[e] = sel_off(ok, (rb + static_cast<uint32_t>(f) * OHW) * 4u);
    bias[e] = a.bias && f < a.F ? a.bias[f] : -0.f;  // -0.0: the exact additive identity
  }
  float rv[4] = {0.f, 0.f, 0.f, 0.f};
  if (a.res) {
#pragma unroll
    for (int e = 0; e < 4; ++e) rv[e] = buf_ld1s(resR, vr[e], 0);
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    float v = s[e] + bias[e];  // nConvolutionLayer.pas:524 (forwardBias)
    if (a.act == TNH_AC_LEAKY)
      v = v < 0.f ? 0.1f * v : v;  // leaky_array (nactivation.pas:234)
    else if (a.act == TNH_AC_LOGISTIC)
      v = 1.f / (1.f + expf(-v));
    if (a.res) v = v + rv[e];  // the fused shortcut (naddlayer.pas:698)
    st1(outR, v, vo[e]);
  }
}

// NCHW form of conv_wsplit_nhwc_kernel: the (32*FM) filters x (32*FN)
// pixels tile on v_mfma_f32_32x32x2_f32.
template <class Cfg, int MODE, bool VB>
__global__ __launch_bounds__(Cfg::NT) void conv_wsplit_nchw_kernel(ConvArgs a) {
  constexpr int FM = Cfg::FM, FN = Cfg::FN, W = Cfg::W, UNITS = Cfg::UNITS;
  using Ops = NchwOps<32 * FM, 32 * FN, MODE, VB>;
  using AL = typename Ops::AL;
  using BL = typename Ops::BL;
  using Pan = LeanCfg<32 * FM, 32 * FN, 32, 1, 1, 1>;  // one wave's panel: two 16-deep chunks
  using Loop = LeanLoop<Pan, AL, BL>;
  constexpr int STAGE = AL::SIZE + BL::SIZE;
  constexpr int LDS = W * STAGE > Cfg::RED_FLOATS ? W * STAGE : Cfg::RED_FLOATS;
  __shared__ __attribute__((aligned(16))) float smem[LDS];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: K bounds stay scalar
  const int r = lane & 31, h = lane >> 5;
  int tm, tn;
  tile_coords(blockIdx.x, a.tilesM, a.tilesN, tm, tn);
  const int64_t m0 = static_cast<int64_t>(tm) * Cfg::BM, n0 = static_cast<int64_t>(tn) * Cfg::BN;
  const int64_t K = a.g.K;

  // two register sets of each operand in rotation (identical bindings)
  AL a0, a1;
  BL b0, b1;
  Ops::initA(a, m0, lane, a0);
  Ops::initA(a, m0, lane, a1);
  Ops::initB(a, n0, lane, b0);
  Ops::initB(a, n0, lane, b1);

  // MFMA operand offsets inside a panel (blocks start at multiples of 32
  // rows, so a row's swizzle is that of lane % 32)
  typename Loop::Lanes LN;
#pragma unroll
  for (int c = 0; c < 2; ++c)
#pragma unroll
    for (int e = 0; e < 2; ++e) LN.lo[c][e] = SwzPanel<32, 32>::chunk(r, 4 * c + 2 * h + e);
  LN.aRow = 0;
  LN.bRow = 0;

  f32x16 acc[FM][FN];
  Loop::zero(acc);
  lds_t* panel = (lds_t*)smem + wave * STAGE;
  const int P = static_cast<int>(K / 32);
  const int p0 = wave * P / W, np = (wave + 1) * P / W - p0;
  // K offset of the wave's panel i, clamped to its last panel: the loop
  // issues its loads unconditionally (a conditional load makes the compiler
  // wait for every load in flight), the surplus fetches are never used
  auto kOf = [&](int i) { return 32 * (p0 + min(i, np - 1)); };
  auto multiply = [&]() {
    typename Loop::Frag f0, f1;
    Loop::read(panel, 0, LN, f0);
    Loop::read(panel, 1, LN, f1);
    Loop::mma(f0, acc);
    Loop::mma(f1, acc);
  };
  // Two register sets in rotation: panel i is written to LDS and multiplied
  // while panels i+1 and i+2 are in flight.  The panel is rewritten only
  // after the reads of the previous one were issued (in-order LDS).
  if (np > 0) {
    a0.load(kOf(0));
    b0.load(kOf(0));
    a1.load(kOf(1));
    b1.load(kOf(1));
    for (int i = 0; i < np; i += 2) {
      a0.store(panel);
      b0.store(panel + AL::SIZE);
      a0.load(kOf(i + 2));
      b0.load(kOf(i + 2));
      multiply();
      if (i + 1 < np) {
        a1.store(panel);
        b1.store(panel + AL::SIZE);
      }
      a1.load(kOf(i + 3));
      b1.load(kOf(i + 3));
      if (i + 1 < np) multiply();
    }
  }
  __syncthreads();  // every wave is done with its panel: the LDS now holds the partial tiles

  // Partial tiles to LDS: quad u = (i*FN + j)*4 + q of wave w (registers
  // 4q .. 4q+3 of block (i, j)) at red[(w*UNITS + u)*64 + lane] as 16 bytes,
  // so each store and load is 64 consecutive 16-byte chunks.
  lds_f4* R = (lds_f4*)smem;
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q)
        R[(wave * UNITS + (i * FN + j) * 4 + q) * 64 + lane] =
            f32x4{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
  __syncthreads();

  const __amdgpu_buffer_rsrc_t outR = make_rsrc(a.out, a.outBytes);
  const __amdgpu_buffer_rsrc_t resR = make_rsrc(a.res, a.resBytes);
  for (int u = wave; u < UNITS; u += W) {
    const int i = u / (FN * 4), j = (u / 4) % FN, q = u % 4;
    // every partial's loads first, then the sum in wave order
    f32x4 p[W];
#pragma unroll
    for (int w = 0; w < W; ++w) p[w] = R[(w * UNITS + u) * 64 + lane];
    f32x4 s = p[0];
#pragma unroll
    for (int w = 1; w < W; ++w) s = s + p[w];
    // lane owns column n0 + 32j + r; register e of the quad is row
    // m0 + 32i + 8q + 4h + e
    ws_finish_nchw(a, outR, resR, s, m0 + 32 * i + 8 * q + 4 * h, n0 + 32 * j + r);
  }
}

// NCHW form of conv_wsplit16_nhwc_kernel: 16 filters x (16*BLK) pixels on
// v_mfma_f32_16x16x4_f32.
template <class Cfg, int MODE, bool VB>
__global__ __launch_bounds__(Cfg::NT) void conv_wsplit16_nchw_kernel(ConvArgs a) {
  constexpr int W = Cfg::W, BLK = Cfg::BLK, UNITS = Cfg::UNITS;
  using Ops = NchwOps<16, Cfg::BN, MODE, VB>;
  using AL = typename Ops::AL;
  using BL = typename Ops::BL;
  constexpr int STAGE = AL::SIZE + BL::SIZE;
  constexpr int LDS = W * STAGE > Cfg::RED_FLOATS ? W * STAGE : Cfg::RED_FLOATS;
  __shared__ __attribute__((aligned(16))) float smem[LDS];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r16 = lane & 15, g = lane >> 4;
  int tm, tn;
  tile_coords(blockIdx.x, a.tilesM, a.tilesN, tm, tn);
  const int64_t m0 = static_cast<int64_t>(tm) * Cfg::BM, n0 = static_cast<int64_t>(tn) * Cfg::BN;
  const int64_t K = a.g.K;

  AL a0, a1;
  BL b0, b1;
  Ops::initA(a, m0, lane, a0);
  Ops::initA(a, m0, lane, a1);
  Ops::initB(a, n0, lane, b0);
  Ops::initB(a, n0, lane, b1);

  // LDS offsets of this lane's 16-byte operand reads, chunk c: A row r16,
  // B rows 16*jj + r16, quad 4c + g
  int aOff[2], bOff[2][BLK];
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    aOff[c] = SwzPanel<16, 32>::chunk(r16, 4 * c + g);
#pragma unroll
    for (int jj = 0; jj < BLK; ++jj) bOff[c][jj] = AL::SIZE + SwzPanel<Cfg::BN, 32>::chunk(16 * jj + r16, 4 * c + g);
  }
  f32x4 acc[BLK];
#pragma unroll
  for (int jj = 0; jj < BLK; ++jj) acc[jj] = f32x4{0.f, 0.f, 0.f, 0.f};
  lds_t* panel = (lds_t*)smem + wave * STAGE;
  const int P = static_cast<int>(K / 32);
  const int p0 = wave * P / W, np = (wave + 1) * P / W - p0;
  auto kOf = [&](int i) { return 32 * (p0 + min(i, np - 1)); };
  auto multiply = [&]() {
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const f32x4 fa = *reinterpret_cast<const lds_f4*>(panel + aOff[c]);
      f32x4 fb[BLK];
#pragma unroll
      for (int jj = 0; jj < BLK; ++jj) fb[jj] = *reinterpret_cast<const lds_f4*>(panel + bOff[c][jj]);
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int jj = 0; jj < BLK; ++jj) acc[jj] = __builtin_amdgcn_mfma_f32_16x16x4f32(fa[e], fb[jj][e], acc[jj], 0, 0, 0);
    }
  };
  if (np > 0) {
    a0.load(kOf(0));
    b0.load(kOf(0));
    a1.load(kOf(1));
    b1.load(kOf(1));
    for (int i = 0; i < np; i += 2) {
      a0.store(panel);
      b0.store(panel + AL::SIZE);
      a0.load(kOf(i + 2));
      b0.load(kOf(i + 2));
      multiply();
      if (i + 1 < np) {
        a1.store(panel);
        b1.store(panel + AL::SIZE);
      }
      a1.load(kOf(i + 3));
      b1.load(kOf(i + 3));
      if (i + 1 < np) multiply();
    }
  }
  __syncthreads();

  // partial tiles to LDS: quad jj of wave w at red[(w*UNITS + jj)*64 + lane]
  lds_f4* R = (lds_f4*)smem;
#pragma unroll
  for (int jj = 0; jj < BLK; ++jj) R[(wave * UNITS + jj) * 64 + lane] = acc[jj];
  __syncthreads();

  const __amdgpu_buffer_rsrc_t outR = make_rsrc(a.out, a.outBytes);
  const __amdgpu_buffer_rsrc_t resR = make_rsrc(a.res, a.resBytes);
  for (int u = wave; u < UNITS; u += W) {
    f32x4 p[W];
#pragma unroll
    for (int w = 0; w < W; ++w) p[w] = R[(w * UNITS + u) * 64 + lane];
    f32x4 s = p[0];
#pragma unroll
    for (int w = 1; w < W; ++w) s = s + p[w];
    // lane owns column n0 + 16u + r16; register e is row m0 + 4g + e
    ws_finish_nchw(a, outR, resR, s, m0 + 4 * g, n0 + 16 * u + r16);
  }
}

// Grid of one wave-split launch: (rows / BM) x (columns / BN) tiles, whole K
// (rows: pixels channels-last, filters NCHW).
template <class Cfg>
int ws_grid(ConvArgs& a, bool nchw, dim3& grid) {
  const int64_t rows = nchw ? a.F : a.g.N, cols = nchw ? a.g.N : a.F;
  const int64_t tm = (rows + Cfg::BM - 1) / Cfg::BM, tn = (cols + Cfg::BN - 1) / Cfg::BN;
  if (tm * tn > INT32_MAX) return fail(TNH_ERR_UNSUPPORTED, "conv2d: grid too large");
  a.tilesM = static_cast<int>(tm);
  a.tilesN = static_cast<int>(tn);
  a.splits = 1;
  a.tailSplits = 0;
  a.kChunk = a.g.K;
  grid = dim3(static_cast<unsigned>(tm * tn));
  return TNH_OK;
}

template <class Cfg>
int launch_cfg16(ConvArgs a, int mode, hipStream_t s) {
  dim3 grid;
  if (int st = ws_grid<Cfg>(a, false, grid)) return st;
  if (mode == kTap3)
    hipLaunchKernelGGL((conv_wsplit16_nhwc_kernel<Cfg, kTap3>), grid, dim3(Cfg::NT), 0, s, a);
  else
    hipLaunchKernelGGL((conv_wsplit16_nhwc_kernel<Cfg, k1x1>), grid, dim3(Cfg::NT), 0, s, a);
  return launch_status("conv_wsplit16_nhwc_kernel");
}

template <class Cfg>
int launch_cfg(ConvArgs a, int mode, hipStream_t s) {
  dim3 grid;
  if (int st = ws_grid<Cfg>(a, false, grid)) return st;
  if (mode == kTap3)
    hipLaunchKernelGGL((conv_wsplit_nhwc_kernel<Cfg, kTap3>), grid, dim3(Cfg::NT), 0, s, a);
  else
    hipLaunchKernelGGL((conv_wsplit_nhwc_kernel<Cfg, k1x1>), grid, dim3(Cfg::NT), 0, s, a);
  return launch_status("conv_wsplit_nhwc_kernel");
}

template <class Cfg>
int launch_cfg16_nchw(ConvArgs a, int mode, bool vb, hipStream_t s) {
  dim3 grid;
  if (int st = ws_grid<Cfg>(a, true, grid)) return st;
  constexpr bool kVec = Cfg::BN >= 32;  // the 4x4-block 1x1 loader needs 32 or more pixels per panel
  const bool vec = kVec && vb;
  if (mode == kTap3)
    hipLaunchKernelGGL((conv_wsplit16_nchw_kernel<Cfg, kTap3, false>), grid, dim3(Cfg::NT), 0, s, a);
  else if (vec)
    hipLaunchKernelGGL((conv_wsplit16_nchw_kernel<Cfg, k1x1, kVec>), grid, dim3(Cfg::NT), 0, s, a);
  else
    hipLaunchKernelGGL((conv_wsplit16_nchw_kernel<Cfg, k1x1, false>), grid, dim3(Cfg::NT), 0, s, a);
  return launch_status("conv_wsplit16_nchw_kernel");
}

template <class Cfg>
int launch_cfg_nchw(ConvArgs a, int mode, bool vb, hipStream_t s) {
  dim3 grid;
  if (int st = ws_grid<Cfg>(a, true, grid)) return st;
  if (mode == kTap3)
    hipLaunchKernelGGL((conv_wsplit_nchw_kernel<Cfg, kTap3, false>), grid, dim3(Cfg::NT), 0, s, a);
  else if (vb)
    hipLaunchKernelGGL((conv_wsplit_nchw_kernel<Cfg, k1x1, true>), grid, dim3(Cfg::NT), 0, s, a);
  else
    hipLaunchKernelGGL((conv_wsplit_nchw_kernel<Cfg, k1x1, false>), grid, dim3(Cfg::NT), 0, s, a);
  return launch_status("conv_wsplit_nchw_kernel");
}

}  // namespace

int launch_wsplit_nhwc(int ws, ConvArgs a, int mode, hipStream_t s) {
  if (a.g.K % 32 != 0 || a.g.C % 32 != 0 || (mode != kTap3 && mode != k1x1))
    return fail(TNH_ERR_UNSUPPORTED, "conv2d: the wave-split kernel needs C %% 32 == 0 and a 3x3 or 1x1 kernel");
  switch (ws) {
    case 0: return launch_cfg<WsCfg<1, 1, 4>>(a, mode, s);
    case 1: return launch_cfg<WsCfg<1, 1, 8>>(a, mode, s);
    case 2: return launch_cfg<WsCfg<1, 2, 4>>(a, mode, s);
    case 3: return launch_cfg16<Ws16Cfg<2, 4>>(a, mode, s);
    case 4: return launch_cfg16<Ws16Cfg<2, 8>>(a, mode, s);
    case 5: return launch_cfg16<Ws16Cfg<1, 4>>(a, mode, s);
    case 6: return launch_cfg16<Ws16Cfg<1, 8>>(a, mode, s);
    default: return fail(TNH_ERR_UNSUPPORTED, "conv2d: wave-split tile %d", ws);
  }
}

int launch_wsplit_nchw(int ws, ConvArgs a, int mode, bool vb, hipStream_t s) {
  if (a.g.K % 32 != 0 || a.g.C % 32 != 0 || (mode != kTap3 && mode != k1x1))
    return fail(TNH_ERR_UNSUPPORTED, "conv2d: the wave-split kernel needs C %% 32 == 0 and a 3x3 or 1x1 kernel");
  switch (ws) {
    case 0: return launch_cfg_nchw<WsCfg<1, 1, 4>>(a, mode, vb, s);
    case 1: return launch_cfg_nchw<WsCfg<1, 1, 8>>(a, mode, vb, s);
    case 2: return launch_cfg_nchw<WsCfg<1, 2, 4>>(a, mode, vb, s);
    case 3: return launch_cfg16_nchw<Ws16Cfg<2, 4>>(a, mode, vb, s);
    case 4: return launch_cfg16_nchw<Ws16Cfg<2, 8>>(a, mode, vb, s);
    case 5: return launch_cfg16_nchw<Ws16Cfg<1, 4>>(a, mode, vb, s);
    case 6: return launch_cfg16_nchw<Ws16Cfg<1, 8>>(a, mode, vb, s);
    default: return fail(TNH_ERR_UNSUPPORTED, "conv2d: wave-split tile %d", ws);
  }
}

}  // namespace conv
}  // namespace tnh
