// Lean implicit-GEMM convolution on fp32 MFMA (gfx950).
//
// The fastest conv kernel family of the library.  What makes it lean:
//   * Both operand panels are k-contiguous in LDS with their 16-byte chunks
//     XOR-swizzled by row % 8: every LDS access is a conflict-free 16-byte
//     ds_read/ds_write_b128 and no padding is needed.  The B gather writes 4
//     consecutive k of one output column per 16-byte store.
//   * Per-lane global offsets are fixed for the whole K loop; what varies
//     along K is wave-uniform and rides in the buffer instruction's scalar
//     offset.  The 3x3 padding test is a per-lane 9-bit tap mask computed
//     once, so a K panel costs a few vector ALU operations instead of two per
//     load.
//   * Schedule of panel p (two LDS stages; the loaders' registers hold panel
//     p+1; the fragments of chunk 0 of panel p are in registers):
//       chunks 0 .. KCH-2: read the fragments of chunk c+1, then the MFMAs of
//         chunk c; during chunk 0 the registers of panel p+1 go to the other
//         stage and the global loads of panel p+2 are issued;
//       barrier (every wave stored panel p+1 and read all of panel p);
//       read the fragments of chunk 0 of panel p+1, then the MFMAs of chunk
//       KCH-1 of panel p.
//     The other stage held panel p-1, whose last reads precede the previous
//     barrier, so overwriting it during panel p is safe; panel p+1 is read
//     only after this panel's barrier.  A wave reaches the barrier with the
//     last chunk's MFMAs still to issue, and the first fragment reads of the
//     next panel hide behind them.  The panel loop is unrolled over the two
//     stages (LDS addresses are per-lane constants plus immediates) and the
//     last panels are peeled, so the steady-state body is one basic block.
//
// Requirements (checked by the host): K % BK == 0 (tap-major 3x3 with
// C % BK == 0, or 1x1 stride 1 with C % BK == 0), 16-byte weight rows, and
// output / residual / split-K partials within 2 GiB each (conv_store_buf).
#pragma once
#include "conv_args.hpp"

namespace tnh {
namespace conv {

template <int BM_, int BN_, int BK_, int WM_, int WN_, int OCC_>
struct LeanCfg {
  static constexpr int BM = BM_, BN = BN_, BK = BK_, WM = WM_, WN = WN_, OCC = OCC_;
  static constexpr int NT = WM * WN * 64;
  static constexpr int WTM = BM / WM, WTN = BN / WN;
  static constexpr int FM = WTM / 32, FN = WTN / 32;
  static constexpr int KCH = BK / 16;
  static_assert(FM >= 1 && FN >= 1 && WTM % 32 == 0 && WTN % 32 == 0, "tile");
  static_assert(BK % 32 == 0 && KCH % 2 == 0, "BK: 32 or 64");
};

// k-contiguous panel [ROWS][BK] (floats) whose 16-byte chunks are
// XOR-swizzled: logical chunk q of row r sits at physical chunk q ^ swz(r).
// The LDS has 64 four-byte banks (256 bytes) and serves a 16-byte access 16
// lanes at a time, so 16 consecutive rows at one logical chunk must land in
// 16 different 16-byte bank groups.  A 32-float row is half a bank line: the
// row parity picks the half and swz(r) = (r / 2) % 8 spreads each half's 8
// rows over its 8 groups.  A 64-float row spans all 64 banks: swz(r) =
// r % 16.  One row's chunks, and two consecutive rows' chunks, are always
// distinct groups too (the row-wise stores of the loaders).
template <int ROWS, int BK>
struct SwzPanel {
  static constexpr int SIZE = ROWS * BK;
  static_assert(BK == 32 || BK == 64, "panel depth");
  __device__ static inline int swz(int row) { return BK == 32 ? (row >> 1) & 7 : row & 15; }
  __device__ static inline int chunk(int row, int q) { return row * BK + 4 * (q ^ swz(row)); }
};

// k-contiguous operand: row r of the panel is memory row r0 + r (row stride
// ld floats, rows >= `rows` read 0), 16-byte loads.  Thread t owns chunk
// t % (BK/4) of rows t / (BK/4) + v * ROWSTEP (ROWSTEP % 16 == 0, so every row
// of a thread has the same swizzle).  The conv weights [F][K] (ld = K), and
// the GEMM operands A (not transposed) and B (transposed).  KT: K is not a
// multiple of BK (set by klimit()); a chunk at k >= K reads 0 instead of the
// start of the next row.
template <int ROWS, int BK_, int NT_, bool KT = false>
struct LeanRowsK {
  static constexpr int BK = BK_, NT = NT_;
  static constexpr int QPR = BK / 4;
  static constexpr int ROWSTEP = NT / QPR;
  static constexpr int PER = ROWS / ROWSTEP;
  using L = SwzPanel<ROWS, BK>;
  static constexpr int SIZE = L::SIZE;
  static_assert(NT % QPR == 0 && ROWS % ROWSTEP == 0 && PER >= 1 && ROWSTEP % 16 == 0, "LeanRowsK split");
  __amdgpu_buffer_rsrc_t rsrc;
  uint32_t voff[PER];
  int ldsOff;
  int kq4, kLim;  // KT: this thread's k offset in a panel, and K
  f32x4 reg[PER];

  __device__ inline void init(const float* p, int64_t bytes, int64_t ld, int64_t rows, int64_t r0, int tid) {
    rsrc = make_rsrc(p, bytes);
    const int row = tid / QPR, kq = tid % QPR;
#pragma unroll
    for (int v = 0; v < PER; ++v) {
      const int64_t gr = r0 + row + v * ROWSTEP;
      voff[v] = sel_off(gr < rows, static_cast<uint32_t>((gr * ld + kq * 4) * 4));
    }
    ldsOff = L::chunk(row, kq);
    kq4 = 4 * kq;
    kLim = 0;
  }
  __device__ inline void klimit(int64_t K) { kLim = static_cast<int>(K); }
  __device__ inline void load(int64_t k0) {
    const uint32_t so = static_cast<uint32_t>(k0) * 4u;
    if constexpr (KT) {
      const bool in = static_cast<int>(k0) + kq4 < kLim;  // K % 4 == 0: a chunk is whole or past K
#pragma unroll
      for (int v = 0; v < PER; ++v) reg[v] = buf_ld4s(rsrc, sel_off(in, voff[v]), so);
    } else {
#pragma unroll
      for (int v = 0; v < PER; ++v) reg[v] = buf_ld4s(rsrc, voff[v], so);
    }
  }
  __device__ inline void store(lds_t* stage) const {
#pragma unroll
    for (int v = 0; v < PER; ++v) *reinterpret_cast<lds_f4*>(stage + ldsOff + v * ROWSTEP * BK) = reg[v];
  }
};

template <class Cfg>
using LeanA = LeanRowsK<Cfg::BM, Cfg::BK, Cfg::NT>;

// Row-contiguous operand: element (row r, k) at (r0 + r) + k * ld floats
// (rows >= `rows` read 0): the GEMM operands A (transposed) and B (not
// transposed).  VEC (ld % 4 == 0, rows % 4 == 0, 16-byte aligned base):
// thread t owns rows 4 * (t % (ROWS/4)) .. +3 and k-quads t / (ROWS/4) + j *
// QSTEP; it loads a 4 (k) x 4 (row) block with four 16-byte loads and stores
// its transpose, one 16-byte LDS write per row.  Scalar: one row per thread,
// 4 loads ld floats apart per k-quad.
template <int ROWS, int BK_, int NT_, bool VEC>
struct LeanRowsMN {
  static constexpr int BK = BK_, NT = NT_;
  static constexpr int CPT = VEC ? 4 : 1;
  static constexpr int TPR = ROWS / CPT;
  static constexpr int QSTEP = NT / TPR, NQ = (BK / 4) / QSTEP;
  using L = SwzPanel<ROWS, BK>;
  static constexpr int SIZE = L::SIZE;
  static_assert(NT % TPR == 0 && (BK / 4) % QSTEP == 0 && NQ >= 1, "LeanRowsMN split");
  using Reg = typename std::conditional<VEC, f32x4, float>::type;
  __amdgpu_buffer_rsrc_t rsrc;
  uint32_t voff, ld4;
  int ldsOff[NQ][CPT];
  Reg reg[NQ][4];

  __device__ inline void init(const float* p, int64_t bytes, int64_t ld, int64_t rows, int64_t r0, int tid) {
    rsrc = make_rsrc(p, bytes);
    ld4 = static_cast<uint32_t>(ld) * 4u;
    const int row = (tid % TPR) * CPT, q0 = tid / TPR;
    const int64_t gr = r0 + row;
    voff = sel_off(gr < rows, static_cast<uint32_t>((gr + 4 * q0 * ld) * 4));
#pragma unroll
    for (int j = 0; j < NQ; ++j)
#pragma unroll
      for (int c = 0; c < CPT; ++c) ldsOff[j][c] = L::chunk(row + c, q0 + j * QSTEP);
  }
  __device__ inline void load(int64_t k0) {
#pragma unroll
    for (int j = 0; j < NQ; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t so = static_cast<uint32_t>(static_cast<int>(k0) + 4 * j * QSTEP + e) * ld4;
        if constexpr (VEC)
          reg[j][e] = buf_ld4s(rsrc, voff, so);
        else
          reg[j][e] = buf_ld1s(rsrc, voff, so);
      }
  }
  __device__ inline void store(lds_t* stage) const {
#pragma unroll
    for (int j = 0; j < NQ; ++j) {
      if constexpr (VEC) {
#pragma unroll
        for (int c = 0; c < 4; ++c)
          *reinterpret_cast<lds_f4*>(stage + ldsOff[j][c]) =
              f32x4{reg[j][0][c], reg[j][1][c], reg[j][2][c], reg[j][3][c]};
      } else {
        *reinterpret_cast<lds_f4*>(stage + ldsOff[j][0]) = f32x4{reg[j][0], reg[j][1], reg[j][2], reg[j][3]};
      }
    }
  }
};

// Channels-last tap gather as the A operand (row r of the panel = output
// pixel m0 + r, k = tap*C + c with a panel inside one tap): a row's BK
// channels are contiguous, so each thread issues PER 16-byte loads per panel.
// Thread t owns chunk t % (BK/4) of rows t / (BK/4) + v * ROWSTEP.  A row's
// pixel offset at tap (0, 0) is fixed for the K loop (modulo 2^32: it may
// point before the image at the border); the uniform tap offset is added per
// panel, the channel offset rides in the scalar operand, and a per-row tap
// mask (computed once) sends taps in the padding to kOOB.
template <int ROWS, int BK_, int NT_, int KH, int KW>
struct NhwcTapRows {
  static constexpr int BK = BK_, NT = NT_;
  static constexpr int QPR = BK / 4;
  static constexpr int ROWSTEP = NT / QPR;
  static constexpr int PER = ROWS / ROWSTEP;
  using L = SwzPanel<ROWS, BK>;
  static constexpr int SIZE = L::SIZE;
  static_assert(NT % QPR == 0 && ROWS % ROWSTEP == 0 && PER >= 1 && ROWSTEP % 16 == 0 && KH * KW <= 32,
                "NhwcTapRows split");
  __amdgpu_buffer_rsrc_t rsrc;
  uint32_t rowOff[PER];
  uint32_t tapMask[PER];
  uint32_t pix4, rowPix4;  // bytes per pixel step, per image row
  int C;
  int ldsOff;
  f32x4 reg[PER];

  __device__ inline void init(const ConvGeom& g, int xPix, int64_t m0, int tid) {
    rsrc = make_rsrc(g.x, g.xBytes);
    C = g.C;
    pix4 = static_cast<uint32_t>(xPix) * 4u;
    rowPix4 = static_cast<uint32_t>(g.W) * pix4;
    const int row = tid / QPR, kq = tid % QPR;
#pragma unroll
    for (int v = 0; v < PER; ++v) {
      const int64_t n = m0 + row + v * ROWSTEP;
      const bool ok = n < g.N;
      const int64_t nn = ok ? n : 0;
      const int64_t b = nn / g.OHW;
      const int p = static_cast<int>(nn - b * g.OHW);
      const int oy = p / g.OW, ox = p - (p / g.OW) * g.OW;
      const int iy0 = oy * g.sY - g.pH, ix0 = ox * g.sX - g.pW;
      rowOff[v] = static_cast<uint32_t>(((b * g.H + iy0) * g.W + ix0) * xPix * 4 + kq * 16);
      uint32_t m = 0;
#pragma unroll
      for (int ky = 0; ky < KH; ++ky)
#pragma unroll
        for (int kx = 0; kx < KW; ++kx) {
          const bool in = static_cast<unsigned>(iy0 + ky) < static_cast<unsigned>(g.H) &&
                          static_cast<unsigned>(ix0 + kx) < static_cast<unsigned>(g.W);
          m |= (ok && in ? 1u : 0u) << (ky * KW + kx);
        }
      tapMask[v] = m;
    }
    ldsOff = L::chunk(row, kq);
  }
  __device__ inline void load(int64_t k0) {
    const int kk = static_cast<int>(k0);
    const int tap = kk / C;  // uniform
    const int c0 = kk - tap * C;
    const int ky = tap / KW, kx = tap - (tap / KW) * KW;
    const uint32_t tapOff = static_cast<uint32_t>(ky) * rowPix4 + static_cast<uint32_t>(kx) * pix4;
#pragma unroll
    for (int v = 0; v < PER; ++v)
      reg[v] = buf_ld4s(rsrc, sel_off((tapMask[v] >> tap) & 1u, rowOff[v] + tapOff), static_cast<uint32_t>(c0) * 4u);
  }
  __device__ inline void store(lds_t* stage) const {
#pragma unroll
    for (int v = 0; v < PER; ++v) *reinterpret_cast<lds_f4*>(stage + ldsOff + v * ROWSTEP * BK) = reg[v];
  }
};

// NhwcTapRows for 3x3 windows over any C % 4 == 0: a panel may span taps
// (C = 4, 8, 16: 32/C taps per panel; C = 48, 80, ...: a panel crosses one
// tap boundary) and the last panel may run past K = 9C (those chunks read
// 0).  A thread's chunk sits at k = k0 + 4*(t % (BK/4)): its tap and channel
// are found per panel (one approximate float division, corrected to the
// exact quotient); the rows' tap masks and pixel offsets are as in
// NhwcTapRows, the channel offset is per thread.
template <int ROWS, int BK_, int NT_>
struct NhwcTapRowsAny {
  static constexpr int BK = BK_, NT = NT_;
  static constexpr int QPR = BK / 4;
  static constexpr int ROWSTEP = NT / QPR;
  static constexpr int PER = ROWS / ROWSTEP;
  using L = SwzPanel<ROWS, BK>;
  static constexpr int SIZE = L::SIZE;
  static_assert(NT % QPR == 0 && ROWS % ROWSTEP == 0 && PER >= 1 && ROWSTEP % 16 == 0, "NhwcTapRowsAny split");
  __amdgpu_buffer_rsrc_t rsrc;
  uint32_t rowOff[PER];  // byte offset of the row's pixel at tap (0, 0), channel 0, modulo 2^32
  uint32_t tapMask[PER];
  uint32_t pix4, rowPix4;
  int C, K, kq4;
  float invC;
  int ldsOff;
  f32x4 reg[PER];

  __device__ inline void init(const ConvGeom& g, int xPix, int64_t m0, int tid) {
    rsrc = make_rsrc(g.x, g.xBytes);
    C = g.C;
    K = 9 * g.C;
    invC = 1.f / static_cast<float>(g.C);
    pix4 = static_cast<uint32_t>(xPix) * 4u;
    rowPix4 = static_cast<uint32_t>(g.W) * pix4;
    const int row = tid / QPR, kq = tid % QPR;
    kq4 = 4 * kq;
#pragma unroll
    for (int v = 0; v < PER; ++v) {
      const int64_t n = m0 + row + v * ROWSTEP;
      const bool ok = n < g.N;
      const int64_t nn = ok ? n : 0;
      const int64_t b = nn / g.OHW;
      const int p = static_cast<int>(nn - b * g.OHW);
      const int oy = p / g.OW, ox = p - (p / g.OW) * g.OW;
      const int iy0 = oy * g.sY - g.pH, ix0 = ox * g.sX - g.pW;
      rowOff[v] = static_cast<uint32_t>(((b * g.H + iy0) * g.W + ix0) * xPix * 4);
      uint32_t m = 0;
#pragma unroll
      for (int ky = 0; ky < 3; ++ky)
#pragma unroll
        for (int kx = 0; kx < 3; ++kx) {
          const bool in = static_cast<unsigned>(iy0 + ky) < static_cast<unsigned>(g.H) &&
                          static_cast<unsigned>(ix0 + kx) < static_cast<unsigned>(g.W);
          m |= (ok && in ? 1u : 0u) << (ky * 3 + kx);
        }
      tapMask[v] = m;
    }
    ldsOff = L::chunk(row, kq);
  }
  __device__ inline void load(int64_t k0) {
    const int k = static_cast<int>(k0) + kq4;
    // k / C: the float quotient is within one of the exact one for k < 2^22
    int tap = static_cast<int>(static_cast<float>(k) * invC);
    tap += (tap + 1) * C <= k ? 1 : 0;
    tap -= tap * C > k ? 1 : 0;
    const int c = k - tap * C;
    const bool kin = k < K;  // past K: tap >= 9, at most 9 + 31/4
    const int ky = tap / 3, kx = tap - (tap / 3) * 3;
    const uint32_t off = static_cast<uint32_t>(ky) * rowPix4 + static_cast<uint32_t>(kx) * pix4 +
                         static_cast<uint32_t>(c) * 4u;
#pragma unroll
    for (int v = 0; v < PER; ++v)
      reg[v] = buf_ld4s(rsrc, sel_off(kin && ((tapMask[v] >> tap) & 1u), rowOff[v] + off), 0u);
  }
  __device__ inline void store(lds_t* stage) const {
#pragma unroll
    for (int v = 0; v < PER; ++v) *reinterpret_cast<lds_f4*>(stage + ldsOff + v * ROWSTEP * BK) = reg[v];
  }
};

// Tap-major 3x3 gather (k = tap*C + c, a panel inside one tap): thread t
// owns output column t % BN and the k-quads t / BN + j * QSTEP; a quad is 4
// consecutive channels of one input pixel (4 loads HW floats apart), stored
// with one 16-byte LDS write.
template <class Cfg, int KH, int KW>
struct LeanTapB {
  static constexpr int BK = Cfg::BK, BN = Cfg::BN, NT = Cfg::NT;
  static constexpr int QSTEP = NT / BN, NQ = (BK / 4) / QSTEP;
  using L = SwzPanel<BN, BK>;
  static constexpr int SIZE = L::SIZE;
  static_assert(NT % BN == 0 && (BK / 4) % QSTEP == 0 && NQ >= 1 && KH * KW <= 32, "LeanTapB split");
  __amdgpu_buffer_rsrc_t rsrc;
  uint32_t colOff;   // byte offset of (image, iy0, ix0, channel 4 * first quad), modulo 2^32
  uint32_t tapMask;  // bit ky*KW + kx: that tap reads inside the image
  uint32_t HW4;
  int C, W;
  int ldsOff[NQ];
  float reg[NQ][4];

  __device__ inline void init(const ConvGeom& g, int64_t n0, int tid) {
    rsrc = make_rsrc(g.x, g.xBytes);
    C = g.C;
    W = g.W;
    HW4 = static_cast<uint32_t>(g.H) * static_cast<uint32_t>(g.W) * 4u;
    const int col = tid % BN, q0 = tid / BN;
    const int64_t n = n0 + col;
    const bool colOk = n < g.N;
    const int64_t nn = colOk ? n : 0;
    const int64_t b = nn / g.OHW;
    const int p = static_cast<int>(nn - b * g.OHW);
    const int oy = p / g.OW, ox = p - (p / g.OW) * g.OW;
    const int iy0 = oy * g.sY - g.pH, ix0 = ox * g.sX - g.pW;
    colOff = static_cast<uint32_t>((b * g.xBatchStride + static_cast<int64_t>(iy0) * g.W + ix0) * 4) +
             static_cast<uint32_t>(4 * q0) * HW4;
    uint32_t m = 0;
#pragma unroll
    for (int ky = 0; ky < KH; ++ky)
#pragma unroll
      for (int kx = 0; kx < KW; ++kx) {
        const bool in = static_cast<unsigned>(iy0 + ky) < static_cast<unsigned>(g.H) &&
                        static_cast<unsigned>(ix0 + kx) < static_cast<unsigned>(g.W);
        m |= (colOk && in ? 1u : 0u) << (ky * KW + kx);
      }
    tapMask = m;
#pragma unroll
    for (int j = 0; j < NQ; ++j) ldsOff[j] = L::chunk(col, q0 + j * QSTEP);
  }
  __device__ inline void load(int64_t k0) {
    const int kk = static_cast<int>(k0);
    const int tap = kk / C;  // uniform
    const int c0 = kk - tap * C;
    const int ky = tap / KW, kx = tap - (tap / KW) * KW;
    const uint32_t vo = sel_off((tapMask >> tap) & 1u, colOff + static_cast<uint32_t>(ky * W + kx) * 4u);
#pragma unroll
    for (int j = 0; j < NQ; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        reg[j][e] = buf_ld1s(rsrc, vo, static_cast<uint32_t>(c0 + 4 * j * QSTEP + e) * HW4);
  }
  __device__ inline void store(lds_t* stage) const {
#pragma unroll
    for (int j = 0; j < NQ; ++j)
      *reinterpret_cast<lds_f4*>(stage + ldsOff[j]) = f32x4{reg[j][0], reg[j][1], reg[j][2], reg[j][3]};
  }
};

// 1x1 stride 1: B[k = c][n = b*HW + p] = x_b[c][p].  Scalar: as LeanTapB
// without the tap (4 loads HW apart per quad).  VEC (HW % 4 == 0, batch
// stride % 4 == 0, x aligned): thread t owns columns 4 * (t % (BN/4)) .. +3
// and k-quads t / (BN/4) + j * QSTEP; it loads a 4 (k) x 4 (column) block
// with four 16-byte loads and stores its transpose, one 16-byte LDS write
// per column.
template <class Cfg, bool VEC>
struct Lean1x1B {
  static constexpr int BK = Cfg::BK, BN = Cfg::BN, NT = Cfg::NT;
  static constexpr int CPT = VEC ? 4 : 1;
  static constexpr int TPR = BN / CPT;
  static constexpr int QSTEP = NT / TPR, NQ = (BK / 4) / QSTEP;
  using L = SwzPanel<BN, BK>;
  static constexpr int SIZE = L::SIZE;
  static_assert(NT % TPR == 0 && (BK / 4) % QSTEP == 0 && NQ >= 1, "Lean1x1B split");
  using Reg = typename std::conditional<VEC, f32x4, float>::type;
  __amdgpu_buffer_rsrc_t rsrc;
  uint32_t voff, HW4;
  int ldsOff[NQ][CPT];
  Reg reg[NQ][4];

  __device__ inline void init(const ConvGeom& g, int64_t n0, int tid) {
    rsrc = make_rsrc(g.x, g.xBytes);
    const int64_t HW = g.OHW;
    HW4 = static_cast<uint32_t>(HW) * 4u;
    const int col = (tid % TPR) * CPT, q0 = tid / TPR;
    const int64_t n = n0 + col;
    const bool colOk = n < g.N;
    const int64_t nn = colOk ? n : 0;
    const int64_t b = nn / HW;
    voff = sel_off(colOk, static_cast<uint32_t>((b * g.xBatchStride + (nn - b * HW) + 4 * q0 * HW) * 4));
#pragma unroll
    for (int j = 0; j < NQ; ++j)
#pragma unroll
      for (int c = 0; c < CPT; ++c) ldsOff[j][c] = L::chunk(col + c, q0 + j * QSTEP);
  }
  __device__ inline void load(int64_t k0) {
#pragma unroll
    for (int j = 0; j < NQ; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t so = static_cast<uint32_t>(static_cast<int>(k0) + 4 * j * QSTEP + e) * HW4;
        if constexpr (VEC)
          reg[j][e] = buf_ld4s(rsrc, voff, so);
        else
          reg[j][e] = buf_ld1s(rsrc, voff, so);
      }
  }
  __device__ inline void store(lds_t* stage) const {
#pragma unroll
    for (int j = 0; j < NQ; ++j) {
      if constexpr (VEC) {
#pragma unroll
        for (int c = 0; c < 4; ++c)
          *reinterpret_cast<lds_f4*>(stage + ldsOff[j][c]) =
              f32x4{reg[j][0][c], reg[j][1][c], reg[j][2][c], reg[j][3][c]};
      } else {
        *reinterpret_cast<lds_f4*>(stage + ldsOff[j][0]) = f32x4{reg[j][0], reg[j][1], reg[j][2], reg[j][3]};
      }
    }
  }
};

template <class Cfg, class AL, class BL>
struct LeanLoop {
  static constexpr int FM = Cfg::FM, FN = Cfg::FN, KCH = Cfg::KCH, BK = Cfg::BK;
  static constexpr int STAGE = AL::SIZE + BL::SIZE;
  static constexpr int LDS_FLOATS = 2 * STAGE;

  // Eight k per lane and 32x32 block as two 16-byte halves: step s uses
  // element s % 4 of half s / 4 (k = 16*chunk + 8*(lane/32) + s).
  struct Frag {
    f32x4 a[FM][2];
    f32x4 b[FN][2];
  };

  // Per-lane float offsets inside a 32-row block of either panel (blocks
  // start at multiples of 32 rows, so a row's swizzle is that of lane % 32):
  // lo[c][e] addresses half e of chunk c.
  struct Lanes {
    int lo[KCH][2];
    int aRow, bRow;  // first row of the wave's blocks, times BK
  };

  __device__ static inline void read(const lds_t* stage, int c, const Lanes& L, Frag& f) {
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int e = 0; e < 2; ++e)
        f.a[i][e] = *reinterpret_cast<const lds_f4*>(stage + L.aRow + i * 32 * BK + L.lo[c][e]);
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int e = 0; e < 2; ++e)
        f.b[j][e] = *reinterpret_cast<const lds_f4*>(stage + AL::SIZE + L.bRow + j * 32 * BK + L.lo[c][e]);
  }

  __device__ static inline void mma(const Frag& f, f32x16 (&acc)[FM][FN]) {
#pragma unroll
    for (int s = 0; s < 8; ++s)
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(f.a[i][s >> 2][s & 3], f.b[j][s >> 2][s & 3], acc[i][j], 0,
                                                           0, 0);
  }

  // Panel p in stage S, fragments of its chunk 0 in f0.  MORE: panel p+1
  // exists (its registers are stored to the other stage); MORE2: panel p+2
  // exists (its loads are issued, at K offset kNext2).
  template <int S, bool MORE, bool MORE2>
  __device__ static inline void panel(AL& al, BL& bl, int64_t kNext2, lds_t* lds, Frag& f0, Frag& f1, const Lanes& L,
                                      f32x16 (&acc)[FM][FN]) {
    const lds_t* cur = lds + S * STAGE;
    lds_t* nxt = lds + (1 - S) * STAGE;
#pragma unroll
    for (int c = 0; c < KCH - 1; ++c) {
      Frag& fc = (c & 1) ? f1 : f0;
      Frag& fn = (c & 1) ? f0 : f1;
      read(cur, c + 1, L, fn);
      if (c == 0 && MORE) {
        al.store(nxt);
        bl.store(nxt + AL::SIZE);
        if (MORE2) {
          al.load(kNext2);
          bl.load(kNext2);
        }
      }
      mma(fc, acc);
    }
    if (MORE) {
      __syncthreads();
      read(nxt, 0, L, f0);
    }
    mma(f1, acc);  // chunk KCH-1 (KCH is even)
  }

  __device__ static inline Lanes lanes() {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave / Cfg::WN, wn = wave % Cfg::WN;
    const int r = lane & 31, h = lane >> 5;
    Lanes L;
#pragma unroll
    for (int c = 0; c < KCH; ++c)
#pragma unroll
      for (int e = 0; e < 2; ++e) L.lo[c][e] = SwzPanel<32, BK>::chunk(r, 4 * c + 2 * h + e);
    L.aRow = wm * Cfg::WTM * BK;
    L.bRow = wn * Cfg::WTN * BK;
    return L;
  }

  __device__ static inline void zero(f32x16 (&acc)[FM][FN]) {
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;
  }

  // Loads panel 0 into stage 0 and panel 1 into the registers, then reads
  // the fragments of chunk 0 of panel 0 (nk panels from kBegin).
  __device__ static inline void prologue(AL& al, BL& bl, int64_t kBegin, int64_t nk, lds_t* lds, const Lanes& L,
                                         Frag& f0) {
    al.load(kBegin);
    bl.load(kBegin);
    al.store(lds);
    bl.store(lds + AL::SIZE);
    if (nk > 1) {
      al.load(kBegin + BK);
      bl.load(kBegin + BK);
    }
    __syncthreads();
    read(lds, 0, L, f0);
  }

  __device__ static inline void add(f32x16 (&acc)[FM][FN], const f32x16 (&g)[FM][FN]) {
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[i][j][e] = acc[i][j][e] + g[i][j][e];
  }

  // Two-level sum over K: the MFMAs of each pair of panels (64 k) accumulate
  // from zero into g, which is then added to acc (the last partial sum may
  // hold up to three panels).  The matrix cores round
  // every step of a running sum; a long K (4608 in YOLOv3) summed in one
  // chain carries a rounding error several times that of 72 partial sums of
  // 64 products added in order, and that error compounds over a network's
  // layers (the CPU reference's own rounding is of the single-chain size,
  // so the GPU result's distance to it is mostly the reference's).
  // Measured on YOLOv3 against a float64 evaluation: head convolutions
  // 3.5-8.3e-6 -> 0.8-2.2e-6 (per tensor), batch-16 forward +0.8% (flushing
  // every 4 or 8 panels was no faster and less accurate).
  __device__ static inline void exec(AL& al, BL& bl, int64_t kBegin, int64_t nk, lds_t* lds,
                                     f32x16 (&acc)[FM][FN]) {
    const Lanes L = lanes();
    zero(acc);
    if (nk <= 0) return;
    Frag f0, f1;
    prologue(al, bl, kBegin, nk, lds, L, f0);
    f32x16 g[FM][FN];
    zero(g);
    int64_t p = 0;
    for (; p + 3 < nk; p += 2) {
      panel<0, true, true>(al, bl, kBegin + (p + 2) * BK, lds, f0, f1, L, g);
      panel<1, true, true>(al, bl, kBegin + (p + 3) * BK, lds, f0, f1, L, g);
      add(acc, g);
      zero(g);
    }
    const int64_t rest = nk - p;  // 1, 2 or 3 panels left; p is even (stage 0)
    if (rest == 3) {
      panel<0, true, true>(al, bl, kBegin + (p + 2) * BK, lds, f0, f1, L, g);
      panel<1, true, false>(al, bl, 0, lds, f0, f1, L, g);
      panel<0, false, false>(al, bl, 0, lds, f0, f1, L, g);
    } else if (rest == 2) {
      panel<0, true, false>(al, bl, 0, lds, f0, f1, L, g);
      panel<1, false, false>(al, bl, 0, lds, f0, f1, L, g);
    } else {
      panel<0, false, false>(al, bl, 0, lds, f0, f1, L, g);
    }
    add(acc, g);
  }
};

template <class Cfg, int MODE, bool VB>
struct LeanTraits;
template <class Cfg, bool VB>
struct LeanTraits<Cfg, kTap3, VB> {
  using BL = LeanTapB<Cfg, 3, 3>;
};
template <class Cfg, bool VB>
struct LeanTraits<Cfg, k1x1, VB> {
  // the 4x4 blocks of the vector loader must tile the panel exactly
  static constexpr bool kVec = VB && (Cfg::BK / 4) % (Cfg::NT / (Cfg::BN / 4)) == 0;
  using BL = Lean1x1B<Cfg, kVec>;
};

// A tail piece is one workgroup's raw accumulators (a BM x BN block) in
// register order, in 16-byte quads: quad q (registers 4q .. 4q+3) of
// accumulator block (i, j) of a wave is 64 lanes x 16 consecutive bytes, so
// every piece store and load is one coalesced 1 KB access per wave.
template <class Cfg>
__device__ inline int piece_quad(int wave, int lane, int i, int j, int q) {
  return (((wave * Cfg::FM * Cfg::FN + i * Cfg::FN + j) * 4 + q) * 64 + lane) * 4;
}

// Pieces are written through (kStoreThrough), like the epilogue's outputs:
// they are written in the last round and would otherwise stay dirty in L2
// until the end-of-kernel release.
template <class Cfg>
__device__ inline void store_piece(float* dst, int wave, int lane, const f32x16 (&acc)[Cfg::FM][Cfg::FN]) {
  const __amdgpu_buffer_rsrc_t r = make_rsrc(dst, static_cast<int64_t>(Cfg::BM) * Cfg::BN * 4);
#pragma unroll
  for (int i = 0; i < Cfg::FM; ++i)
#pragma unroll
    for (int j = 0; j < Cfg::FN; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const f32x4 v{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(__attribute__((ext_vector_type(4))) uint32_t, v), r,
                                               static_cast<uint32_t>(piece_quad<Cfg>(wave, lane, i, j, q)) * 4u, 0,
                                               kStoreThrough);
      }
}

// Sums the P pieces of one tail tile (src: piece 0 of the tile) in K order,
// piece 0 first, into the accumulator registers of `wave` that the conv
// kernel would have held.  The loads of G pieces are issued together (one
// memory round trip per G pieces instead of per piece); the sum still runs
// in piece order, so the result does not depend on which workgroup sums.
// SYS: the loads are system-scope (they read the pieces where the pieces'
// write-through stores put them, past any copy in this XCD's caches), for a
// reduction inside the kernel that wrote them.
template <class Cfg, bool SYS = false>
__device__ inline void sum_pieces(const float* src, int P, int wave, int lane, f32x16 (&acc)[Cfg::FM][Cfg::FN]) {
  constexpr int TILE = Cfg::BM * Cfg::BN;
  constexpr int G = Cfg::FM * Cfg::FN <= 2 ? 4 : 2;
  const __amdgpu_buffer_rsrc_t r = make_rsrc(src, static_cast<int64_t>(P) * TILE * 4);
  for (int s0 = 0; s0 < P; s0 += G) {
    f32x4 part[G][Cfg::FM][Cfg::FN][4];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const int64_t base = static_cast<int64_t>(s0 + g < P ? s0 + g : P - 1) * TILE;
#pragma unroll
      for (int i = 0; i < Cfg::FM; ++i)
#pragma unroll
        for (int j = 0; j < Cfg::FN; ++j)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int64_t e = base + piece_quad<Cfg>(wave, lane, i, j, q);
            if constexpr (SYS)
              part[g][i][j][q] = __builtin_bit_cast(
                  f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<uint32_t>(e) * 4u, 0, kStoreThrough));
            else
              part[g][i][j][q] = *reinterpret_cast<const f32x4*>(src + e);
          }
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
      if (s0 + g >= P) break;  // uniform
#pragma unroll
      for (int i = 0; i < Cfg::FM; ++i)
#pragma unroll
        for (int j = 0; j < Cfg::FN; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const float v = part[g][i][j][r >> 2][r & 3];
            acc[i][j][r] = s0 + g == 0 ? v : acc[i][j][r] + v;
          }
    }
  }
}

// A piece's workgroup, after storing its piece, counts itself in tile t's
// arrival counter; returns true in every thread of the workgroup that
// arrives last, which then owns the tile's reduction and epilogue and has
// reset the counter to 0 for the next launch.  The pieces are stored
// write-through at system scope (store_piece), so once each wave's stores
// have completed (s_waitcnt 0, before the barrier that precedes thread 0's
// increment) they are in memory; the last workgroup reads them back with
// system-scope loads (sum_pieces<Cfg, true>), which fetch from memory past
// its XCD's caches.  An agent-scope fence pair would do the same at the cost
// of an L2 write-back per piece and an L2 invalidation under the workgroups
// still running on that XCD (measured: +0.45 ms per batch-16 YOLOv3
// forward).  No workgroup waits for another.
__device__ inline bool tail_arrive(const ConvArgs& a, int t, int* flag) {
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) {
    const int before = __hip_atomic_fetch_add(a.tileCount + t, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int last = before == a.tailSplits - 1;
    if (last) __hip_atomic_store(a.tileCount + t, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *flag = last;
  }
  __syncthreads();
  return *flag != 0;
}

template <class Cfg, int MODE, bool VB>
__global__ __launch_bounds__(Cfg::NT, Cfg::OCC) void conv_lean_kernel(ConvArgs a) {
  using AL = LeanA<Cfg>;
  using BL = typename LeanTraits<Cfg, MODE, VB>::BL;
  using Loop = LeanLoop<Cfg, AL, BL>;
  __shared__ __attribute__((aligned(16))) float smem[Loop::LDS_FLOATS];
  lds_t* lds = (lds_t*)smem;

  int tile = blockIdx.x;
  int64_t kBegin = blockIdx.y * a.kChunk;
  int piece = -1;
  if (a.tailSplits > 0 && tile >= a.nFull) {  // a K piece of a tail tile
    const int u = tile - a.nFull;
    tile = a.nFull + u / a.tailSplits;
    kBegin = static_cast<int64_t>(u % a.tailSplits) * a.kChunk;
    piece = u;
  }
  const int64_t kEnd = a.tailSplits > 0 && piece < 0 ? a.g.K : min(a.g.K, kBegin + a.kChunk);
  int tm, tn;
  tile_coords(tile, a.tilesM, a.tilesN, tm, tn);
  const int64_t m0 = static_cast<int64_t>(tm) * Cfg::BM, n0 = static_cast<int64_t>(tn) * Cfg::BN;
  AL al;
  al.init(a.w, a.wBytes, a.g.K, a.F, m0, threadIdx.x);
  BL bl;
  bl.init(a.g, n0, threadIdx.x);
  f32x16 acc[Cfg::FM][Cfg::FN];
  Loop::exec(al, bl, kBegin, (kEnd - kBegin) / Cfg::BK, lds, acc);

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (piece >= 0) {
    store_piece<Cfg>(a.part + static_cast<int64_t>(piece) * (Cfg::BM * Cfg::BN), wave, lane, acc);
    if (!a.tileCount) return;
    __shared__ int lastFlag;
    const int t = tile - a.nFull;
    if (!tail_arrive(a, t, &lastFlag)) return;
    sum_pieces<Cfg, true>(a.part + static_cast<int64_t>(t) * a.tailSplits * (Cfg::BM * Cfg::BN), a.tailSplits,
                          wave, lane, acc);
  }
  const int wm = wave / Cfg::WN, wn = wave % Cfg::WN;
  conv_store_buf<Cfg::FM, Cfg::FN>(a, acc, m0 + wm * Cfg::WTM, n0 + wn * Cfg::WTN, lane);
}

// Second launch of a tail split: one workgroup per tail tile sums the tile's
// pieces in K order (piece 0 first, as conv_splitk_reduce does) into the
// accumulator registers the conv kernel would have held, then applies the
// conv kernel's own epilogue.
template <class Cfg, bool NHWC = false, bool VAR = false>
__global__ __launch_bounds__(64) void conv_tail_reduce(ConvArgs a) {
  // one single-wave workgroup per wave of a tail tile: the reduction of a
  // few tail tiles still spreads over every CU
  constexpr int NW = Cfg::NT / 64;
  const int t = blockIdx.x / NW;
  int tm, tn;
  tile_coords(a.nFull + t, a.tilesM, a.tilesN, tm, tn);
  const int64_t m0 = static_cast<int64_t>(tm) * Cfg::BM, n0 = static_cast<int64_t>(tn) * Cfg::BN;
  const int lane = threadIdx.x, wave = blockIdx.x - t * NW;
  constexpr int TILE = Cfg::BM * Cfg::BN;
  const int P = a.tailSplits;
  f32x16 acc[Cfg::FM][Cfg::FN];
  sum_pieces<Cfg>(a.part + static_cast<int64_t>(t) * P * TILE, P, wave, lane, acc);
  const int wm = wave / Cfg::WN, wn = wave % Cfg::WN;
  if constexpr (NHWC)
    conv_store_nhwc<Cfg::FM, Cfg::FN, VAR>(a, acc, m0 + wm * Cfg::WTM, n0 + wn * Cfg::WTN, lane);
  else
    conv_store_buf<Cfg::FM, Cfg::FN>(a, acc, m0 + wm * Cfg::WTM, n0 + wn * Cfg::WTN, lane);
}

// Channels-last convolution: rows of the GEMM are output pixels (A: the
// input gathered per tap, or for a 1x1 stride-1 conv the input rows
// themselves), columns are filters (B: the tap-major weights [F][K], k
// contiguous), so both operands load 16 bytes along k and the epilogue
// writes 32 consecutive channels of a pixel per half-wave.  Tail split as in
// conv_lean_kernel (nFull may be 0: every tile cut into K pieces; with
// ConvArgs::tileCount the last piece's workgroup reduces the tile).  The Any
// modes (C % 32 != 0) take ceil(K / BK) panels with the K tail reading 0, and
// no tail split.  VAR: the instantiation for the epilogue variants (an
// upsampled output or a yolo head; the plain kernels carry no code for them).
template <class Cfg, int MODE, bool VAR = false>
__global__ __launch_bounds__(Cfg::NT, Cfg::OCC) void conv_nhwc_kernel(ConvArgs a) {
  constexpr bool ANY = MODE == kTap3Any || MODE == k1x1Any;
  constexpr bool TAP = MODE == kTap3 || MODE == kTap3Any;
  using AL = typename std::conditional<
      MODE == kTap3, NhwcTapRows<Cfg::BM, Cfg::BK, Cfg::NT, 3, 3>,
      typename std::conditional<MODE == kTap3Any, NhwcTapRowsAny<Cfg::BM, Cfg::BK, Cfg::NT>,
                                LeanRowsK<Cfg::BM, Cfg::BK, Cfg::NT, ANY>>::type>::type;
  using BL = LeanRowsK<Cfg::BN, Cfg::BK, Cfg::NT, ANY>;
  using Loop = LeanLoop<Cfg, AL, BL>;
  __shared__ __attribute__((aligned(16))) float smem[Loop::LDS_FLOATS];
  lds_t* lds = (lds_t*)smem;

  int tile = blockIdx.x;
  int64_t kBegin = 0;
  int piece = -1;
  if (a.tailSplits > 0 && tile >= a.nFull) {  // a K piece of a tail tile
    const int u = tile - a.nFull;
    tile = a.nFull + u / a.tailSplits;
    kBegin = static_cast<int64_t>(u % a.tailSplits) * a.kChunk;
    piece = u;
  }
  const int64_t kEnd = piece < 0 ? a.g.K : min(a.g.K, kBegin + a.kChunk);
  int tm, tn;
  tile_coords(tile, a.tilesM, a.tilesN, tm, tn);
  const int64_t m0 = static_cast<int64_t>(tm) * Cfg::BM, n0 = static_cast<int64_t>(tn) * Cfg::BN;
  AL al;
  if constexpr (TAP) {
    al.init(a.g, a.xPix, m0, threadIdx.x);
  } else {
    al.init(a.g.x, a.g.xBytes, a.xPix, a.g.N, m0, threadIdx.x);
    if constexpr (ANY) al.klimit(a.g.K);
  }
  BL bl;
  bl.init(a.w, a.wBytes, a.g.K, a.F, n0, threadIdx.x);
  if constexpr (ANY) bl.klimit(a.g.K);
  f32x16 acc[Cfg::FM][Cfg::FN];
  Loop::exec(al, bl, kBegin, (kEnd - kBegin + Cfg::BK - 1) / Cfg::BK, lds, acc);

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (!ANY && piece >= 0) {
    store_piece<Cfg>(a.part + static_cast<int64_t>(piece) * (Cfg::BM * Cfg::BN), wave, lane, acc);
    if (!a.tileCount) return;
    __shared__ int lastFlag;
    const int t = tile - a.nFull;
    if (!tail_arrive(a, t, &lastFlag)) return;
    sum_pieces<Cfg, true>(a.part + static_cast<int64_t>(t) * a.tailSplits * (Cfg::BM * Cfg::BN), a.tailSplits, wave,
                    lane, acc);
  }
  const int wm = wave / Cfg::WN, wn = wave % Cfg::WN;
  conv_store_nhwc<Cfg::FM, Cfg::FN, VAR>(a, acc, m0 + wm * Cfg::WTM, n0 + wn * Cfg::WTN, lane);
}

}  // namespace conv
}  // namespace tnh
