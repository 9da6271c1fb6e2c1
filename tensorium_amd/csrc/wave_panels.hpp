// Per-wave operand panels for the wave-split kernels (conv_wsplit.hip,
// sgemm.hip): each wave of a workgroup fetches its own K range of a tile's
// operands into its own LDS panel [ROWS][32] (k-contiguous, 16-byte chunks
// XOR-swizzled as SwzPanel), so the K loop needs no barrier.
#pragma once
#include "conv_lean.hpp"

namespace tnh {
namespace conv {

// One wave's k-contiguous operand rows r0 .. r0 + ROWS - 1 (row stride ld
// floats, rows >= `rows` read 0): lane t fetches chunk t % 8 (16 bytes) of
// rows t / 8 + 8v.  The weights [F][K], and for a 1x1 stride-1 conv the
// input pixels themselves.
template <int ROWS>
struct WaveRowsK {
  static constexpr int PER = ROWS / 8;
  using L = SwzPanel<ROWS, 32>;
  static constexpr int SIZE = L::SIZE;
  __amdgpu_buffer_rsrc_t rsrc;
  uint32_t voff[PER];
  int ldsOff[PER];
  f32x4 reg[PER];
  __device__ inline void init(const float* p, int64_t bytes, int64_t ld, int64_t rows, int64_t r0, int lane) {
    rsrc = make_rsrc(p, bytes);
#pragma unroll
    for (int v = 0; v < PER; ++v) {
      const int row = lane / 8 + 8 * v, q = lane % 8;
      const int64_t gr = r0 + row;
      voff[v] = sel_off(gr < rows, static_cast<uint32_t>((gr * ld + 4 * q) * 4));
      ldsOff[v] = L::chunk(row, q);
    }
  }
  __device__ inline void load(int k0) {
#pragma unroll
    for (int v = 0; v < PER; ++v) reg[v] = buf_ld4s(rsrc, voff[v], static_cast<uint32_t>(k0) * 4u);
  }
  __device__ inline void store(lds_t* panel) const {
#pragma unroll
    for (int v = 0; v < PER; ++v) *reinterpret_cast<lds_f4*>(panel + ldsOff[v]) = reg[v];
  }
};

// One wave's row-contiguous operand (element (row r, k) at (r0 + r) + k * ld
// floats, rows >= `rows` read 0; rows % 4 == 0 and ld % 4 == 0 with a 16-byte
// aligned base, so a 4-row vector is whole or absent): lane t takes the 4 x 4
// blocks b = t + 64v, rows 4*(b % (ROWS/4)) .. +3 and k 4*(b / (ROWS/4)) ..
// +3, as four 16-byte loads (one per k), and stores their transpose, one
// 16-byte LDS write per row.  The GEMM operands A transposed and B not
// transposed.
template <int ROWS>
struct WaveRowsMN {
  static constexpr int RQ = ROWS / 4;
  static constexpr int PER = RQ * 8 / 64;
  using L = SwzPanel<ROWS, 32>;
  static constexpr int SIZE = L::SIZE;
  static_assert(ROWS % 32 == 0 && PER >= 1, "WaveRowsMN rows");
  __amdgpu_buffer_rsrc_t rsrc;
  uint32_t voff[PER], ld4;
  int ldsOff[PER][4];
  f32x4 reg[PER][4];
  __device__ inline void init(const float* p, int64_t bytes, int64_t ld, int64_t rows, int64_t r0, int lane) {
    rsrc = make_rsrc(p, bytes);
    ld4 = static_cast<uint32_t>(ld) * 4u;
#pragma unroll
    for (int v = 0; v < PER; ++v) {
      const int b = lane + 64 * v;
      const int rq = b % RQ, kq = b / RQ;
      const int64_t gr = r0 + 4 * rq;
      voff[v] = sel_off(gr < rows, static_cast<uint32_t>((gr + 4 * kq * ld) * 4));
#pragma unroll
      for (int c = 0; c < 4; ++c) ldsOff[v][c] = L::chunk(4 * rq + c, kq);
    }
  }
  __device__ inline void load(int k0) {
#pragma unroll
    for (int v = 0; v < PER; ++v)
#pragma unroll
      for (int e = 0; e < 4; ++e) reg[v][e] = buf_ld4s(rsrc, voff[v], static_cast<uint32_t>(k0 + e) * ld4);
  }
  __device__ inline void store(lds_t* panel) const {
#pragma unroll
    for (int v = 0; v < PER; ++v)
#pragma unroll
      for (int c = 0; c < 4; ++c)
        *reinterpret_cast<lds_f4*>(panel + ldsOff[v][c]) = f32x4{reg[v][0][c], reg[v][1][c], reg[v][2][c], reg[v][3][c]};
  }
};

}  // namespace conv
}  // namespace tnh
