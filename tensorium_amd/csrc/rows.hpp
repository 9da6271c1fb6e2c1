// Row walk of per-channel element-wise passes, shared by the element-wise
// and training kernels.  A tensor [groups][nb][block] is walked as rows of
// `block` contiguous floats; row r belongs to channel r % nb.  A kernel loads
// a channel's constants once per row, so its element loop holds no index
// division, and reads and writes a row 16 bytes at a time when block % 4 ==
// 0 and the bases are 16-byte aligned.  A workgroup pass covers rpw rows of
// cpt threads each (short rows share a workgroup; long rows loop over their
// chunks).
#pragma once
#include "common.hpp"

namespace tnh {

struct Rows {
  int64_t rows, block, nb;
  int64_t cpr;  // VW-wide chunks per row
  int cpt;      // threads per row in one pass
  int rpw;      // rows per workgroup pass
};

constexpr int kRowThreads = 256;

inline Rows make_rows(int64_t n, int64_t block, int64_t nb, int vw) {
  Rows g;
  g.rows = n / block;
  g.block = block;
  g.nb = nb;
  g.cpr = block / vw;
  g.cpt = static_cast<int>(g.cpr < kRowThreads ? g.cpr : kRowThreads);
  g.rpw = kRowThreads / g.cpt;
  return g;
}

inline unsigned grid_rows(const Rows& g) {
  const int64_t b = (g.rows + g.rpw - 1) / g.rpw;
  return static_cast<unsigned>(b < 16384 ? (b > 0 ? b : 1) : 16384);
}

inline bool rows_al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// Calls body(row, chunk) for the rows and VW-wide chunks of this thread
// (threads beyond rpw rows of a workgroup do nothing).
template <class Body>
__device__ inline void rows_walk(const Rows& g, Body body) {
  const int t = threadIdx.x, lr = t / g.cpt, lc = t - lr * g.cpt;
  if (lr >= g.rpw) return;
  for (int64_t r = static_cast<int64_t>(blockIdx.x) * g.rpw + lr; r < g.rows;
       r += static_cast<int64_t>(gridDim.x) * g.rpw)
    body(r, lc);
}

}  // namespace tnh
