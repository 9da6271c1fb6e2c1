// fp32 GEMM core on CDNA4 matrix cores (gfx950), shared by the plain SGEMM
// entry points and the implicit-GEMM convolution.
//
// One workgroup computes a BM x BN tile of C with NWAVES = WM*WN wavefronts;
// each wave owns a (BM/WM) x (BN/WN) sub-tile made of 32x32 blocks, each
// accumulated by v_mfma_f32_32x32x2_f32.  Operands stream through LDS in
// BK = 16 deep panels, double buffered, one barrier per panel; the next
// panel's global loads are issued before the current panel's MFMAs so that
// their latency hides behind matrix work.
//
// MFMA operand layout of v_mfma_f32_32x32x2_f32 (one 32x32x2 block):
//   A: lane l supplies A[m = l%32][kk = l/32]
//   B: lane l supplies B[kk = l/32][n = l%32]
//   D: lane l, register r holds D[m = 8*(r/4) + 4*(l/32) + r%4][n = l%32]
// Within a BK = 16 panel, MFMA step s (0..7) pairs k = s (lanes 0-31) with
// k = 8 + s (lanes 32-63), so a lane's eight A values of the panel are 8
// contiguous k and can be read from a k-contiguous LDS tile with two 16-byte
// loads.  The sum over k is unchanged; only the fp32 accumulation order
// differs from the reference's sequential chain (covered by the 1e-5
// per-tensor tolerance; exact for integer-valued data).
//
// Operand tiles live in LDS in one of two layouts, chosen so that the
// global->LDS copy never transposes:
//   KC ("k contiguous"):   tile[row][BK + 4]   (A normal, B transposed)
//   MC ("row contiguous"): tile[BK][ROWS + 4]  (A transposed, B normal,
//                                               implicit im2col gather)
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>
#include <type_traits>

namespace tnh {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kBK = 16;   // panel depth
constexpr int kPad = 4;   // LDS row padding (floats)

template <int BM_, int BN_, int WM_, int WN_>
struct TileCfg {
  static constexpr int BM = BM_, BN = BN_, WM = WM_, WN = WN_;
  static constexpr int NWAVES = WM * WN;
  static constexpr int NT = NWAVES * 64;
  static constexpr int WTM = BM / WM, WTN = BN / WN;  // wave tile
  static constexpr int FM = WTM / 32, FN = WTN / 32;  // 32x32 blocks per wave
  static_assert(FM >= 1 && FN >= 1 && WTM % 32 == 0 && WTN % 32 == 0, "tile");
};

// LDS footprint (floats) of one operand panel in a layout.
template <bool KC, int ROWS>
struct PanelLayout {
  static constexpr int PITCH = KC ? (kBK + kPad) : (ROWS + kPad);
  static constexpr int SIZE = KC ? ROWS * PITCH : kBK * PITCH;
  __device__ static inline int at(int row, int k) { return KC ? row * PITCH + k : k * PITCH + row; }
};

// Reads the eight per-step operand values of one 32-row block for this lane.
template <bool KC, int ROWS>
__device__ inline void read_frag(const float* __restrict__ lds, int row0, int lane, float (&v)[8]) {
  using L = PanelLayout<KC, ROWS>;
  const int r = lane & 31, h = lane >> 5;
  if constexpr (KC) {
    const f32x4* p = reinterpret_cast<const f32x4*>(lds + L::at(row0 + r, h * 8));
    f32x4 a = p[0], b = p[1];
    v[0] = a[0]; v[1] = a[1]; v[2] = a[2]; v[3] = a[3];
    v[4] = b[0]; v[5] = b[1]; v[6] = b[2]; v[7] = b[3];
  } else {
#pragma unroll
    for (int s = 0; s < 8; ++s) v[s] = lds[L::at(row0 + r, h * 8 + s)];
  }
}

// ---------------------------------------------------------------------------
// Dense operand loaders.  Operand element (row, k) of op(X):
//   KC (k contiguous in memory):   X[(row0+row)*ld + k0 + k]
//   MC (row contiguous in memory): X[(k0+k)*ld + row0 + row]
// VEC: 16-byte loads (caller guarantees alignment, ld % 4 == 0 and the
// contiguous extent % 4 == 0, so a vector is entirely in or out of range).
// ---------------------------------------------------------------------------
template <bool KC, bool VEC, int ROWS, int NT>
struct DenseLoader {
  static constexpr bool kKC = KC;
  static constexpr int ELEMS = ROWS * kBK;
  static constexpr int PER = VEC ? ELEMS / 4 / NT : ELEMS / NT;  // loads per thread
  static_assert(PER >= 1 && (VEC ? ELEMS / 4 : ELEMS) % NT == 0, "loader split");
  using Reg = typename std::conditional<VEC, f32x4, float>::type;

  const float* __restrict__ base;  // already offset to the batch item
  int64_t ld;
  int64_t rows;  // M (or N) extent
  int64_t K;

  Reg reg[PER];

  __device__ inline void coords(int idx, int& row, int& k) const {
    if constexpr (KC) {
      constexpr int PR = VEC ? kBK / 4 : kBK;  // vectors per row
      row = idx / PR;
      k = (idx % PR) * (VEC ? 4 : 1);
    } else {
      constexpr int PR = VEC ? ROWS / 4 : ROWS;
      k = idx / PR;
      row = (idx % PR) * (VEC ? 4 : 1);
    }
  }

  __device__ inline void load(int64_t row0, int64_t k0, int tid) {
#pragma unroll
    for (int v = 0; v < PER; ++v) {
      int row, k;
      coords(tid + v * NT, row, k);
      const int64_t gr = row0 + row, gk = k0 + k;
      const bool ok = gr < rows && gk < K;
      const int64_t off = KC ? gr * ld + gk : gk * ld + gr;
      if constexpr (VEC) {
        reg[v] = ok ? *reinterpret_cast<const f32x4*>(base + off) : f32x4{0.f, 0.f, 0.f, 0.f};
      } else {
        reg[v] = ok ? base[off] : 0.f;
      }
    }
  }

  __device__ inline void store(float* __restrict__ lds, int tid) const {
    using L = PanelLayout<KC, ROWS>;
#pragma unroll
    for (int v = 0; v < PER; ++v) {
      int row, k;
      coords(tid + v * NT, row, k);
      if constexpr (VEC)
        *reinterpret_cast<f32x4*>(lds + L::at(row, k)) = reg[v];
      else
        lds[L::at(row, k)] = reg[v];
    }
  }
};

// ---------------------------------------------------------------------------
// Implicit im2col gather for the B operand of a convolution (MC layout).
// Column n = b*OH*OW + oy*OW + ox (batch merged into N); row k = (c*KH + ky)*KW
// + kx; value = x_b[c][oy*sY - pH + ky][ox*sX - pW + kx] or 0 (sim2Col's
// formula, ntensors.pas:11440-11455, dilation 1).  Each thread owns one
// column for the whole K loop and BK*BN/NT rows of each panel.
// ---------------------------------------------------------------------------
template <int KH, int KW, int BN, int NT>
struct ConvGatherLoader {
  static constexpr bool kKC = false;
  static constexpr int RSTEP = NT / BN;       // rows between a thread's loads
  static constexpr int PER = kBK * BN / NT;   // loads per thread per panel
  static_assert(NT % BN == 0 && PER >= 1, "gather split");

  const float* __restrict__ x;
  int64_t xBatchStride;
  int H, W, OW, OHW;
  int sY, sX, pH, pW;
  int64_t N, K;

  // per-thread column state
  int64_t colBase;  // x offset of image b, row iy0, col ix0 (may be "negative")
  int iy0, ix0;
  bool colOk;
  int myCol, myRow0;

  float reg[PER];

  __device__ inline void init_col(int64_t n0, int tid) {
    myCol = tid % BN;
    myRow0 = tid / BN;
    const int64_t n = n0 + myCol;
    colOk = n < N;
    const int64_t nn = colOk ? n : 0;
    const int64_t b = nn / OHW;
    const int p = static_cast<int>(nn - b * OHW);
    const int oy = p / OW, ox = p - (p / OW) * OW;
    iy0 = oy * sY - pH;
    ix0 = ox * sX - pW;
    colBase = b * xBatchStride + static_cast<int64_t>(iy0) * W + ix0;
  }

  __device__ inline void load(int64_t /*row0*/, int64_t k0, int /*tid*/) {
    const int64_t HW = static_cast<int64_t>(H) * W;
#pragma unroll
    for (int v = 0; v < PER; ++v) {
      const int k = static_cast<int>(k0) + myRow0 + v * RSTEP;
      const int c = k / (KH * KW);
      const int r = k - c * (KH * KW);
      const int ky = r / KW, kx = r - (r / KW) * KW;
      const int iy = iy0 + ky, ix = ix0 + kx;
      const bool ok = colOk && k < static_cast<int>(K) && static_cast<unsigned>(iy) < static_cast<unsigned>(H) &&
                      static_cast<unsigned>(ix) < static_cast<unsigned>(W);
      reg[v] = ok ? x[colBase + c * HW + ky * W + kx] : 0.f;
    }
  }

  __device__ inline void store(float* __restrict__ lds, int /*tid*/) const {
    using L = PanelLayout<false, BN>;
#pragma unroll
    for (int v = 0; v < PER; ++v) lds[L::at(myCol, myRow0 + v * RSTEP)] = reg[v];
  }
};

// 1x1 stride-1 convolution: B[k = c][n = b*HW + p] = x_b[c][p]; VEC loads 4
// consecutive columns (requires HW % 4 == 0, xBatchStride % 4 == 0, aligned).
template <bool VEC, int BN, int NT>
struct Conv1x1Loader {
  static constexpr bool kKC = false;
  static constexpr int CPT = VEC ? 4 : 1;              // columns per load
  static constexpr int TPR = BN / CPT;                 // threads per k row
  static constexpr int RSTEP = NT / TPR;
  static constexpr int PER = kBK / RSTEP;
  static_assert(NT % TPR == 0 && PER >= 1 && kBK % RSTEP == 0, "1x1 split");
  using Reg = typename std::conditional<VEC, f32x4, float>::type;

  const float* __restrict__ x;
  int64_t xBatchStride;
  int64_t HW;
  int64_t N, K;

  int64_t colBase;
  bool colOk;
  int myCol, myRow0;
  Reg reg[PER];

  __device__ inline void init_col(int64_t n0, int tid) {
    myCol = (tid % TPR) * CPT;
    myRow0 = tid / TPR;
    const int64_t n = n0 + myCol;
    colOk = n < N;
    const int64_t nn = colOk ? n : 0;
    const int64_t b = nn / HW;
    colBase = b * xBatchStride + (nn - b * HW);
  }

  __device__ inline void load(int64_t, int64_t k0, int) {
#pragma unroll
    for (int v = 0; v < PER; ++v) {
      const int64_t k = k0 + myRow0 + v * RSTEP;
      const bool ok = colOk && k < K;
      if constexpr (VEC)
        reg[v] = ok ? *reinterpret_cast<const f32x4*>(x + colBase + k * HW) : f32x4{0.f, 0.f, 0.f, 0.f};
      else
        reg[v] = ok ? x[colBase + k * HW] : 0.f;
    }
  }

  __device__ inline void store(float* __restrict__ lds, int) const {
    using L = PanelLayout<false, BN>;
#pragma unroll
    for (int v = 0; v < PER; ++v) {
      if constexpr (VEC)
        *reinterpret_cast<f32x4*>(lds + L::at(myCol, myRow0 + v * RSTEP)) = reg[v];
      else
        lds[L::at(myCol, myRow0 + v * RSTEP)] = reg[v];
    }
  }
};

// ---------------------------------------------------------------------------
// Tile scheduling: workgroups are dispatched round-robin over the 8 XCDs
// (each with its own L2).  Remap the linear id so that each XCD receives a
// contiguous range of tiles, then walk that range in GROUP_M-row groups so
// the tiles an XCD runs together share A rows and B columns in its L2.
// ---------------------------------------------------------------------------
__device__ inline void tile_coords(int pid, int tilesM, int tilesN, int& tm, int& tn) {
  const int total = tilesM * tilesN;
  constexpr int XCD = 8;
  if (total % XCD == 0) pid = (pid % XCD) * (total / XCD) + pid / XCD;
  constexpr int GROUP_M = 8;
  const int groupSize = GROUP_M * tilesN;
  const int g = pid / groupSize;
  const int firstM = g * GROUP_M;
  const int gm = min(tilesM - firstM, GROUP_M);
  const int inGroup = pid - g * groupSize;
  tm = firstM + inGroup % gm;
  tn = inGroup / gm;
}

// ---------------------------------------------------------------------------
// The main loop.  ALoader/BLoader fill LDS panels; Epi receives every
// accumulated element with its (row, col) in C.
// ---------------------------------------------------------------------------
template <class Cfg, class AL, class BL>
struct GemmMainloop {
  using LA = PanelLayout<AL::kKC, Cfg::BM>;
  using LB = PanelLayout<BL::kKC, Cfg::BN>;
  static constexpr int LDS_FLOATS = 2 * (LA::SIZE + LB::SIZE);

  // acc[i][j] is the 32x32 block (i, j) of this wave's sub-tile.
  __device__ static inline void run(AL& al, BL& bl, int64_t m0, int64_t n0, int64_t kBegin, int64_t kEnd,
                                    float* lds, f32x16 (&acc)[Cfg::FM][Cfg::FN]) {
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave / Cfg::WN, wn = wave % Cfg::WN;
    float* ldsA[2] = {lds, lds + LA::SIZE + LB::SIZE};
    float* ldsB[2] = {lds + LA::SIZE, lds + 2 * LA::SIZE + LB::SIZE};

#pragma unroll
    for (int i = 0; i < Cfg::FM; ++i)
#pragma unroll
      for (int j = 0; j < Cfg::FN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    const int64_t nk = (kEnd - kBegin + kBK - 1) / kBK;
    if (nk <= 0) return;
    al.load(m0, kBegin, tid);
    bl.load(n0, kBegin, tid);
    al.store(ldsA[0], tid);
    bl.store(ldsB[0], tid);
    __syncthreads();

    for (int64_t kt = 0; kt < nk; ++kt) {
      const int cur = static_cast<int>(kt & 1);
      const bool more = kt + 1 < nk;
      if (more) {
        al.load(m0, kBegin + (kt + 1) * kBK, tid);
        bl.load(n0, kBegin + (kt + 1) * kBK, tid);
      }
      float a[Cfg::FM][8], b[Cfg::FN][8];
#pragma unroll
      for (int i = 0; i < Cfg::FM; ++i)
        read_frag<AL::kKC, Cfg::BM>(ldsA[cur], wm * Cfg::WTM + i * 32, lane, a[i]);
#pragma unroll
      for (int j = 0; j < Cfg::FN; ++j)
        read_frag<BL::kKC, Cfg::BN>(ldsB[cur], wn * Cfg::WTN + j * 32, lane, b[j]);
#pragma unroll
      for (int s = 0; s < 8; ++s)
#pragma unroll
        for (int i = 0; i < Cfg::FM; ++i)
#pragma unroll
          for (int j = 0; j < Cfg::FN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i][s], b[j][s], acc[i][j], 0, 0, 0);
      if (more) {
        al.store(ldsA[cur ^ 1], tid);
        bl.store(ldsB[cur ^ 1], tid);
      }
      __syncthreads();
    }
  }

  // Visits every accumulator element: f(row, col, value) with row/col local
  // to the workgroup tile.
  template <class F>
  __device__ static inline void for_each(const f32x16 (&acc)[Cfg::FM][Cfg::FN], F&& f) {
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave / Cfg::WN, wn = wave % Cfg::WN;
    const int col = lane & 31, h = lane >> 5;
#pragma unroll
    for (int i = 0; i < Cfg::FM; ++i)
#pragma unroll
      for (int j = 0; j < Cfg::FN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int row = wm * Cfg::WTM + i * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
          f(row, wn * Cfg::WTN + j * 32 + col, acc[i][j][r]);
        }
  }
};

}  // namespace tnh
