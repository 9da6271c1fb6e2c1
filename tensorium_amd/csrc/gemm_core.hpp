// fp32 GEMM core on CDNA4 matrix cores (gfx950), shared by the plain SGEMM
// entry points and the implicit-GEMM convolutions.
//
// One workgroup computes a BM x BN tile of C with WM x WN wavefronts; each
// wave owns a (BM/WM) x (BN/WN) sub-tile made of 32x32 blocks, each
// accumulated by v_mfma_f32_32x32x2_f32.  Operands stream through LDS in BK
// deep panels (BK a multiple of 16), double buffered with one barrier per
// panel; the next panel's global loads are issued before the current panel's
// MFMAs so that their latency hides behind matrix work.
//
// Global loads are raw buffer loads: an out-of-range offset (kOOB) reads as
// 0.0 in hardware, so edge tiles, K tails and convolution padding need no
// branches.  LDS is addressed through address_space(3) pointers so that the
// compiler emits ds_read/ds_write (a generic pointer would become flat_*
// accesses, which share the vector-memory counter with the prefetch and
// serialize it).
//
// MFMA operand layout of v_mfma_f32_32x32x2_f32 (one 32x32x2 block):
//   A: lane l supplies A[m = l%32][kk = l/32]
//   B: lane l supplies B[kk = l/32][n = l%32]
//   D: lane l, register r holds D[m = 8*(r/4) + 4*(l/32) + r%4][n = l%32]
// Within each 16-deep chunk of a panel, MFMA step s (0..7) pairs k = s
// (lanes 0-31) with k = 8 + s (lanes 32-63), so a lane's eight A values of a
// chunk are 8 contiguous k and come from a k-contiguous LDS tile with two
// 16-byte reads.  The sum over k is unchanged; only the fp32 accumulation
// order differs from the reference's sequential chain (covered by the 1e-5
// per-tensor tolerance; exact for integer-valued data).
//
// Operand tiles live in LDS in one of two layouts, chosen so that the
// global->LDS copy never transposes:
//   KC ("k contiguous"):   tile[row][BK + 4]   (A normal, B transposed)
//   MC ("row contiguous"): tile[BK][ROWS + 4]  (A transposed, B normal,
//                                               implicit im2col gathers)
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>
#include <type_traits>

namespace tnh {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) float lds_t;
typedef __attribute__((address_space(3))) f32x4 lds_f4;

constexpr int kPad = 4;                 // LDS row padding (floats)
constexpr uint32_t kOOB = 0x80000000u;  // buffer offset beyond every range: reads 0
constexpr int64_t kMaxBufBytes = 0x7FFFFFF0;  // largest operand a buffer resource spans

template <int BM_, int BN_, int BK_, int WM_, int WN_, int PF_ = 2, int OCC_ = 1>
struct TileCfg {
  static constexpr int BM = BM_, BN = BN_, BK = BK_, WM = WM_, WN = WN_;
  static constexpr int PF = PF_;    // prefetch depth in panels (1 or 2)
  static constexpr int OCC = OCC_;  // minimum waves per SIMD asked of the register allocator
  static constexpr int NWAVES = WM * WN;
  static constexpr int NT = NWAVES * 64;
  static constexpr int WTM = BM / WM, WTN = BN / WN;  // wave tile
  static constexpr int FM = WTM / 32, FN = WTN / 32;  // 32x32 blocks per wave
  static constexpr int KCH = BK / 16;                 // 16-deep chunks per panel
  static_assert(FM >= 1 && FN >= 1 && WTM % 32 == 0 && WTN % 32 == 0 && BK % 16 == 0, "tile");
};

// ---------------------------------------------------------------------------
// buffer resources
// ---------------------------------------------------------------------------
__device__ inline __amdgpu_buffer_rsrc_t make_rsrc(const float* p, int64_t bytes) {
  const int n = static_cast<int>(bytes < kMaxBufBytes ? bytes : kMaxBufBytes);
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(p), 0, n, 0x00020000);
}
// `off` when `ok`, else kOOB (the load reads 0).  The selected offset passes
// through an empty asm statement: without it the compiler pushes the select
// into the buffer load and splits the load into two divergent branches, whose
// join then waits for every outstanding load (s_waitcnt vmcnt(0)) in the
// middle of the prefetch.
__device__ inline uint32_t sel_off(bool ok, uint32_t off) {
  uint32_t r = ok ? off : kOOB;
  asm("" : "+v"(r));
  return r;
}

__device__ inline float buf_ld1(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
}
__device__ inline f32x4 buf_ld4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}
// Loads with a per-lane offset `voff` plus a wave-uniform offset `soff` (an
// SGPR operand of the instruction).  Callers keep every valid voff + soff
// inside the buffer and give invalid lanes voff = kOOB, so the result does
// not depend on whether the hardware range check includes soff.
__device__ inline float buf_ld1s(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0));
}
__device__ inline f32x4 buf_ld4s(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}

// ---------------------------------------------------------------------------
// LDS panels
// ---------------------------------------------------------------------------
template <bool KC, int ROWS, int BK>
struct PanelLayout {
  static constexpr int PITCH = KC ? (BK + kPad) : (ROWS + kPad);
  static constexpr int SIZE = KC ? ROWS * PITCH : BK * PITCH;
  __device__ static inline int at(int row, int k) { return KC ? row * PITCH + k : k * PITCH + row; }
};

// The eight per-step operand values of chunk `ch` of one 32-row block.
template <bool KC, int ROWS, int BK>
__device__ inline void read_frag(const lds_t* lds, int row0, int ch, int lane, float (&v)[8]) {
  using L = PanelLayout<KC, ROWS, BK>;
  const int r = lane & 31, h = lane >> 5;
  if constexpr (KC) {
    const lds_f4* p = reinterpret_cast<const lds_f4*>(lds + L::at(row0 + r, ch * 16 + h * 8));
    const f32x4 a = p[0], b = p[1];
    v[0] = a[0]; v[1] = a[1]; v[2] = a[2]; v[3] = a[3];
    v[4] = b[0]; v[5] = b[1]; v[6] = b[2]; v[7] = b[3];
  } else {
#pragma unroll
    for (int s = 0; s < 8; ++s) v[s] = lds[L::at(row0 + r, ch * 16 + h * 8 + s)];
  }
}

// ---------------------------------------------------------------------------
// Operand loaders.  A loader is bound to one tile (init) and then fetches
// K panels into registers (load(k0)) and writes them to an LDS panel
// (store).  Offsets are 32-bit byte offsets into a buffer resource whose
// range is at most 2 GiB; per-element work is one add and one select (an
// invalid element gets kOOB through sel_off, which the hardware returns as
// 0).
// ---------------------------------------------------------------------------

// Dense operand.  Element (row, k) of op(X):
//   KC (k contiguous in memory):   X[(row0+row)*ld + k]
//   MC (row contiguous in memory): X[k*ld + row0 + row]
// VEC: 16-byte loads (the host guarantees 16-byte alignment, ld % 4 == 0 and
// contiguous extent % 4 == 0, so a vector is entirely in or out of range).
template <bool KC, bool VEC, int ROWS, int BK, int NT>
struct DenseLoader {
  static constexpr bool kKC = KC;
  static constexpr int ELEMS = ROWS * BK;
  static constexpr int UNITS = VEC ? ELEMS / 4 : ELEMS;
  static constexpr int PER = (UNITS + NT - 1) / NT;  // loads per thread
  static constexpr bool kPartial = UNITS % NT != 0;
  using Reg = typename std::conditional<VEC, f32x4, float>::type;

  __amdgpu_buffer_rsrc_t rsrc;
  uint32_t off0[PER];   // byte offset of this thread's element v at k0 = 0
  uint32_t kStep;       // byte offset per unit of k
  int kIdx[PER];        // k of element v within the panel
  bool rowOk[PER];
  int K;
  Reg reg[PER];

  __device__ static inline void coords(int idx, int& row, int& k) {
    if constexpr (KC) {
      constexpr int PR = VEC ? BK / 4 : BK;
      row = idx / PR;
      k = (idx % PR) * (VEC ? 4 : 1);
    } else {
      constexpr int PR = VEC ? ROWS / 4 : ROWS;
      k = idx / PR;
      row = (idx % PR) * (VEC ? 4 : 1);
    }
  }

  __device__ inline void init(const float* base, int64_t bytes, int64_t ld, int64_t rows, int64_t K_, int64_t row0,
                              int tid) {
    rsrc = make_rsrc(base, bytes);
    K = static_cast<int>(K_);
    kStep = KC ? 4u : static_cast<uint32_t>(ld * 4);
#pragma unroll
    for (int v = 0; v < PER; ++v) {
      const int idx = tid + v * NT;
      int row, k;
      coords(idx, row, k);
      const int64_t gr = row0 + row;
      rowOk[v] = gr < rows && (!kPartial || idx < UNITS);
      kIdx[v] = k;
      off0[v] = static_cast<uint32_t>(KC ? (gr * ld + k) * 4 : (k * ld + gr) * 4);
    }
  }

  __device__ inline void load(int64_t k0) {
    const uint32_t koff = static_cast<uint32_t>(k0) * kStep;
#pragma unroll
    for (int v = 0; v < PER; ++v) {
      const bool ok = rowOk[v] && static_cast<int>(k0) + kIdx[v] < K;
      const uint32_t off = sel_off(ok, off0[v] + koff);
      if constexpr (VEC)
        reg[v] = buf_ld4(rsrc, off);
      else
        reg[v] = buf_ld1(rsrc, off);
    }
  }

  __device__ inline void store(lds_t* lds, int tid) const {
    using L = PanelLayout<KC, ROWS, BK>;
#pragma unroll
    for (int v = 0; v < PER; ++v) {
      const int idx = tid + v * NT;
      if (kPartial && idx >= UNITS) break;
      int row, k;
      coords(idx, row, k);
      if constexpr (VEC)
        *reinterpret_cast<lds_f4*>(lds + L::at(row, k)) = reg[v];
      else
        lds[L::at(row, k)] = reg[v];
    }
  }
};

// ---------------------------------------------------------------------------
// Convolution B operands (MC layout, batch merged into N):
//   column n = b*OH*OW + oy*OW + ox
// Each thread owns one column for the whole K loop and BK*BN/NT rows of each
// panel (rows myRow0 + v*RSTEP).
// ---------------------------------------------------------------------------
struct ConvGeom {
  const float* x;
  int64_t xBytes;        // extent of x addressed by the gathers
  int64_t xBatchStride;  // floats
  int C, H, W, OW, OHW;
  int sY, sX, pH, pW;
  int64_t N, K;
  int kh, kw;  // kernel size (read by the run-time-size gather)
  int tapW;    // the run-time-size gather: weights tap-major (1) or [F][C][kh][kw] (0)
};

template <int BN, int BK, int NT>
struct ColumnState {
  static constexpr int RSTEP = NT / BN;
  static constexpr int PER = BK * BN / NT;
  static_assert(NT % BN == 0 && PER >= 1 && BK % RSTEP == 0, "column split");
  uint32_t colOff;  // byte offset of image b at (iy0, ix0), modulo 2^32 (may wrap)
  int iy0, ix0;
  bool colOk;
  int myCol, myRow0;

  __device__ inline void init_col(const ConvGeom& g, int64_t n0, int tid) {
    myCol = tid % BN;
    myRow0 = tid / BN;
    const int64_t n = n0 + myCol;
    colOk = n < g.N;
    const int64_t nn = colOk ? n : 0;
    const int64_t b = nn / g.OHW;
    const int p = static_cast<int>(nn - b * g.OHW);
    const int oy = p / g.OW, ox = p - (p / g.OW) * g.OW;
    iy0 = oy * g.sY - g.pH;
    ix0 = ox * g.sX - g.pW;
    colOff = static_cast<uint32_t>((b * g.xBatchStride + static_cast<int64_t>(iy0) * g.W + ix0) * 4);
  }
};

// General gather, any C.  TAP = false: the reference K order
// k = (c*KH + ky)*KW + kx (sim2Col, ntensors.pas:11425-11463) for weights as
// the reference stores them ([F][C][kh][kw]); TAP = true: tap-major order
// k = (ky*KW + kx)*C + c for packed weights.
template <int KH, int KW, int BN, int BK, int NT, bool TAP = false>
struct ConvGatherLoader : ColumnState<BN, BK, NT> {
  using S = ColumnState<BN, BK, NT>;
  static constexpr bool kKC = false;
  __amdgpu_buffer_rsrc_t rsrc;
  int C, H, W, K;
  uint32_t HW4;
  float reg[S::PER];

  __device__ inline void init(const ConvGeom& g, int64_t n0, int tid) {
    rsrc = make_rsrc(g.x, g.xBytes);
    C = g.C;
    H = g.H;
    W = g.W;
    K = static_cast<int>(g.K);
    HW4 = static_cast<uint32_t>(g.H) * static_cast<uint32_t>(g.W) * 4u;
    S::init_col(g, n0, tid);
  }

  __device__ inline void load(int64_t k0) {
#pragma unroll
    for (int v = 0; v < S::PER; ++v) {
      const int k = static_cast<int>(k0) + S::myRow0 + v * S::RSTEP;
      int c, r;
      if constexpr (TAP) {
        r = k / C;
        c = k - r * C;
      } else {
        c = k / (KH * KW);
        r = k - c * (KH * KW);
      }
      const int ky = r / KW, kx = r - (r / KW) * KW;
      const int iy = S::iy0 + ky, ix = S::ix0 + kx;
      const bool ok = S::colOk && k < K && static_cast<unsigned>(iy) < static_cast<unsigned>(H) &&
                      static_cast<unsigned>(ix) < static_cast<unsigned>(W);
      const uint32_t o = S::colOff + static_cast<uint32_t>(c) * HW4 + static_cast<uint32_t>(ky * W + kx) * 4u;
      reg[v] = buf_ld1(rsrc, sel_off(ok, o));
    }
  }

  __device__ inline void store(lds_t* lds, int) const {
    using L = PanelLayout<false, BN, BK>;
#pragma unroll
    for (int v = 0; v < S::PER; ++v) lds[L::at(S::myCol, S::myRow0 + v * S::RSTEP)] = reg[v];
  }
};

template <int KH, int KW, int BN, int BK, int NT>
using ConvGatherTapLoader = ConvGatherLoader<KH, KW, BN, BK, NT, true>;

// The same gather for a kernel size known only at run time (any kh x kw:
// 5x5, 7x7, 1x3, ... layers), in either K order (g.tapW).  Two integer
// divisions per element more than the compile-time loaders; for the rare
// layer shapes those do not cover.
template <int BN, int BK, int NT>
struct ConvGatherDynLoader : ColumnState<BN, BK, NT> {
  using S = ColumnState<BN, BK, NT>;
  static constexpr bool kKC = false;
  __amdgpu_buffer_rsrc_t rsrc;
  int C, H, W, K, KW, KHW;
  bool tap;
  uint32_t HW4;
  float reg[S::PER];

  __device__ inline void init(const ConvGeom& g, int64_t n0, int tid) {
    rsrc = make_rsrc(g.x, g.xBytes);
    C = g.C;
    H = g.H;
    W = g.W;
    K = static_cast<int>(g.K);
    KW = g.kw;
    KHW = g.kh * g.kw;
    tap = g.tapW != 0;
    HW4 = static_cast<uint32_t>(g.H) * static_cast<uint32_t>(g.W) * 4u;
    S::init_col(g, n0, tid);
  }

  __device__ inline void load(int64_t k0) {
#pragma unroll
    for (int v = 0; v < S::PER; ++v) {
      const int k = static_cast<int>(k0) + S::myRow0 + v * S::RSTEP;
      int c, r;
      if (tap) {
        r = k / C;
        c = k - r * C;
      } else {
        c = k / KHW;
        r = k - c * KHW;
      }
      const int ky = r / KW, kx = r - ky * KW;
      const int iy = S::iy0 + ky, ix = S::ix0 + kx;
      const bool ok = S::colOk && k < K && static_cast<unsigned>(iy) < static_cast<unsigned>(H) &&
                      static_cast<unsigned>(ix) < static_cast<unsigned>(W);
      const uint32_t o = S::colOff + static_cast<uint32_t>(c) * HW4 + static_cast<uint32_t>(ky * W + kx) * 4u;
      reg[v] = buf_ld1(rsrc, sel_off(ok, o));
    }
  }

  __device__ inline void store(lds_t* lds, int) const {
    using L = PanelLayout<false, BN, BK>;
#pragma unroll
    for (int v = 0; v < S::PER; ++v) lds[L::at(S::myCol, S::myRow0 + v * S::RSTEP)] = reg[v];
  }
};

// Tap-major K order k = (ky*KW + kx)*C + c, weights packed [F][kh][kw][C]
// (tnh_conv2d_pack_weights).  With C % BK == 0 a panel lies inside one tap,
// so the tap, its bounds test and the base offset are computed once per
// panel and each element is one add.
template <int KW, int BN, int BK, int NT>
struct ConvTapLoader : ColumnState<BN, BK, NT> {
  using S = ColumnState<BN, BK, NT>;
  static constexpr bool kKC = false;
  __amdgpu_buffer_rsrc_t rsrc;
  int C, H, W;
  uint32_t HW4, rowOff, vStride;
  float reg[S::PER];

  __device__ inline void init(const ConvGeom& g, int64_t n0, int tid) {
    rsrc = make_rsrc(g.x, g.xBytes);
    C = g.C;
    H = g.H;
    W = g.W;
    HW4 = static_cast<uint32_t>(g.H) * static_cast<uint32_t>(g.W) * 4u;
    S::init_col(g, n0, tid);
    rowOff = S::colOff + static_cast<uint32_t>(S::myRow0) * HW4;
    vStride = static_cast<uint32_t>(S::RSTEP) * HW4;
  }

  __device__ inline void load(int64_t k0) {
    const int kk = static_cast<int>(k0);
    const int tap = kk / C;  // uniform over the workgroup
    const int c0 = kk - tap * C;
    const int ky = tap / KW, kx = tap - (tap / KW) * KW;
    const int iy = S::iy0 + ky, ix = S::ix0 + kx;
    const bool ok = S::colOk && static_cast<unsigned>(iy) < static_cast<unsigned>(H) &&
                    static_cast<unsigned>(ix) < static_cast<unsigned>(W);
    const uint32_t base = rowOff + static_cast<uint32_t>(c0) * HW4 + static_cast<uint32_t>(ky * W + kx) * 4u;
#pragma unroll
    for (int v = 0; v < S::PER; ++v) reg[v] = buf_ld1(rsrc, sel_off(ok, base + v * vStride));
  }

  __device__ inline void store(lds_t* lds, int) const {
    using L = PanelLayout<false, BN, BK>;
#pragma unroll
    for (int v = 0; v < S::PER; ++v) lds[L::at(S::myCol, S::myRow0 + v * S::RSTEP)] = reg[v];
  }
};

// Quad-vectorised variants: the B panel is stored k-contiguous (KC,
// [BN][BK+4], the layout of A) and each thread gathers 4 consecutive k of
// one column, written with one 16-byte LDS store; fragments are then read
// with 16-byte LDS reads.  Thread t owns column t % BN and k-quads
// t / BN + j*(NT/BN).
template <int BN, int BK, int NT>
struct QuadColumnState {
  static constexpr int QSTEP = NT / BN;           // quads between a thread's quads
  static constexpr int NQ = (BK / 4) / QSTEP;     // quads per thread per panel
  static_assert(NT % BN == 0 && NQ >= 1 && (BK / 4) % QSTEP == 0, "quad split");
  int myCol, myQ0;
};

// tap-major K (packed weights), C % BK == 0
template <int KW, int BN, int BK, int NT>
struct ConvTapQuadLoader : ColumnState<BN, BK, NT> {
  using S = ColumnState<BN, BK, NT>;
  using Q = QuadColumnState<BN, BK, NT>;
  static constexpr bool kKC = true;
  __amdgpu_buffer_rsrc_t rsrc;
  int C, H, W;
  uint32_t HW4, qOff, qStride;
  int myQ0;
  float reg[Q::NQ][4];

  __device__ inline void init(const ConvGeom& g, int64_t n0, int tid) {
    rsrc = make_rsrc(g.x, g.xBytes);
    C = g.C;
    H = g.H;
    W = g.W;
    HW4 = static_cast<uint32_t>(g.H) * static_cast<uint32_t>(g.W) * 4u;
    S::init_col(g, n0, tid);  // column tid % BN
    myQ0 = tid / BN;
    qOff = S::colOff + static_cast<uint32_t>(myQ0 * 4) * HW4;
    qStride = static_cast<uint32_t>(Q::QSTEP * 4) * HW4;
  }

  __device__ inline void load(int64_t k0) {
    const int kk = static_cast<int>(k0);
    const int tap = kk / C;
    const int c0 = kk - tap * C;
    const int ky = tap / KW, kx = tap - (tap / KW) * KW;
    const int iy = S::iy0 + ky, ix = S::ix0 + kx;
    const bool ok = S::colOk && static_cast<unsigned>(iy) < static_cast<unsigned>(H) &&
                    static_cast<unsigned>(ix) < static_cast<unsigned>(W);
    const uint32_t base = qOff + static_cast<uint32_t>(c0) * HW4 + static_cast<uint32_t>(ky * W + kx) * 4u;
#pragma unroll
    for (int q = 0; q < Q::NQ; ++q)
#pragma unroll
      for (int e = 0; e < 4; ++e) reg[q][e] = buf_ld1(rsrc, sel_off(ok, base + q * qStride + e * HW4));
  }

  __device__ inline void store(lds_t* lds, int) const {
    using L = PanelLayout<true, BN, BK>;
#pragma unroll
    for (int q = 0; q < Q::NQ; ++q)
      *reinterpret_cast<lds_f4*>(lds + L::at(S::myCol, (myQ0 + q * Q::QSTEP) * 4)) =
          f32x4{reg[q][0], reg[q][1], reg[q][2], reg[q][3]};
  }
};

// 1x1 stride-1: B[k = c][n] with 4 consecutive channels per thread
template <int BN, int BK, int NT>
struct Conv1x1QuadLoader {
  using Q = QuadColumnState<BN, BK, NT>;
  static constexpr bool kKC = true;
  __amdgpu_buffer_rsrc_t rsrc;
  uint32_t qOff, HW4, qStride;
  int K;
  bool colOk;
  int myCol, myQ0;
  float reg[Q::NQ][4];

  __device__ inline void init(const ConvGeom& g, int64_t n0, int tid) {
    rsrc = make_rsrc(g.x, g.xBytes);
    const int64_t HW = g.OHW;
    HW4 = static_cast<uint32_t>(HW) * 4u;
    K = static_cast<int>(g.K);
    myCol = tid % BN;
    myQ0 = tid / BN;
    const int64_t n = n0 + myCol;
    colOk = n < g.N;
    const int64_t nn = colOk ? n : 0;
    const int64_t b = nn / HW;
    qOff = static_cast<uint32_t>((b * g.xBatchStride + (nn - b * HW) + static_cast<int64_t>(myQ0 * 4) * HW) * 4);
    qStride = static_cast<uint32_t>(Q::QSTEP * 4) * HW4;
  }

  __device__ inline void load(int64_t k0) {
    const uint32_t base = qOff + static_cast<uint32_t>(k0) * HW4;
#pragma unroll
    for (int q = 0; q < Q::NQ; ++q)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const bool ok = colOk && static_cast<int>(k0) + (myQ0 + q * Q::QSTEP) * 4 + e < K;
        reg[q][e] = buf_ld1(rsrc, sel_off(ok, base + q * qStride + e * HW4));
      }
  }

  __device__ inline void store(lds_t* lds, int) const {
    using L = PanelLayout<true, BN, BK>;
#pragma unroll
    for (int q = 0; q < Q::NQ; ++q)
      *reinterpret_cast<lds_f4*>(lds + L::at(myCol, (myQ0 + q * Q::QSTEP) * 4)) =
          f32x4{reg[q][0], reg[q][1], reg[q][2], reg[q][3]};
  }
};

// 1x1 stride-1 convolution: B[k = c][n = b*HW + p] = x_b[c][p].  VEC loads 4
// consecutive columns (HW % 4 == 0, xBatchStride % 4 == 0, x aligned).
template <bool VEC, int BN, int BK, int NT>
struct Conv1x1Loader {
  static constexpr bool kKC = false;
  static constexpr int CPT = VEC ? 4 : 1;  // columns per load
  static constexpr int TPR = BN / CPT;     // threads per k row
  static constexpr int RSTEP = NT / TPR;
  static constexpr int PER = BK / RSTEP;
  static_assert(NT % TPR == 0 && PER >= 1 && BK % RSTEP == 0, "1x1 split");
  using Reg = typename std::conditional<VEC, f32x4, float>::type;

  __amdgpu_buffer_rsrc_t rsrc;
  uint32_t rowOff, HW4;
  int K;
  bool colOk;
  int myCol, myRow0;
  Reg reg[PER];

  __device__ inline void init(const ConvGeom& g, int64_t n0, int tid) {
    rsrc = make_rsrc(g.x, g.xBytes);
    const int64_t HW = g.OHW;
    HW4 = static_cast<uint32_t>(HW) * 4u;
    K = static_cast<int>(g.K);
    myCol = (tid % TPR) * CPT;
    myRow0 = tid / TPR;
    const int64_t n = n0 + myCol;
    colOk = n < g.N;
    const int64_t nn = colOk ? n : 0;
    const int64_t b = nn / HW;
    rowOff = static_cast<uint32_t>((b * g.xBatchStride + (nn - b * HW) + static_cast<int64_t>(myRow0) * HW) * 4);
  }

  __device__ inline void load(int64_t k0) {
    const uint32_t base = rowOff + static_cast<uint32_t>(k0) * HW4;
#pragma unroll
    for (int v = 0; v < PER; ++v) {
      const bool ok = colOk && static_cast<int>(k0) + myRow0 + v * RSTEP < K;
      const uint32_t off = sel_off(ok, base + static_cast<uint32_t>(v * RSTEP) * HW4);
      if constexpr (VEC)
        reg[v] = buf_ld4(rsrc, off);
      else
        reg[v] = buf_ld1(rsrc, off);
    }
  }

  __device__ inline void store(lds_t* lds, int) const {
    using L = PanelLayout<false, BN, BK>;
#pragma unroll
    for (int v = 0; v < PER; ++v) {
      if constexpr (VEC)
        *reinterpret_cast<lds_f4*>(lds + L::at(myCol, myRow0 + v * RSTEP)) = reg[v];
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
// Workgroup id -> the id of the block of work it takes, such that the
// workgroups one XCD runs (ids x, x + 8, x + 16, ...: the dispatcher deals
// workgroups round-robin over the 8 XCDs, each with its own L2) take one
// contiguous range of blocks.  A bijection on [0, total) for any total.
__device__ inline int xcd_block(int pid, int total) {
  constexpr int XCD = 8;
  const int q = total / XCD, r = total % XCD, x = pid % XCD;
  return x * q + min(x, r) + pid / XCD;
}

__device__ inline void tile_coords(int pid, int tilesM, int tilesN, int& tm, int& tn) {
  const int total = tilesM * tilesN;
  pid = xcd_block(pid, total);
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
// The main loop over K panels [kBegin, kEnd) (kBegin a multiple of BK).
// PF = 1: one panel of register prefetch; PF = 2: two (run2).
// ---------------------------------------------------------------------------
template <class Cfg, class AL, class BL>
struct GemmMainloop {
  using LA = PanelLayout<AL::kKC, Cfg::BM, Cfg::BK>;
  using LB = PanelLayout<BL::kKC, Cfg::BN, Cfg::BK>;
  static constexpr int STAGE = LA::SIZE + LB::SIZE;
  static constexpr int LDS_FLOATS = 2 * STAGE;

  // Dispatches on the configuration's prefetch depth; al/bl are bound to the
  // tile (init) already.
  __device__ static inline void exec(AL& al, BL& bl, int64_t kBegin, int64_t kEnd, lds_t* lds,
                                     f32x16 (&acc)[Cfg::FM][Cfg::FN]) {
    if constexpr (Cfg::PF == 2) {
      AL al1 = al;
      BL bl1 = bl;
      run2(al, bl, al1, bl1, kBegin, kEnd, lds, acc);
    } else {
      run(al, bl, kBegin, kEnd, lds, acc);
    }
  }

  __device__ static inline void run(AL& al, BL& bl, int64_t kBegin, int64_t kEnd, lds_t* lds,
                                    f32x16 (&acc)[Cfg::FM][Cfg::FN]) {
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave / Cfg::WN, wn = wave % Cfg::WN;

#pragma unroll
    for (int i = 0; i < Cfg::FM; ++i)
#pragma unroll
      for (int j = 0; j < Cfg::FN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    const int64_t nk = (kEnd - kBegin + Cfg::BK - 1) / Cfg::BK;
    if (nk <= 0) return;
    al.load(kBegin);
    bl.load(kBegin);
    al.store(lds, tid);
    bl.store(lds + LA::SIZE, tid);
    __syncthreads();

    for (int64_t kt = 0; kt < nk; ++kt) {
      lds_t* cur = lds + (kt & 1) * STAGE;
      lds_t* nxt = lds + ((kt + 1) & 1) * STAGE;
      const bool more = kt + 1 < nk;
      if (more) {
        al.load(kBegin + (kt + 1) * Cfg::BK);
        bl.load(kBegin + (kt + 1) * Cfg::BK);
      }
#pragma unroll
      for (int ch = 0; ch < Cfg::KCH; ++ch) {
        float a[Cfg::FM][8], b[Cfg::FN][8];
#pragma unroll
        for (int i = 0; i < Cfg::FM; ++i)
          read_frag<AL::kKC, Cfg::BM, Cfg::BK>(cur, wm * Cfg::WTM + i * 32, ch, lane, a[i]);
#pragma unroll
        for (int j = 0; j < Cfg::FN; ++j)
          read_frag<BL::kKC, Cfg::BN, Cfg::BK>(cur + LA::SIZE, wn * Cfg::WTN + j * 32, ch, lane, b[j]);
#pragma unroll
        for (int s = 0; s < 8; ++s)
#pragma unroll
          for (int i = 0; i < Cfg::FM; ++i)
#pragma unroll
            for (int j = 0; j < Cfg::FN; ++j)
              acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i][s], b[j][s], acc[i][j], 0, 0, 0);
      }
      if (more) {
        al.store(nxt, tid);
        bl.store(nxt + LA::SIZE, tid);
      }
      __syncthreads();
    }
  }

  // Two-deep prefetch: panel kt+2 is loaded into registers while panel kt is
  // multiplied and panel kt+1 (loaded one iteration earlier) is written to
  // LDS, so a global load has two iterations of MFMA work to land.  The two
  // loader copies hold the two register sets; all fragments of a chunk are
  // read before its MFMAs.
  __device__ static inline void run2(AL& al0, BL& bl0, AL& al1, BL& bl1, int64_t kBegin, int64_t kEnd, lds_t* lds,
                                     f32x16 (&acc)[Cfg::FM][Cfg::FN]) {
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave / Cfg::WN, wn = wave % Cfg::WN;

#pragma unroll
    for (int i = 0; i < Cfg::FM; ++i)
#pragma unroll
      for (int j = 0; j < Cfg::FN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    const int64_t nk = (kEnd - kBegin + Cfg::BK - 1) / Cfg::BK;
    if (nk <= 0) return;
    al0.load(kBegin);
    bl0.load(kBegin);
    if (nk > 1) {
      al1.load(kBegin + Cfg::BK);
      bl1.load(kBegin + Cfg::BK);
    }
    al0.store(lds, tid);
    bl0.store(lds + LA::SIZE, tid);
    __syncthreads();

    auto step = [&](int64_t kt, AL& alNext, BL& blNext, AL& alFree, BL& blFree) {
      lds_t* cur = lds + (kt & 1) * STAGE;
      lds_t* nxt = lds + ((kt + 1) & 1) * STAGE;
      if (kt + 2 < nk) {
        alFree.load(kBegin + (kt + 2) * Cfg::BK);
        blFree.load(kBegin + (kt + 2) * Cfg::BK);
      }
#pragma unroll
      for (int ch = 0; ch < Cfg::KCH; ++ch) {
        float a[Cfg::FM][8], b[Cfg::FN][8];
#pragma unroll
        for (int i = 0; i < Cfg::FM; ++i)
          read_frag<AL::kKC, Cfg::BM, Cfg::BK>(cur, wm * Cfg::WTM + i * 32, ch, lane, a[i]);
#pragma unroll
        for (int j = 0; j < Cfg::FN; ++j)
          read_frag<BL::kKC, Cfg::BN, Cfg::BK>(cur + LA::SIZE, wn * Cfg::WTN + j * 32, ch, lane, b[j]);
#pragma unroll
        for (int s = 0; s < 8; ++s)
#pragma unroll
          for (int i = 0; i < Cfg::FM; ++i)
#pragma unroll
            for (int j = 0; j < Cfg::FN; ++j)
              acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i][s], b[j][s], acc[i][j], 0, 0, 0);
      }
      if (kt + 1 < nk) {
        alNext.store(nxt, tid);
        blNext.store(nxt + LA::SIZE, tid);
      }
      __syncthreads();
    };
    for (int64_t kt = 0; kt < nk; kt += 2) {
      step(kt, al1, bl1, al0, bl0);          // panel kt+1 is in set 1; set 0 is free
      if (kt + 1 < nk) step(kt + 1, al0, bl0, al1, bl1);
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
