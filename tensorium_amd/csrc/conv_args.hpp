// Arguments and the shared epilogue of the fused convolution kernels
// (conv.hip, conv_lean.hpp).
//
// Epilogue per element, in the reference order (nConvolutionLayer.pas:508-545
// then the shortcut add of naddlayer.pas:698):
//   v = acc + bias[f];  v = act(v);  v = v + residual.
#pragma once
#include "common.hpp"
#include "gemm_core.hpp"
#include "yolo_math.hpp"

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
  int64_t outBytes; // extent of out addressed by the kernel
  int64_t resBytes; // extent of res addressed by the kernel (0 without residual)
  // Tail split (lean kernels; splits == 1): workgroups [0, nFull) own the
  // whole K range of tiles [0, nFull); the remaining tiles are cut into
  // tailSplits K pieces of kChunk each, one workgroup per piece, whose raw
  // accumulators go to part (one BM x BN block per piece, tile-major) for
  // conv_tail_reduce.  tailSplits == 0: off.
  int tailSplits;
  int nFull;
  int tailUnit;  // host only: tiles per whole round (the CU count, or CUs x resident workgroups)
  // One arrival counter per tail tile (zero between launches), or nullptr.
  // With counters the workgroup that stores a tail tile's last piece sums
  // the tile's pieces and runs the epilogue itself; without them a second
  // launch (conv_tail_reduce) does.
  int* tileCount;
  // Channels-last (NHWC) tensors: floats between consecutive pixels of x, out
  // and res (the channel count of the buffer a tensor lives in, so a tensor
  // can be a channel slice of a wider one); images are H*W*pixel-stride apart.
  int xPix, outPix, resPix;
  // Channels-last epilogue variants (0 / nullptr: off):
  //   upS > 0: the result is written only as its nearest-upsampled image, the
  //     output of the TUpSampleLayer that follows (nupsamplelayer.pas:83-146):
  //     pixel (b, y, x) goes to pixels (b, upS*y + dy, upS*x + dx) of out
  //     (pixel stride outPix), times upScale;
  //   yolo: the result is also written through TYoloLayer.forward's transform
  //     (nyololayer.pas:786-830) to the NCHW head yolo[b][f][y][x]
  //     (yoloEntries = 5 + classes channels per anchor).
  int upS;
  float upScale;
  float* yolo;
  int yoloEntries;
  // yolo head extent in bytes when it lies within 2 GiB (0: per-element
  // stores), and whether 4 consecutive pixels of one channel are one aligned
  // 16-byte vector there (OH*OW % 4 == 0, 16-byte aligned head)
  int64_t yoloBytes;
  int yoloVec;
  // few-channel NCHW kernel: filters per grid.y group (a multiple of 4)
  int64_t fGroup;
};

// K walk / B operand of a convolution kernel
// kGatherDyn: any kernel size (kh x kw given at run time), either weight
// layout (tap-major when ConvArgs::tapW)
enum Mode {
  kGatherRef3 = 0,
  kGatherTap3 = 1,
  kGatherRef1 = 2,
  kTap3 = 3,
  k1x1 = 4,
  kGatherDyn = 5,
  kTap3Any = 6,  // channels-last 3x3 with C % 4 == 0 but C % 32 != 0 (a panel may span taps, K tail)
  k1x1Any = 7,   // channels-last 1x1 with C % 4 == 0 but C % 32 != 0 (K tail)
};

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
  // Per column: the residual values are all loaded before the first store
  // (a store may alias a later residual element), and the wave-uniform
  // activation selects straight-line code.
  auto column = [&](auto actTag, int j) {
    constexpr int ACT = decltype(actTag)::value;
    const int64_t n = n0w + j * 32 + (lane & 31);
    if (n >= a.g.N) return;
    const int64_t b = n / OHW, p = n - b * OHW;
    float* out = a.out + b * a.outBatchStride + p;
    float rv[FM][16];
    if (a.res) {
      const float* res = a.res + b * a.rBatchStride + p;
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int64_t f = m0w + i * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
          rv[i][r] = f < a.F ? res[f * OHW] : 0.f;
        }
    }
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t f = m0w + i * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
        if (f >= a.F) continue;
        float v = acc[i][j][r];
        if (a.bias) v = v + a.bias[f];
        v = apply_act(v, ACT);
        if (a.res) v = v + rv[i][r];
        out[f * OHW] = v;
      }
  };
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    if (a.act == TNH_AC_LEAKY)
      column(std::integral_constant<int, TNH_AC_LEAKY>{}, j);
    else if (a.act == TNH_AC_LOGISTIC)
      column(std::integral_constant<int, TNH_AC_LOGISTIC>{}, j);
    else
      column(std::integral_constant<int, TNH_AC_LINEAR>{}, j);
  }
}

// Output stores of the conv and GEMM epilogues: system-scope (sc0 sc1), so
// they write through the XCD's L2 as the tiles finish instead of staying
// dirty there until the end-of-kernel release writes the whole output back
// at once (measured on YOLOv3-416 batch 16: 8.81-8.82 -> 8.73 ms; device
// scope alone: 8.75).
constexpr int kStoreThrough = 17;  // buffer cache-policy bits: sc0 | sc1
__device__ inline void buf_st1s(__amdgpu_buffer_rsrc_t r, float v, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), r, voff, soff, kStoreThrough);
}

// conv_store through buffer instructions (same results): each lane's
// column part of an offset is a 32-bit per-lane value, the row part
// (block i, register r) is wave-uniform and rides in the scalar offset, and
// an element outside [0, F) x [0, N) gets the lane offset kOOB, whose store
// the hardware drops, so there are no per-element branches.  The host
// guarantees that out, res and the split-K partials each span at most 2 GiB.
template <int FM, int FN>
__device__ inline void conv_store_buf(const ConvArgs& a, const f32x16 (&acc)[FM][FN], int64_t m0w, int64_t n0w,
                                      int lane) {
  const int h = lane >> 5;
  const int F = static_cast<int>(a.F);
  const int rowBase = static_cast<int>(m0w) + 4 * h;  // row of element (i = 0, r = 0)
  const bool allRows = m0w + FM * 32 <= a.F;          // wave-uniform
  auto rowOk = [&](int c) { return allRows || rowBase + c < F; };
  if (a.splits > 1) {
    const uint32_t N = static_cast<uint32_t>(a.g.N);
    const int64_t slice = a.F * a.g.N;
    const __amdgpu_buffer_rsrc_t pr = make_rsrc(a.part + static_cast<int64_t>(blockIdx.y) * slice, slice * 4);
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int64_t n = n0w + j * 32 + (lane & 31);
      const uint32_t vo = sel_off(n < a.g.N, (static_cast<uint32_t>(rowBase) * N + static_cast<uint32_t>(n)) * 4u);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int c = i * 32 + 8 * (r >> 2) + (r & 3);
          buf_st1s(pr, acc[i][j][r], rowOk(c) ? vo : kOOB, static_cast<uint32_t>(c) * N * 4u);
        }
    }
    return;
  }
  const uint32_t OHW = static_cast<uint32_t>(a.g.OHW);
  const __amdgpu_buffer_rsrc_t outR = make_rsrc(a.out, a.outBytes);
  const __amdgpu_buffer_rsrc_t resR = make_rsrc(a.res, a.resBytes);
  // without bias the add uses -0.0, the exact additive identity (x + -0.0
  // == x for every x, signed zeros included), so it needs no branch
  float bias[FM][16];
  if (a.bias) {
    const __amdgpu_buffer_rsrc_t bR = make_rsrc(a.bias, a.F * 4);
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        bias[i][r] = buf_ld1s(bR, static_cast<uint32_t>(rowBase) * 4u,
                              static_cast<uint32_t>(i * 32 + 8 * (r >> 2) + (r & 3)) * 4u);
  } else {
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) bias[i][r] = -0.f;
  }
  uint32_t vOut[FN], vRes[FN];
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    const int64_t n = n0w + j * 32 + (lane & 31);
    const bool okN = n < a.g.N;
    const uint32_t nn = okN ? static_cast<uint32_t>(n) : 0u;
    const uint32_t b = nn / OHW, p = nn - b * OHW;
    const uint32_t rowOff = static_cast<uint32_t>(rowBase) * OHW + p;
    vOut[j] = sel_off(okN, (b * static_cast<uint32_t>(a.outBatchStride) + rowOff) * 4u);
    vRes[j] = sel_off(okN, (b * static_cast<uint32_t>(a.rBatchStride) + rowOff) * 4u);
  }
  auto so = [&](int i, int r) { return static_cast<uint32_t>(i * 32 + 8 * (r >> 2) + (r & 3)) * OHW * 4u; };
  // The activation and the residual are wave-uniform: each combination gets
  // its own straight-line code, and every residual load is issued before the
  // first store (a store may alias a later residual element, so interleaved
  // loads would each wait for a full memory round trip).
  auto finish = [&](auto actTag, auto resTag) {
    constexpr int ACT = decltype(actTag)::value;
    constexpr bool RES = decltype(resTag)::value;
    float rv[FN][FM][16];
    if constexpr (RES) {
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int r = 0; r < 16; ++r) rv[j][i][r] = buf_ld1s(resR, vRes[j], so(i, r));
    }
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int c = i * 32 + 8 * (r >> 2) + (r & 3);
          float v = apply_act(acc[i][j][r] + bias[i][r], ACT);
          if constexpr (RES) v = v + rv[j][i][r];
          buf_st1s(outR, v, rowOk(c) ? vOut[j] : kOOB, so(i, r));
        }
  };
  using Leaky = std::integral_constant<int, TNH_AC_LEAKY>;
  using Logistic = std::integral_constant<int, TNH_AC_LOGISTIC>;
  using Linear = std::integral_constant<int, TNH_AC_LINEAR>;
  if (a.res) {
    if (a.act == TNH_AC_LEAKY)
      finish(Leaky{}, std::true_type{});
    else if (a.act == TNH_AC_LOGISTIC)
      finish(Logistic{}, std::true_type{});
    else
      finish(Linear{}, std::true_type{});
  } else {
    if (a.act == TNH_AC_LEAKY)
      finish(Leaky{}, std::false_type{});
    else if (a.act == TNH_AC_LOGISTIC)
      finish(Logistic{}, std::false_type{});
    else
      finish(Linear{}, std::false_type{});
  }
}

// One finished result v of output pixel m, filter f (both in range) under
// the epilogue variants a.upS / a.yolo (see ConvArgs), channels-last.  Off
// the hot path: the per-element index arithmetic is plain.
__device__ inline void store_nhwc_variant(const ConvArgs& a, __amdgpu_buffer_rsrc_t outR, int64_t m, int64_t f,
                                          float v) {
  const int64_t OHW = a.g.OHW, OW = a.g.OW;
  const int64_t b = m / OHW, p = m - b * OHW;
  if (a.upS > 0) {
    const int64_t s = a.upS, OH = OHW / OW, y = p / OW, x = p - y * OW, OWs = OW * s;
    const int64_t base = (b * OH * s + y * s) * OWs + x * s;
    const float sv = a.upScale * v;
    for (int64_t dy = 0; dy < s; ++dy)
      for (int64_t dx = 0; dx < s; ++dx)
        buf_st1s(outR, sv, static_cast<uint32_t>(((base + dy * OWs + dx) * a.outPix + f) * 4), 0);
  } else {
    buf_st1s(outR, v, static_cast<uint32_t>((m * a.outPix + f) * 4), 0);
  }
  if (a.yolo) a.yolo[(b * a.F + f) * OHW + p] = yolo_entry(v, static_cast<int>(f % a.yoloEntries));
}

// Channels-last epilogue (rows m = output pixels, columns = filters): the
// result of pixel m, filter f goes to out[m * outPix + f] (residual likewise
// with resPix).  Each lane owns FN filter columns (bias per lane); the pixel
// part of an offset is wave-uniform (scalar operand).  Residual loads are all
// issued before the first store; out-of-range elements get kOOB.
template <int FM, int FN, bool VAR = false>
__device__ __attribute__((always_inline)) inline void conv_store_nhwc(const ConvArgs& a, const f32x16 (&acc)[FM][FN], int64_t m0w, int64_t n0w,
                                       int lane) {
  const int h = lane >> 5;
  const int64_t M = a.g.N;
  const int rowBase = static_cast<int>(m0w) + 4 * h;  // pixel of element (i = 0, r = 0)
  const bool allRows = m0w + FM * 32 <= M;
  auto rowOk = [&](int c) { return allRows || rowBase + c < M; };
  const uint32_t op4 = static_cast<uint32_t>(a.outPix) * 4u, rp4 = static_cast<uint32_t>(a.resPix) * 4u;
  const __amdgpu_buffer_rsrc_t outR = make_rsrc(a.out, a.outBytes);
  const __amdgpu_buffer_rsrc_t resR = make_rsrc(a.res, a.resBytes);
  float bias[FN];
  uint32_t vOut[FN], vRes[FN];
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    const int64_t f = n0w + j * 32 + (lane & 31);
    const bool okF = f < a.F;
    bias[j] = a.bias && okF ? a.bias[f] : -0.f;  // -0.0: the exact additive identity
    vOut[j] = sel_off(okF, static_cast<uint32_t>(rowBase) * op4 + static_cast<uint32_t>(f) * 4u);
    vRes[j] = sel_off(okF, static_cast<uint32_t>(rowBase) * rp4 + static_cast<uint32_t>(f) * 4u);
  }
  auto rc = [](int i, int r) { return i * 32 + 8 * (r >> 2) + (r & 3); };
  if constexpr (VAR) {  // epilogue variants (a.upS > 0 or a.yolo): their own kernel instantiations
    if (a.yolo && a.upS == 0 && a.yoloBytes > 0 && !a.res) {
      // A yolo head: the plain stores of `out` and the NCHW head
      // yolo[(b*F + f)*OHW + p].  Registers 4g .. 4g+3 of a lane hold 4
      // consecutive pixels of its filter, so with yoloVec they are one 16-byte
      // store into the head (lanes l and l + 32 fill 32 consecutive bytes, the
      // four groups g a 128-byte line); else 4 single stores.  Both outputs
      // are stored with the default cache policy, not written through: a
      // head store covers 32 bytes of 32 lines, and a pixel row of `out`
      // (5 + classes values per anchor, e.g. 255) is not line-aligned, so L2
      // merges the partial lines (52x52 head at batch 16: 82 -> 74 -> 67 us).
      const uint32_t OHW = static_cast<uint32_t>(a.g.OHW), F32 = static_cast<uint32_t>(a.F);
      const __amdgpu_buffer_rsrc_t yR = make_rsrc(a.yolo, a.yoloBytes);
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int64_t f = n0w + j * 32 + (lane & 31);
        const bool okF = f < a.F;
        const uint32_t fu = okF ? static_cast<uint32_t>(f) : 0u;
        const int entry = static_cast<int>(fu % static_cast<uint32_t>(a.yoloEntries));
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const int c0 = i * 32 + 8 * g;  // row of register 4g, relative to rowBase
            float v[4], y[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              v[e] = apply_act(acc[i][j][4 * g + e] + bias[j], a.act);
              y[e] = yolo_entry(v[e], entry);
              __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v[e]), outR,
                                                    rowOk(c0 + e) ? vOut[j] : kOOB,
                                                    static_cast<uint32_t>(c0 + e) * op4, 0);
            }
            const uint32_t m = static_cast<uint32_t>(rowBase + c0);
            if (a.yoloVec) {  // m % 4 == 0 and M % 4 == 0: the 4 pixels are in range together, in one image
              const uint32_t b = m / OHW, px = m - b * OHW;
              const uint32_t off = sel_off(okF && rowOk(c0), ((b * F32 + fu) * OHW + px) * 4u);
              __builtin_amdgcn_raw_buffer_store_b128(
                  __builtin_bit_cast(__attribute__((ext_vector_type(4))) uint32_t, f32x4{y[0], y[1], y[2], y[3]}), yR,
                  off, 0, 0);
            } else {
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                const uint32_t b = (m + e) / OHW, px = m + e - b * OHW;
                __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, y[e]), yR,
                                                      sel_off(okF && rowOk(c0 + e), ((b * F32 + fu) * OHW + px) * 4u),
                                                      0, 0);
              }
            }
          }
      }
      return;
    }
    if (a.upS > 0 || a.yolo) {  // epilogue variants: generic per-element stores
      const __amdgpu_buffer_rsrc_t resG = make_rsrc(a.res, a.resBytes);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          const int64_t f = n0w + j * 32 + (lane & 31);
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int64_t m = rowBase + rc(i, r);
            if (f >= a.F || m >= M) continue;
            float v = acc[i][j][r] + bias[j];
            v = apply_act(v, a.act);
            if (a.res) v = v + buf_ld1s(resG, static_cast<uint32_t>((m * a.resPix + f) * 4), 0);
            store_nhwc_variant(a, outR, m, f, v);
          }
        }
      return;
    }
  }
  auto finish = [&](auto actTag, auto resTag) {
    constexpr int ACT = decltype(actTag)::value;
    constexpr bool RES = decltype(resTag)::value;
    float rv[FM][FN][16];
    if constexpr (RES) {
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r)
            rv[i][j][r] = buf_ld1s(resR, rowOk(rc(i, r)) ? vRes[j] : kOOB, static_cast<uint32_t>(rc(i, r)) * rp4);
    }
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          float v = apply_act(acc[i][j][r] + bias[j], ACT);
          if constexpr (RES) v = v + rv[i][j][r];
          buf_st1s(outR, v, rowOk(rc(i, r)) ? vOut[j] : kOOB, static_cast<uint32_t>(rc(i, r)) * op4);
        }
  };
  using Leaky = std::integral_constant<int, TNH_AC_LEAKY>;
  using Logistic = std::integral_constant<int, TNH_AC_LOGISTIC>;
  using Linear = std::integral_constant<int, TNH_AC_LINEAR>;
  if (a.res) {
    if (a.act == TNH_AC_LEAKY)
      finish(Leaky{}, std::true_type{});
    else if (a.act == TNH_AC_LOGISTIC)
      finish(Logistic{}, std::true_type{});
    else
      finish(Linear{}, std::true_type{});
  } else {
    if (a.act == TNH_AC_LEAKY)
      finish(Leaky{}, std::false_type{});
    else if (a.act == TNH_AC_LOGISTIC)
      finish(Logistic{}, std::false_type{});
    else
      finish(Linear{}, std::false_type{});
  }
}

}  // namespace conv
}  // namespace tnh
