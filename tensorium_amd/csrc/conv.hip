// Fused convolution forward: implicit GEMM (im2col gathered straight into
// LDS) on MFMA with the bias + activation (+ shortcut) epilogue applied to
// the accumulators before the single write of the output.
//
// GEMM view (Conv2D, ntensors.pas:8252-8345, batch merged into N):
//   M = F filters, N = batch*OH*OW, K = C*kh*kw
//   A = weights [F][K] row-major
//   B = im2col(x) gathered on the fly
// Epilogue per element (reference order, nConvolutionLayer.pas:508-545 and
// naddlayer.pas:698):  v = acc + bias[f];  v = act(v);  v = v + residual.
//
// Weight layouts: TNH_WEIGHTS_REFERENCE = [F][C][kh][kw] (the reference's
// filter-major storage, nConvolutionLayer.pas:206), TNH_WEIGHTS_TAP_MAJOR =
// [F][kh][kw][C] (tnh_conv2d_pack_weights).  With tap-major weights and
// C % BK == 0 each K panel lies inside one (ky, kx) tap and the gather does
// one bounds test per panel.
//
// Kernel choice: several tile shapes are compiled; the first call for a
// shape times the valid candidates with HIP events (when autotuning is on
// and the stream is not being captured) and caches the fastest; otherwise a
// wave-quantization cost model picks one.
#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <mutex>
#include <unordered_map>
#include <vector>

#include "common.hpp"
#include "conv_args.hpp"
#include "conv_first.hpp"
#include "conv_lean.hpp"
#include "conv_wsplit.hpp"
#include "gemm_core.hpp"

// Scratch of the no-allocation entry point tnh_conv2d_fwd_nhwc_noalloc: the
// K pieces of tail-split / split-K tiles go here instead of the context's
// growable workspace.  Each device holds its own copy of the array from the
// library's init call until the process ends.  Host code never uses the
// array's name as an address: it keeps the per-device pointer
// hipGetSymbolAddress returns (conv_scratch_setup) and passes that.
constexpr int64_t kNoAllocScratchFloats = int64_t(16) << 20;  // 64 MiB
static __device__ __align__(256) float scratch[kNoAllocScratchFloats];

namespace tnh {

namespace {
std::mutex g_scratch_mu;
std::unordered_map<int, float*> g_scratch_ptr;  // device -> address of `scratch` there
}  // namespace

int conv_scratch_setup(int device) {
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (g_scratch_ptr.count(device)) return TNH_OK;
  void* p = nullptr;
  if (int st = hip_status(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)")) return st;
  if (!p) return fail(TNH_ERR_HIP, "hipGetSymbolAddress(scratch) returned NULL on device %d", device);
  g_scratch_ptr[device] = static_cast<float*>(p);
  return TNH_OK;
}

namespace conv {
namespace {

float* scratch_for(int device) {
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  auto it = g_scratch_ptr.find(device);
  return it == g_scratch_ptr.end() ? nullptr : it->second;
}


template <class Cfg, int MODE, bool VA, bool VB>
struct KernelTraits;

template <class Cfg, bool VA, bool VB>
struct KernelTraits<Cfg, kGatherRef3, VA, VB> { using BL = ConvGatherLoader<3, 3, Cfg::BN, Cfg::BK, Cfg::NT>; };
template <class Cfg, bool VA, bool VB>
struct KernelTraits<Cfg, kGatherRef1, VA, VB> { using BL = ConvGatherLoader<1, 1, Cfg::BN, Cfg::BK, Cfg::NT>; };
template <class Cfg, bool VA, bool VB>
struct KernelTraits<Cfg, kTap3, VA, VB> { using BL = ConvTapLoader<3, Cfg::BN, Cfg::BK, Cfg::NT>; };
template <class Cfg, bool VA, bool VB>
struct KernelTraits<Cfg, k1x1, VA, VB> { using BL = Conv1x1Loader<VB, Cfg::BN, Cfg::BK, Cfg::NT>; };
template <class Cfg, bool VA, bool VB>
struct KernelTraits<Cfg, kGatherTap3, VA, VB> { using BL = ConvGatherTapLoader<3, 3, Cfg::BN, Cfg::BK, Cfg::NT>; };
template <class Cfg, bool VA, bool VB>
struct KernelTraits<Cfg, kGatherDyn, VA, VB> { using BL = ConvGatherDynLoader<Cfg::BN, Cfg::BK, Cfg::NT>; };

template <class Cfg, int MODE, bool VA, bool VB>
__global__ __launch_bounds__(Cfg::NT, Cfg::OCC) void conv_kernel(ConvArgs a) {
  using AL = DenseLoader<true, VA, Cfg::BM, Cfg::BK, Cfg::NT>;
  using BL = typename KernelTraits<Cfg, MODE, VA, VB>::BL;
  using Main = GemmMainloop<Cfg, AL, BL>;
  __shared__ __attribute__((aligned(16))) float smem[Main::LDS_FLOATS];
  lds_t* lds = (lds_t*)smem;

  int tm, tn;
  tile_coords(blockIdx.x, a.tilesM, a.tilesN, tm, tn);
  const int64_t m0 = static_cast<int64_t>(tm) * Cfg::BM, n0 = static_cast<int64_t>(tn) * Cfg::BN;

  AL al;
  al.init(a.w, a.wBytes, a.g.K, a.F, a.g.K, m0, threadIdx.x);
  BL bl;
  bl.init(a.g, n0, threadIdx.x);

  f32x16 acc[Cfg::FM][Cfg::FN];
  const int64_t kBegin = blockIdx.y * a.kChunk;
  const int64_t kEnd = min(a.g.K, kBegin + a.kChunk);
  Main::exec(al, bl, kBegin, kEnd, lds, acc);

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave / Cfg::WN, wn = wave % Cfg::WN;
  conv_store<Cfg::FM, Cfg::FN>(a, acc, m0 + wm * Cfg::WTM, n0 + wn * Cfg::WTN, lane);
}


// Few-channel 3x3 convolution (C <= 4, e.g. the RGB input layer): the
// output is store-bound (F outputs per pixel against 9*C inputs), so instead
// of a GEMM each thread owns one output pixel, keeps its 9*C window inputs
// in registers and walks the filters four at a time.  The weights and the
// bias are wave-uniform: they are read through the scalar cache into SGPRs
// and feed the fused multiply-adds directly, and the activation is a template
// argument, so the filter loop holds no vector load and no branch (a vector
// load there would make every filter wait for the stores already issued).
// Every store is coalesced along the pixel row.  Each output is a sequential
// fused multiply-add chain over k in the reference order k = (c*3 + ky)*3 +
// kx from 0, padding taps included as zeros: exactly the arithmetic of the
// reference CPU path (im2col, then the saxpy chain of ntensors.pas:1308-1436),
// then bias, activation, residual.
template <int C>
__device__ inline void smallc_window(const ConvArgs& a, bool valid, int b, int p, float (&in)[9 * C]) {
  const int OW = a.g.OW, H = a.g.H, W = a.g.W;
  const int oy = p / OW, ox = p - (p / OW) * OW;
  const int iy0 = oy * a.g.sY - a.g.pH, ix0 = ox * a.g.sX - a.g.pW;
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.g.x, a.g.xBytes);
  const uint32_t base = static_cast<uint32_t>(static_cast<int64_t>(b) * a.g.xBatchStride * 4);
#pragma unroll
  for (int c = 0; c < C; ++c)
#pragma unroll
    for (int ky = 0; ky < 3; ++ky)
#pragma unroll
      for (int kx = 0; kx < 3; ++kx) {
        const int iy = iy0 + ky, ix = ix0 + kx;
        const bool ok = valid && static_cast<unsigned>(iy) < static_cast<unsigned>(H) &&
                        static_cast<unsigned>(ix) < static_cast<unsigned>(W);
        in[(c * 3 + ky) * 3 + kx] =
            buf_ld1(xr, sel_off(ok, base + static_cast<uint32_t>((c * H + iy) * W + ix) * 4u));
      }
}

// weight of filter f at reference index k = c*9 + t (tap-major storage: t*C + c)
template <int C, bool TAP>
__device__ inline float smallc_wt(const float* __restrict__ w, int f, int k) {
  return w[f * 9 * C + (TAP ? (k % 9) * C + k / 9 : k)];
}

// Four filters' sequential chains over one pixel's window, then bias and
// activation.  HB: a bias is given (without one, -0.0 is added: the exact
// additive identity).
template <int C, bool TAP, int ACT, bool HB>
__device__ inline void smallc_quad(const float* __restrict__ w, const float* __restrict__ bias, int f,
                                   const float (&in)[9 * C], float (&v)[4]) {
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int k = 0; k < 9 * C; ++k)
#pragma unroll
    for (int q = 0; q < 4; ++q) acc[q] = fmaf(smallc_wt<C, TAP>(w, f + q, k), in[k], acc[q]);
#pragma unroll
  for (int q = 0; q < 4; ++q) v[q] = apply_act(acc[q] + (HB ? bias[f + q] : -0.f), ACT);
}

template <int C, bool TAP, int ACT, bool HB>
__device__ inline float smallc_one(const float* __restrict__ w, const float* __restrict__ bias, int f,
                                   const float (&in)[9 * C]) {
  float acc = 0.f;
#pragma unroll
  for (int k = 0; k < 9 * C; ++k) acc = fmaf(smallc_wt<C, TAP>(w, f, k), in[k], acc);
  return apply_act(acc + (HB ? bias[f] : -0.f), ACT);
}

// The bias and residual cases are compile-time branches of the kernels
// below: a run-time test inside the filter loop costs about a third of the
// layer's time (the loop's loads and stores can no longer be scheduled
// across it).
template <int C, bool TAP, int ACT>
__global__ __launch_bounds__(256) void conv_smallc_kernel(ConvArgs a, const float* __restrict__ w,
                                                          const float* __restrict__ bias) {
  constexpr int K = 9 * C;
  // consecutive blocks of pixels on one XCD: the input rows a block shares
  // with its neighbours stay in that XCD's L2
  const int64_t n = static_cast<int64_t>(xcd_block(blockIdx.x, gridDim.x)) * 256 + threadIdx.x;
  if (n >= a.g.N) return;
  const int F = static_cast<int>(a.F);
  const int OHW = a.g.OHW;
  const int b = static_cast<int>(n / OHW);
  const int p = static_cast<int>(n - static_cast<int64_t>(b) * OHW);
  // blockIdx.y picks a range of fg filters (a multiple of 4): a small
  // layer gets more waves to hide its window loads' latency behind
  const int fg = static_cast<int>(a.fGroup);
  const int fBeg = static_cast<int>(blockIdx.y) * fg;
  const int fEnd = min(F, fBeg + fg);
  float in[K];
  smallc_window<C>(a, true, b, p, in);
  float* out = a.out + static_cast<int64_t>(b) * a.outBatchStride + p;
  const float* res = a.res ? a.res + static_cast<int64_t>(b) * a.rBatchStride + p : nullptr;
  auto run = [&](auto hbTag, auto resTag) {
    constexpr bool HB = decltype(hbTag)::value, RES = decltype(resTag)::value;
    int f = fBeg;
    for (; f + 4 <= fEnd; f += 4) {
      float rv[4] = {0.f, 0.f, 0.f, 0.f};
      if constexpr (RES) {  // issued before the chains, used after them
#pragma unroll
        for (int q = 0; q < 4; ++q) rv[q] = res[static_cast<int64_t>(f + q) * OHW];
      }
      float v[4];
      smallc_quad<C, TAP, ACT, HB>(w, bias, f, in, v);
#pragma unroll
      for (int q = 0; q < 4; ++q) out[static_cast<int64_t>(f + q) * OHW] = RES ? v[q] + rv[q] : v[q];
    }
    for (; f < fEnd; ++f) {
      const float v = smallc_one<C, TAP, ACT, HB>(w, bias, f, in);
      out[static_cast<int64_t>(f) * OHW] = RES ? v + res[static_cast<int64_t>(f) * OHW] : v;
    }
  };
  if (bias) {
    if (res)
      run(std::true_type{}, std::true_type{});
    else
      run(std::true_type{}, std::false_type{});
  } else {
    if (res)
      run(std::false_type{}, std::true_type{});
    else
      run(std::false_type{}, std::false_type{});
  }
}

// Channels-last output of the few-channel kernel: the same per-pixel
// sequential FMA chains (bit-exact), 32 filters at a time.  Each wave then
// passes its 64 pixels x 32 results through LDS so that 8 consecutive lanes
// store one pixel's 32 channels (128 contiguous bytes) with 16-byte stores.
// The LDS block is 64 rows of eight 16-byte chunks; chunk c of row r sits at
// r*8 + (c ^ ((r / 2) % 8)) (the panel swizzle of the conv kernels), so both
// the row-wise writes (16 lanes write 16 pixels' chunk c) and the pixel-wise
// reads (16 lanes read two rows) touch 16 different 16-byte bank groups of
// the 64-bank LDS.  The common case (no residual, whole
// 32-filter chunks, 16-byte aligned pixel rows) is a compile-time path of
// its own.
template <int C, bool TAP, int ACT>
__global__ __launch_bounds__(256) void conv_smallc_nhwc_kernel(ConvArgs a, const float* __restrict__ w,
                                                               const float* __restrict__ bias) {
  constexpr int K = 9 * C, FC = 32;
  __shared__ f32x4 tile[4][64 * FC / 4];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  // first pixel of this wave; consecutive blocks of pixels on one XCD (L2
  // reuse of the shared input rows)
  const int64_t nWave = static_cast<int64_t>(xcd_block(blockIdx.x, gridDim.x)) * 256 + wave * 64;
  const int64_t n = nWave + lane;
  const bool valid = n < a.g.N;
  const int F = static_cast<int>(a.F);
  const int OHW = a.g.OHW;
  const int64_t nn = valid ? n : 0;
  const int b = static_cast<int>(nn / OHW);
  const int p = static_cast<int>(nn - static_cast<int64_t>(b) * OHW);
  float in[K];
  smallc_window<C>(a, valid, b, p, in);
  f32x4* t = tile[wave];
  float* tf = reinterpret_cast<float*>(t);
  const bool vecOut = a.outPix % 4 == 0 && (reinterpret_cast<uintptr_t>(a.out) & 15) == 0;
  const bool vecRes = a.resPix % 4 == 0 && (reinterpret_cast<uintptr_t>(a.res) & 15) == 0;
  const int sw = (lane >> 1) & 7, qc = lane & 7;
  auto run = [&](auto hbTag, auto fastTag) {
    constexpr bool HB = decltype(hbTag)::value, FAST = decltype(fastTag)::value;
    for (int f0 = 0; f0 < F; f0 += FC) {
      const int fc = FAST ? FC : (F - f0 < FC ? F - f0 : FC);
      int q0 = 0;
      for (; q0 + 4 <= fc; q0 += 4) {  // four independent chains at a time
        float v[4];
        smallc_quad<C, TAP, ACT, HB>(w, bias, f0 + q0, in, v);
        t[lane * 8 + ((q0 >> 2) ^ sw)] = f32x4{v[0], v[1], v[2], v[3]};
      }
      if constexpr (!FAST) {
        for (; q0 < fc; ++q0)
          tf[(lane * 8 + ((q0 >> 2) ^ sw)) * 4 + (q0 & 3)] = smallc_one<C, TAP, ACT, HB>(w, bias, f0 + q0, in);
      }
      __builtin_amdgcn_wave_barrier();
      // pass it: lanes 8j .. 8j+7 store pixel 8*it + j, lane chunk (lane & 7) = channels 4*(lane & 7) .. +3
      const int q = 4 * qc;
#pragma unroll 2
      for (int it = 0; it < 8; ++it) {
        const int px = it * 8 + (lane >> 3);
        const int64_t np = nWave + px;
        const f32x4 v = t[px * 8 + (qc ^ ((px >> 1) & 7))];
        float* dst = a.out + np * a.outPix + f0 + q;
        if constexpr (FAST) {
          if (np < a.g.N) *reinterpret_cast<f32x4*>(dst) = v;
          continue;
        }
        if (np >= a.g.N || q >= fc) continue;
        float o[4] = {v[0], v[1], v[2], v[3]};
        if (a.res) {
          const float* res = a.res + np * a.resPix + f0 + q;
          if (vecRes && q + 4 <= fc) {
            const float4 r = *reinterpret_cast<const float4*>(res);
            o[0] = o[0] + r.x, o[1] = o[1] + r.y, o[2] = o[2] + r.z, o[3] = o[3] + r.w;
          } else {
#pragma unroll
            for (int u = 0; u < 4; ++u)
              if (q + u < fc) o[u] = o[u] + res[u];
          }
        }
        if (vecOut && q + 4 <= fc) {
          *reinterpret_cast<float4*>(dst) = make_float4(o[0], o[1], o[2], o[3]);
        } else {
#pragma unroll
          for (int u = 0; u < 4; ++u)
            if (q + u < fc) dst[u] = o[u];
        }
      }
      __builtin_amdgcn_wave_barrier();
    }
  };
  const bool fast = !a.res && vecOut && F % FC == 0;
  if (bias) {
    if (fast)
      run(std::true_type{}, std::true_type{});
    else
      run(std::true_type{}, std::false_type{});
  } else {
    if (fast)
      run(std::false_type{}, std::true_type{});
    else
      run(std::false_type{}, std::false_type{});
  }
}

template <int C, bool TAP, bool NHWC>
void launch_smallc_act(ConvArgs a, unsigned blocks, hipStream_t s) {
  // NCHW: the filters split into groups over grid.y until the launch has
  // about kWaves waves, keeping at least kMinFilters per group (each group's
  // threads load the pixel's window again, from the caches).  Config 3's
  // conv1 (32 filters, 2048 waves): two groups, 0.318 -> 0.313 ms per step;
  // config 1 (16 filters, 2704 waves) stays whole: two groups of 8 took
  // 7.6 against 7.4 us, four of 4 8.2 us.
  constexpr int64_t kWaves = 4096, kMinFilters = 16;
  int64_t groups = 1;
  if (!NHWC) {
    const int64_t waves = static_cast<int64_t>(blocks) * 4;
    groups = std::max<int64_t>(1, std::min<int64_t>((kWaves + waves - 1) / waves, a.F / kMinFilters));
  }
  a.fGroup = ((a.F + groups - 1) / groups + 3) / 4 * 4;
  groups = (a.F + a.fGroup - 1) / a.fGroup;
  auto go = [&](auto actTag) {
    constexpr int ACT = decltype(actTag)::value;
    if constexpr (NHWC)
      hipLaunchKernelGGL((conv_smallc_nhwc_kernel<C, TAP, ACT>), dim3(blocks), dim3(256), 0, s, a, a.w, a.bias);
    else
      hipLaunchKernelGGL((conv_smallc_kernel<C, TAP, ACT>), dim3(blocks, static_cast<unsigned>(groups)), dim3(256),
                         0, s, a, a.w, a.bias);
  };
  if (a.act == TNH_AC_LEAKY)
    go(std::integral_constant<int, TNH_AC_LEAKY>{});
  else if (a.act == TNH_AC_LOGISTIC)
    go(std::integral_constant<int, TNH_AC_LOGISTIC>{});
  else
    go(std::integral_constant<int, TNH_AC_LINEAR>{});
}

template <bool TAP, bool NHWC>
int launch_smallc(const ConvArgs& a, hipStream_t s) {
  const unsigned blocks = static_cast<unsigned>((a.g.N + 255) / 256);
  auto go = [&](auto cTag) {
    constexpr int C = decltype(cTag)::value;
    launch_smallc_act<C, TAP, NHWC>(a, blocks, s);
  };
  switch (a.g.C) {
    case 1: go(std::integral_constant<int, 1>{}); break;
    case 2: go(std::integral_constant<int, 2>{}); break;
    case 3: go(std::integral_constant<int, 3>{}); break;
    default: go(std::integral_constant<int, 4>{}); break;
  }
  return launch_status(NHWC ? "conv_smallc_nhwc_kernel" : "conv_smallc_kernel");
}

// Sums the split-K partials in split order (deterministic) and applies the
// epilogue: one thread per output element, consecutive threads along n.  S
// is the split count: the S partial loads of an element are issued together
// and summed afterwards, so a thread waits for one memory round trip rather
// than S.
template <int S>
__global__ __launch_bounds__(256) void conv_splitk_reduce(ConvArgs a) {
  const int64_t total = a.F * a.g.N, OHW = a.g.OHW;
  for (int64_t e = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; e < total; e += int64_t(gridDim.x) * blockDim.x) {
    const int64_t f = e / a.g.N, n = e - f * a.g.N;
    float p[S];
#pragma unroll
    for (int s = 0; s < S; ++s) p[s] = a.part[s * total + e];
    float v = p[0];
#pragma unroll
    for (int s = 1; s < S; ++s) v = v + p[s];
    const int64_t b = n / OHW, q = n - b * OHW;
    if (a.bias) v = v + a.bias[f];
    v = apply_act(v, a.act);
    if (a.res) v = v + a.res[b * a.rBatchStride + f * OHW + q];
    a.out[b * a.outBatchStride + f * OHW + q] = v;
  }
}

// ---------------------------------------------------------------------------
// tile configurations
// ---------------------------------------------------------------------------
// LDS-staged tiles (tile M x N x K depth, waves M x N, prefetch depth,
// occupancy), chosen from sweeps of the YOLOv3 layer shapes: small tiles
// with two panels of prefetch keep the most waves resident and win on most
// shapes; the autotuner picks per layer shape.
using Cfg0 = TileCfg<64, 64, 32, 2, 2, 2, 1>;
using Cfg1 = TileCfg<64, 64, 16, 2, 2, 2, 8>;
using Cfg2 = TileCfg<128, 64, 16, 2, 2, 2, 5>;
using Cfg3 = TileCfg<128, 128, 16, 2, 2, 1, 1>;
using Cfg4 = TileCfg<64, 128, 32, 2, 2, 2, 1>;
using Cfg5 = TileCfg<64, 128, 16, 2, 2, 2, 5>;
// ids 6-10 are retired (register-direct tiles that the tuner never chose on
// any profiled shape); the ids of the other tiles stay as they were
// lean tiles (conv_lean.hpp: tile M x N x K depth, waves M x N, occupancy)
using Lean11 = LeanCfg<64, 64, 32, 2, 2, 4>;
using Lean12 = LeanCfg<64, 128, 32, 2, 2, 3>;
using Lean13 = LeanCfg<128, 64, 32, 2, 2, 3>;
using Lean14 = LeanCfg<128, 128, 32, 2, 2, 2>;
using Lean15 = LeanCfg<64, 64, 64, 2, 2, 2>;
using Lean16 = LeanCfg<64, 32, 32, 2, 1, 6>;
using Lean17 = LeanCfg<128, 64, 32, 4, 2, 2>;
using Lean18 = LeanCfg<64, 128, 32, 2, 4, 2>;
using Lean19 = LeanCfg<128, 128, 32, 4, 2, 2>;

// wave-split tiles, both layouts (conv_wsplit.hip: K of one tile split over
// the waves of its workgroup), ids kWsFirst + index into kWsCfgs
constexpr int kWsFirst = 20;

enum CfgKind { kLds = 0, kRetired = 1, kLean = 2, kWsplit = 3 };
struct CfgInfo {
  int BM, BN, BK;
  float eff;  // relative per-CU throughput used by the cost model
  int perCU;  // resident workgroups per CU assumed by the cost model
  int kind;
};
constexpr int kNumCfg = kWsFirst + kNumWs;
const CfgInfo kCfgs[kNumCfg] = {
    {64, 64, 32, 1.00f, 4, kLds},     {64, 64, 16, 1.00f, 8, kLds},     {128, 64, 16, 0.97f, 5, kLds},
    {128, 128, 16, 0.95f, 2, kLds},   {64, 128, 32, 0.97f, 3, kLds},    {64, 128, 16, 0.95f, 5, kLds},
    {0, 0, 0, 0.f, 0, kRetired},      {0, 0, 0, 0.f, 0, kRetired},      {0, 0, 0, 0.f, 0, kRetired},
    {0, 0, 0, 0.f, 0, kRetired},      {0, 0, 0, 0.f, 0, kRetired},      {64, 64, 32, 1.15f, 4, kLean},
    {64, 128, 32, 1.10f, 3, kLean},   {128, 64, 32, 1.10f, 3, kLean},   {128, 128, 32, 1.05f, 2, kLean},
    {64, 64, 64, 1.10f, 2, kLean},    {64, 32, 32, 1.10f, 6, kLean},    {128, 64, 32, 1.10f, 2, kLean},
    {64, 128, 32, 1.10f, 2, kLean},   {128, 128, 32, 1.05f, 2, kLean},
    // wave-split tiles: timed only (the cost model never picks them)
    {32, 32, 32, 1.f, 1, kWsplit},    {32, 32, 32, 1.f, 1, kWsplit},    {32, 64, 32, 1.f, 1, kWsplit},
    {16, 32, 32, 1.f, 1, kWsplit},    {16, 32, 32, 1.f, 1, kWsplit},    {16, 16, 32, 1.f, 1, kWsplit},
    {16, 16, 32, 1.f, 1, kWsplit},
};
static_assert(sizeof(kCfgs) / sizeof(kCfgs[0]) == kNumCfg, "one CfgInfo per configuration");

template <class Cfg>
int grid_for(ConvArgs& a, dim3& grid) {
  const int64_t tm = (a.F + Cfg::BM - 1) / Cfg::BM, tn = (a.g.N + Cfg::BN - 1) / Cfg::BN;
  if (tm * tn > INT32_MAX) return fail(TNH_ERR_UNSUPPORTED, "conv2d: grid too large");
  a.tilesM = static_cast<int>(tm);
  a.tilesN = static_cast<int>(tn);
  if (a.splits > 1) {
    const int64_t panels = (a.g.K + Cfg::BK - 1) / Cfg::BK;
    a.kChunk = (panels + a.splits - 1) / a.splits * Cfg::BK;
    a.splits = static_cast<int>((a.g.K + a.kChunk - 1) / a.kChunk);  // no empty split
  } else {
    a.kChunk = a.g.K;
  }
  grid = dim3(static_cast<unsigned>(tm * tn), static_cast<unsigned>(a.splits));
  return TNH_OK;
}

// Second launch of a split-K convolution: sums the partials and applies the
// epilogue (nothing to do without split-K).
int launch_reduce(const ConvArgs& a, hipStream_t s) {
  if (a.splits <= 1) return TNH_OK;
  const int64_t total = a.F * a.g.N;
  const int64_t blocks = (total + 255) / 256;
  const dim3 grid(static_cast<unsigned>(blocks < 65536 ? blocks : 65536));
  switch (a.splits) {
#define TNH_REDUCE_CASE(S) \
  case S: hipLaunchKernelGGL(conv_splitk_reduce<S>, grid, dim3(256), 0, s, a); break;
    TNH_REDUCE_CASE(2) TNH_REDUCE_CASE(3) TNH_REDUCE_CASE(4) TNH_REDUCE_CASE(5) TNH_REDUCE_CASE(6)
    TNH_REDUCE_CASE(7) TNH_REDUCE_CASE(8) TNH_REDUCE_CASE(9) TNH_REDUCE_CASE(10) TNH_REDUCE_CASE(11)
    TNH_REDUCE_CASE(12) TNH_REDUCE_CASE(13) TNH_REDUCE_CASE(14) TNH_REDUCE_CASE(15) TNH_REDUCE_CASE(16)
#undef TNH_REDUCE_CASE
    default: return fail(TNH_ERR_UNSUPPORTED, "conv2d: %d split-K partitions (at most 16)", a.splits);
  }
  return launch_status("conv_splitk_reduce");
}

template <class Cfg, int MODE>
int launch_mode(ConvArgs a, bool va, bool vb, hipStream_t s) {
  dim3 grid;
  if (int st = grid_for<Cfg>(a, grid)) return st;
  if constexpr (MODE == k1x1) {
    if (va && vb)
      hipLaunchKernelGGL((conv_kernel<Cfg, MODE, true, true>), grid, dim3(Cfg::NT), 0, s, a);
    else if (va)
      hipLaunchKernelGGL((conv_kernel<Cfg, MODE, true, false>), grid, dim3(Cfg::NT), 0, s, a);
    else if (vb)
      hipLaunchKernelGGL((conv_kernel<Cfg, MODE, false, true>), grid, dim3(Cfg::NT), 0, s, a);
    else
      hipLaunchKernelGGL((conv_kernel<Cfg, MODE, false, false>), grid, dim3(Cfg::NT), 0, s, a);
  } else if constexpr (MODE == kTap3) {
    hipLaunchKernelGGL((conv_kernel<Cfg, MODE, true, false>), grid, dim3(Cfg::NT), 0, s, a);
  } else {
    (void)va;
    (void)vb;
    hipLaunchKernelGGL((conv_kernel<Cfg, MODE, false, false>), grid, dim3(Cfg::NT), 0, s, a);
  }
  if (int st = launch_status("conv_kernel")) return st;
  return launch_reduce(a, s);
}

template <class Cfg>
int launch_cfg(const ConvArgs& a, int mode, bool va, bool vb, hipStream_t s) {
  switch (mode) {
    case kGatherRef3: return launch_mode<Cfg, kGatherRef3>(a, va, vb, s);
    case kGatherTap3: return launch_mode<Cfg, kGatherTap3>(a, va, vb, s);
    case kGatherRef1: return launch_mode<Cfg, kGatherRef1>(a, va, vb, s);
    case kGatherDyn: return launch_mode<Cfg, kGatherDyn>(a, va, vb, s);
    case kTap3: return launch_mode<Cfg, kTap3>(a, va, vb, s);
    default: return launch_mode<Cfg, k1x1>(a, va, vb, s);
  }
}

template <class Cfg>
int launch_lean(ConvArgs a, int mode, bool vb, int cus, hipStream_t s) {
  dim3 grid;
  if (int st = grid_for<Cfg>(a, grid)) return st;
  const int64_t tiles = static_cast<int64_t>(a.tilesM) * a.tilesN;
  if (a.tailSplits > 0 && a.splits <= 1) {
    // whole rounds of tiles (over the CUs, or over every resident workgroup
    // slot) stay whole; the remainder is cut along K so that every CU gets
    // about the same work
    const int64_t unit = a.tailUnit > 0 ? a.tailUnit : cus;
    const int64_t full = tiles / unit * unit;
    const int64_t panels = a.g.K / Cfg::BK;
    a.kChunk = (panels + a.tailSplits - 1) / a.tailSplits * Cfg::BK;
    a.tailSplits = static_cast<int>((a.g.K + a.kChunk - 1) / a.kChunk);  // no empty piece
    if (full == tiles || full == 0 || a.tailSplits < 2 ||
        (tiles - full) * std::max<int64_t>(a.tailSplits, Cfg::NT / 64) + full > INT32_MAX) {
      a.tailSplits = 0;
      a.kChunk = a.g.K;
    } else {
      a.nFull = static_cast<int>(full);
      grid = dim3(static_cast<unsigned>(full + (tiles - full) * a.tailSplits), 1);
    }
  } else {
    a.tailSplits = 0;
  }
  if (a.tailSplits == 0 || tiles - a.nFull > kTileCounters) a.tileCount = nullptr;
  if (mode == kTap3)
    hipLaunchKernelGGL((conv_lean_kernel<Cfg, kTap3, false>), grid, dim3(Cfg::NT), 0, s, a);
  else if (vb)
    hipLaunchKernelGGL((conv_lean_kernel<Cfg, k1x1, true>), grid, dim3(Cfg::NT), 0, s, a);
  else
    hipLaunchKernelGGL((conv_lean_kernel<Cfg, k1x1, false>), grid, dim3(Cfg::NT), 0, s, a);
  if (int st = launch_status("conv_lean_kernel")) return st;
  if (a.tailSplits > 0 && !a.tileCount) {
    hipLaunchKernelGGL((conv_tail_reduce<Cfg>), dim3(static_cast<unsigned>((tiles - a.nFull) * (Cfg::NT / 64))),
                       dim3(64), 0, s, a);
    return launch_status("conv_tail_reduce");
  }
  return launch_reduce(a, s);
}

// Floats of tail-split pieces a lean configuration writes for `tiles` tiles
// (0 when they divide evenly into rounds of `unit`).
int64_t tail_floats(int64_t tiles, int BM, int BN, int BK, int64_t K, int64_t unit, int tailSplits) {
  const int64_t rest = tiles % unit;
  const int64_t panels = K / BK;
  const int64_t chunk = (panels + tailSplits - 1) / tailSplits;
  const int64_t pieces = (panels + chunk - 1) / chunk;
  return tiles < unit ? 0 : rest * pieces * BM * BN;
}

// Workgroups of a lean configuration resident per CU (register and LDS
// limits), queried once per kernel.
template <class Cfg>
int lean_occ(int mode, bool vb) {
  auto q = [](const void* k) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, k, Cfg::NT, 0) != hipSuccess) {
      (void)hipGetLastError();
      n = 1;
    }
    return n > 0 ? n : 1;
  };
  static const int occTap = q(reinterpret_cast<const void*>(&conv_lean_kernel<Cfg, kTap3, false>));
  static const int occ1 = q(reinterpret_cast<const void*>(&conv_lean_kernel<Cfg, k1x1, false>));
  static const int occ1v = q(reinterpret_cast<const void*>(&conv_lean_kernel<Cfg, k1x1, true>));
  return mode == kTap3 ? occTap : (vb ? occ1v : occ1);
}

template <class Cfg>
int nhwc_occ(int mode) {
  auto q = [](const void* k) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, k, Cfg::NT, 0) != hipSuccess) {
      (void)hipGetLastError();
      n = 1;
    }
    return n > 0 ? n : 1;
  };
  static const int occTap = q(reinterpret_cast<const void*>(&conv_nhwc_kernel<Cfg, kTap3>));
  static const int occ1 = q(reinterpret_cast<const void*>(&conv_nhwc_kernel<Cfg, k1x1>));
  return mode == kTap3 ? occTap : occ1;
}

// Resident workgroups per CU of a lean configuration's kernel for this
// layout and mode.
int lean_occupancy(int cfg, int mode, bool vb, bool nhwc) {
  switch (cfg) {
    case 11: return nhwc ? nhwc_occ<Lean11>(mode) : lean_occ<Lean11>(mode, vb);
    case 12: return nhwc ? nhwc_occ<Lean12>(mode) : lean_occ<Lean12>(mode, vb);
    case 13: return nhwc ? nhwc_occ<Lean13>(mode) : lean_occ<Lean13>(mode, vb);
    case 14: return nhwc ? nhwc_occ<Lean14>(mode) : lean_occ<Lean14>(mode, vb);
    case 15: return nhwc ? nhwc_occ<Lean15>(mode) : lean_occ<Lean15>(mode, vb);
    case 16: return nhwc ? nhwc_occ<Lean16>(mode) : lean_occ<Lean16>(mode, vb);
    case 17: return nhwc ? nhwc_occ<Lean17>(mode) : lean_occ<Lean17>(mode, vb);
    case 18: return nhwc ? nhwc_occ<Lean18>(mode) : lean_occ<Lean18>(mode, vb);
    default: return nhwc ? nhwc_occ<Lean19>(mode) : lean_occ<Lean19>(mode, vb);
  }
}

// Channels-last launch of a lean configuration: rows are output pixels
// (tiles of BM), columns filters (tiles of BN).  a.tailSplits > 0 cuts the
// tiles beyond the last whole round of a.tailUnit tiles (the CU count when
// 0; every tile when negative) into K pieces.
template <class Cfg>
int launch_nhwc(ConvArgs a, int mode, int cus, hipStream_t s) {
  const int64_t tm = (a.g.N + Cfg::BM - 1) / Cfg::BM, tn = (a.F + Cfg::BN - 1) / Cfg::BN;
  if (tm * tn > INT32_MAX) return fail(TNH_ERR_UNSUPPORTED, "conv2d: grid too large");
  a.tilesM = static_cast<int>(tm);
  a.tilesN = static_cast<int>(tn);
  a.splits = 1;
  a.kChunk = a.g.K;
  const int64_t tiles = tm * tn;
  int64_t grid = tiles;
  if (a.tailSplits > 0) {
    const int64_t unit = a.tailUnit > 0 ? a.tailUnit : cus;
    const int64_t full = a.tailUnit < 0 ? 0 : tiles / unit * unit;
    const int64_t panels = a.g.K / Cfg::BK;
    a.kChunk = (panels + a.tailSplits - 1) / a.tailSplits * Cfg::BK;
    a.tailSplits = static_cast<int>((a.g.K + a.kChunk - 1) / a.kChunk);  // no empty piece
    if (full == tiles || a.tailSplits < 2 ||
        (tiles - full) * std::max<int64_t>(a.tailSplits, Cfg::NT / 64) + full > INT32_MAX) {
      a.tailSplits = 0;
      a.kChunk = a.g.K;
    } else {
      a.nFull = static_cast<int>(full);
      grid = full + (tiles - full) * a.tailSplits;
    }
  } else {
    a.tailSplits = 0;
  }
  if (a.tailSplits == 0 || tiles - a.nFull > kTileCounters) a.tileCount = nullptr;
  const bool var = a.upS > 0 || a.yolo;  // epilogue variant: its own instantiations
  const dim3 g(static_cast<unsigned>(grid)), nt(Cfg::NT);
  if (mode == kTap3 && var)
    hipLaunchKernelGGL((conv_nhwc_kernel<Cfg, kTap3, true>), g, nt, 0, s, a);
  else if (mode == kTap3)
    hipLaunchKernelGGL((conv_nhwc_kernel<Cfg, kTap3>), g, nt, 0, s, a);
  else if (var)
    hipLaunchKernelGGL((conv_nhwc_kernel<Cfg, k1x1, true>), g, nt, 0, s, a);
  else
    hipLaunchKernelGGL((conv_nhwc_kernel<Cfg, k1x1>), g, nt, 0, s, a);
  if (int st = launch_status("conv_nhwc_kernel")) return st;
  if (a.tailSplits > 0 && !a.tileCount) {
    const dim3 rg(static_cast<unsigned>((tiles - a.nFull) * (Cfg::NT / 64)));
    if (var)
      hipLaunchKernelGGL((conv_tail_reduce<Cfg, true, true>), rg, dim3(64), 0, s, a);
    else
      hipLaunchKernelGGL((conv_tail_reduce<Cfg, true>), rg, dim3(64), 0, s, a);
    return launch_status("conv_tail_reduce");
  }
  return TNH_OK;
}

// Channels-last convolution over C % 4 == 0 channels that are not a
// multiple of 32 (kTap3Any / k1x1Any): one fixed tile, 64 x 32 for up to 32
// filters, else 64 x 64; no tuning and no K split (these are the thin early
// layers of small networks, e.g. 16 channels in YOLOv3-tiny).
template <class Cfg>
int launch_nhwc_any_cfg(ConvArgs a, int mode, hipStream_t s) {
  const int64_t tm = (a.g.N + Cfg::BM - 1) / Cfg::BM, tn = (a.F + Cfg::BN - 1) / Cfg::BN;
  if (tm * tn > INT32_MAX) return fail(TNH_ERR_UNSUPPORTED, "conv2d: grid too large");
  a.tilesM = static_cast<int>(tm);
  a.tilesN = static_cast<int>(tn);
  a.splits = 1;
  a.kChunk = a.g.K;
  a.tailSplits = 0;
  const dim3 grid(static_cast<unsigned>(tm * tn));
  const bool var = a.upS > 0 || a.yolo;
  if (mode == kTap3Any && var)
    hipLaunchKernelGGL((conv_nhwc_kernel<Cfg, kTap3Any, true>), grid, dim3(Cfg::NT), 0, s, a);
  else if (mode == kTap3Any)
    hipLaunchKernelGGL((conv_nhwc_kernel<Cfg, kTap3Any>), grid, dim3(Cfg::NT), 0, s, a);
  else if (var)
    hipLaunchKernelGGL((conv_nhwc_kernel<Cfg, k1x1Any, true>), grid, dim3(Cfg::NT), 0, s, a);
  else
    hipLaunchKernelGGL((conv_nhwc_kernel<Cfg, k1x1Any>), grid, dim3(Cfg::NT), 0, s, a);
  return launch_status("conv_nhwc_kernel");
}

int launch_nhwc_any(const ConvArgs& a, int mode, hipStream_t s) {
  return a.F <= 32 ? launch_nhwc_any_cfg<Lean16>(a, mode, s) : launch_nhwc_any_cfg<Lean11>(a, mode, s);
}

int launch_nhwc_cfg(int cfg, const ConvArgs& a, int mode, int cus, hipStream_t s) {
  switch (cfg) {
    case 11: return launch_nhwc<Lean11>(a, mode, cus, s);
    case 12: return launch_nhwc<Lean12>(a, mode, cus, s);
    case 13: return launch_nhwc<Lean13>(a, mode, cus, s);
    case 14: return launch_nhwc<Lean14>(a, mode, cus, s);
    case 15: return launch_nhwc<Lean15>(a, mode, cus, s);
    case 16: return launch_nhwc<Lean16>(a, mode, cus, s);
    case 17: return launch_nhwc<Lean17>(a, mode, cus, s);
    case 18: return launch_nhwc<Lean18>(a, mode, cus, s);
    case 19: return launch_nhwc<Lean19>(a, mode, cus, s);
    default:
      if (cfg >= kWsFirst && cfg < kNumCfg) return launch_wsplit_nhwc(cfg - kWsFirst, a, mode, s);
      return fail(TNH_ERR_UNSUPPORTED, "conv2d: channels-last convolution needs a lean or wave-split tile (11..%d)",
                  kNumCfg - 1);
  }
}

int launch(int cfg, const ConvArgs& a, int mode, bool va, bool vb, int cus, hipStream_t s) {
  switch (cfg) {
    case 0: return launch_cfg<Cfg0>(a, mode, va, vb, s);
    case 1: return launch_cfg<Cfg1>(a, mode, va, vb, s);
    case 2: return launch_cfg<Cfg2>(a, mode, va, vb, s);
    case 3: return launch_cfg<Cfg3>(a, mode, va, vb, s);
    case 4: return launch_cfg<Cfg4>(a, mode, va, vb, s);
    case 5: return launch_cfg<Cfg5>(a, mode, va, vb, s);
    case 11: return launch_lean<Lean11>(a, mode, vb, cus, s);
    case 12: return launch_lean<Lean12>(a, mode, vb, cus, s);
    case 13: return launch_lean<Lean13>(a, mode, vb, cus, s);
    case 14: return launch_lean<Lean14>(a, mode, vb, cus, s);
    case 15: return launch_lean<Lean15>(a, mode, vb, cus, s);
    case 16: return launch_lean<Lean16>(a, mode, vb, cus, s);
    case 17: return launch_lean<Lean17>(a, mode, vb, cus, s);
    case 18: return launch_lean<Lean18>(a, mode, vb, cus, s);
    case 19: return launch_lean<Lean19>(a, mode, vb, cus, s);
    default:
      if (cfg >= kWsFirst && cfg < kNumCfg) return launch_wsplit_nchw(cfg - kWsFirst, a, mode, vb, s);
      return fail(TNH_ERR_UNSUPPORTED, "conv2d: tile configuration %d (0..%d)", cfg, kNumCfg - 1);
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// [F][C][taps] -> [F][taps][C]
// dst[f][t][c] = src[f][c][t] over fc = F*C filter channels: thread q =
// f*C + c reads its `taps` consecutive floats (a wave reads one contiguous
// span) and writes them `C` apart (for each t, consecutive threads write
// consecutive floats).
__global__ void pack_weights_kernel(int64_t fc, int64_t C, int64_t taps, const float* __restrict__ src,
                                    float* __restrict__ dst) {
  for (int64_t q = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; q < fc; q += int64_t(gridDim.x) * blockDim.x) {
    const int64_t f = q / C, c = q - f * C;
    const float* s = src + q * taps;
    float* d = dst + f * C * taps + c;
    for (int64_t t = 0; t < taps; ++t) d[t * C] = s[t];
  }
}

// Both weight copies a training step's convolution needs, from the
// reference weights [F][C][kh][kw] in one pass (thread per (f, c), its taps
// t = ky*kw + kx contiguous): the forward's tap-major [F][kh][kw][C] (when
// tap is not null) and the data gradient's [C][kh][kw][F] with both kernel
// axes flipped: flip[c][taps-1-t][f] = w[f][c][t].  With the flipped copy the
// input delta of a stride-1 convolution is a convolution of the output delta
// (F channels, C filters, padding kh-1-pad).
__global__ void pack_weights_dgrad_kernel(int64_t F, int64_t C, int64_t taps, const float* __restrict__ src,
                                          float* __restrict__ tap, float* __restrict__ flip) {
  const int64_t fc = F * C;
  for (int64_t q = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; q < fc; q += int64_t(gridDim.x) * blockDim.x) {
    const int64_t f = q / C, c = q - f * C;
    const float* s = src + q * taps;
    for (int64_t t = 0; t < taps; ++t) {
      const float v = s[t];
      if (tap) tap[(f * taps + t) * C + c] = v;
      flip[(c * taps + (taps - 1 - t)) * F + f] = v;
    }
  }
}

struct Cand {
  int cfg, splits;
  int tail;   // tail-split pieces per remainder tile (lean configurations), 0: none
  int slots;  // tail split: rounds of every resident workgroup slot (1) or of the CUs (0)
};

// Estimated time (arbitrary units): rounds of resident tiles times the work
// of one tile, divided by the configuration's relative efficiency; split-K
// adds the partial-sum traffic of the reduction.
float cost(const CfgInfo& c, int64_t F, int64_t N, int64_t K, int cus, int splits) {
  const int64_t tiles = ((F + c.BM - 1) / c.BM) * ((N + c.BN - 1) / c.BN) * splits;
  const int64_t slots = static_cast<int64_t>(cus) * c.perCU;
  const int64_t rounds = (tiles + slots - 1) / slots;
  const int64_t kp = ((K + splits - 1) / splits + c.BK - 1) / c.BK * c.BK;
  const float mm = static_cast<float>(rounds) * c.BM * c.BN * static_cast<float>(kp) / (c.eff * c.perCU);
  // ~30 FLOP-units per partial float round trip at this model's scale
  const float red = splits > 1 ? 30.f * static_cast<float>(splits) * F * N / (static_cast<float>(cus) * c.perCU) : 0.f;
  return mm + red;
}

// Everything a cached choice depends on: the GEMM shape, the layout, the
// operand alignment, whether a residual is read, and whether out, residual
// and one split's partial sums lie within 2 GiB (smallIO: the lean kernels
// address them through 2 GiB buffer resources).
struct TuneKey {
  int64_t F, N, K, C, H, W;
  int k, s, mode, va, vb;
  int nhwc, xPix, outPix, resPix;
  int hasRes, smallIO;
  int epi;  // channels-last epilogue variant: 0 plain, 1 upsampled output, 2 yolo head
  bool operator==(const TuneKey& o) const {
    return F == o.F && N == o.N && K == o.K && C == o.C && H == o.H && W == o.W && k == o.k && s == o.s &&
           mode == o.mode && va == o.va && vb == o.vb && nhwc == o.nhwc && xPix == o.xPix && outPix == o.outPix &&
           resPix == o.resPix && hasRes == o.hasRes && smallIO == o.smallIO && epi == o.epi;
  }
};
struct TuneHash {
  size_t operator()(const TuneKey& t) const {
    size_t h = 1469598103934665603ull;
    for (int64_t v : {t.F, t.N, t.K, t.C, t.H, t.W, (int64_t)t.k, (int64_t)t.s, (int64_t)t.mode, (int64_t)t.va,
                      (int64_t)t.vb, (int64_t)t.nhwc, (int64_t)t.xPix, (int64_t)t.outPix, (int64_t)t.resPix,
                      (int64_t)t.hasRes, (int64_t)t.smallIO, (int64_t)t.epi})
      h = (h ^ static_cast<size_t>(v)) * 1099511628211ull;
    return h;
  }
};

std::mutex g_tune_mu;
std::unordered_map<TuneKey, Cand, TuneHash> g_tuned;
bool g_autotune = true;
int g_forced_cfg = -1;

// The wave-split tiles need whole 32-channel panels inside one tap; the
// retired ids take nothing.
bool cfg_valid(int c, int mode, int64_t C, bool va, bool smallIO, bool nhwc = false) {
  if (nhwc) return (kCfgs[c].kind == kLean || kCfgs[c].kind == kWsplit) && smallIO && va && C % kCfgs[c].BK == 0;
  if (kCfgs[c].kind == kWsplit) return (mode == kTap3 || mode == k1x1) && va && smallIO && C % 32 == 0;
  if (kCfgs[c].kind == kLean && !smallIO) return false;
  if (kCfgs[c].kind == kRetired) return false;
  if (kCfgs[c].kind == kLean) return va && (mode == k1x1 || mode == kTap3) && C % kCfgs[c].BK == 0;
  if (mode == kTap3) return C % kCfgs[c].BK == 0;
  return true;
}

// Candidate tile configurations for one convolution call, timed on the
// first call for its shape (and layout), then launched.  fixed: the static
// scratch of the no-allocation entry point (nullptr: the context's growable
// workspace).  With it the call never tunes (a timing graph allocates): it
// runs the forced, the cached or the cost model's choice; a cached choice
// whose split pieces do not fit the array gives way to the cost model's
// (whole K if need be), and only a forced tiling that does not fit fails.
int conv_dispatch(Context* cx, ConvArgs& a, int mode, bool va, bool vb, bool smallIO, bool nhwc, const TuneKey& key,
                  float* fixed = nullptr) {
  const int64_t F = a.F, N = a.g.N, K = a.g.K, C = a.g.C;
  const int kh = key.k, sY = key.s;
  auto tilesOf = [&](const CfgInfo& ci) -> int64_t {
    return nhwc ? ((N + ci.BM - 1) / ci.BM) * ((F + ci.BN - 1) / ci.BN)
                : ((F + ci.BM - 1) / ci.BM) * ((N + ci.BN - 1) / ci.BN);
  };
  // Candidates, first round: every valid tile shape, and for shapes that
  // leave the CUs under-filled also uniform split-K factors.  Second round
  // (timed tuning only): tail splits of the fastest lean shapes whose tiles
  // do not divide into whole rounds.
  const int cus = cx->cu_count;
  const bool det = deterministic();
  std::vector<Cand> cands;
  for (int c = 0; c < kNumCfg; ++c) {
    if (!cfg_valid(c, mode, C, va, smallIO, nhwc)) continue;
    if (kCfgs[c].kind == kWsplit) {
      // whole tiles only; timed, never the cost model's pick, so absent from
      // the deterministic mode's choice; only for layers whose 64x64 tiles
      // leave the GPU under-filled (below two per CU), where they replace a
      // K split and its reduction launch (on larger layers their 32-wide
      // tiles read twice the L2 bytes per FLOP of the lean tiles), and for
      // NCHW layers of at most 32 filters, which fill half of a lean tile's
      // 64 filter rows (config 3's conv2 input delta: 0.3060-0.3074 against
      // 0.3121-0.3138 ms per step)
      const int64_t tiles64 = ((N + 63) / 64) * ((F + 63) / 64);
      const bool narrow = !nhwc && F <= 32;
      if (!det && (tiles64 < 2 * static_cast<int64_t>(cus) || narrow)) cands.push_back({c, 1, 0, 0});
      continue;
    }
    cands.push_back({c, 1, 0, 0});
    const CfgInfo& ci = kCfgs[c];
    const int64_t tiles = tilesOf(ci);
    if (tiles >= 2 * cus || det) continue;
    for (int sp : {2, 4, 8, 16})
      if (tiles * sp <= 8 * cus && K >= static_cast<int64_t>(sp) * ci.BK * 4)
        cands.push_back(nhwc ? Cand{c, 1, sp, 2} : Cand{c, sp, 0, 0});
  }
  auto unitOf = [&](const Cand& c) -> int64_t {
    if (c.slots == 2) return -1;  // every tile cut
    return c.slots ? static_cast<int64_t>(cus) * lean_occupancy(c.cfg, mode, vb, nhwc) : cus;
  };
  auto tailCands = [&](int c, std::vector<Cand>& out) {
    const CfgInfo& ci = kCfgs[c];
    const int64_t tiles = tilesOf(ci);
    for (int sl = 0; sl < 2; ++sl) {
      const int64_t unit = unitOf({c, 1, 2, sl});
      if (tiles <= unit || tiles % unit == 0 || (sl == 1 && unit == cus)) continue;
      for (int tp : {2, 3, 4, 6, 8})
        if (K >= static_cast<int64_t>(tp) * ci.BK * 2) out.push_back({c, 1, tp, sl});
    }
  };
  auto wsFloats = [&](const Cand& c) -> int64_t {
    if (c.tail > 0) {
      const CfgInfo& ci = kCfgs[c.cfg];
      const int64_t unit = unitOf(c);
      const int64_t panels = K / ci.BK, chunk = (panels + c.tail - 1) / c.tail;
      return unit < 0 ? tilesOf(ci) * ((panels + chunk - 1) / chunk) * ci.BM * ci.BN
                      : tail_floats(tilesOf(ci), ci.BM, ci.BN, ci.BK, K, unit, c.tail);
    }
    return c.splits > 1 ? c.splits * F * N : 0;
  };
  auto wsFor = [&](const Cand& c) -> float* {
    const int64_t n = wsFloats(c);
    if (n <= 0) return nullptr;
    if (fixed) return n <= kNoAllocScratchFloats ? fixed : nullptr;
    return static_cast<float*>(workspace(cx, static_cast<size_t>(n) * 4));
  };
  // arrival counters of the in-kernel tail reduction (not for the
  // no-allocation entry point, whose tail splits reduce in a second launch)
  int* counters = fixed ? nullptr : tile_counters(cx);
  auto runOn = [&](const Cand& c, hipStream_t s) -> int {
    ConvArgs b = a;
    b.splits = 1;
    b.tailSplits = 0;
    b.tailUnit = 0;
    b.part = nullptr;
    b.tileCount = nullptr;
    if (c.splits > 1 || c.tail > 0) {
      b.part = wsFor(c);
      if (b.part) {
        b.splits = c.splits;
        b.tailSplits = c.tail;
        b.tailUnit = c.tail > 0 ? static_cast<int>(unitOf(c)) : 0;  // -1: every tile
        b.tileCount = c.tail > 0 ? counters : nullptr;
      }
    }
    return nhwc ? launch_nhwc_cfg(c.cfg, b, mode, cus, s) : launch(c.cfg, b, mode, va, vb, cus, s);
  };
  Cand best = cands[0];
  {
    float bc = 1e30f;
    for (const Cand& c : cands) {
      if (kCfgs[c.cfg].kind == kWsplit) continue;
      const float v = cost(kCfgs[c.cfg], F, N, K, cx->cu_count, c.splits);
      if (v < bc) bc = v, best = c;
    }
  }
  const Cand model = best;  // the cost model's choice (timed tuning may replace `best`)
  // forced: a tiling the caller chose with tnh_conv2d_set_autotune
  auto run = [&](const Cand& c, bool forced = false) -> int {
    if (fixed && wsFloats(c) > kNoAllocScratchFloats) {
      if (forced)
        return fail(TNH_ERR_INVALID_ARG,
                    "conv2d_nhwc_noalloc: the forced tiling needs %lld bytes of scratch, the static scratch holds "
                    "%lld (split the batch, or force another tiling with tnh_conv2d_set_autotune)",
                    (long long)(wsFloats(c) * 4), (long long)(kNoAllocScratchFloats * 4));
      // a tiling tuned by the allocating entry point whose split pieces do
      // not fit the static scratch: the cost model's choice instead, whose
      // pieces (if it splits and they do not fit either) runOn drops for a
      // whole-K launch of the same tile
      return runOn(model, cx->stream);
    }
    return runOn(c, cx->stream);
  };
  bool tune = false;
  const bool aliased = a.res && a.res == a.out;  // in-place add: reruns would accumulate
  {
    std::lock_guard<std::mutex> lk(g_tune_mu);
    if (g_forced_cfg >= 0 && cfg_valid(g_forced_cfg % 64, mode, C, va, smallIO, nhwc)) {
      const int c = g_forced_cfg % 64, hi = g_forced_cfg / 64;
      if (hi > 16 && kCfgs[c].kind != kLean) return fail(TNH_ERR_UNSUPPORTED, "conv2d: tail split of a non-lean tile");
      if (hi > 1 && kCfgs[c].kind == kWsplit) return fail(TNH_ERR_UNSUPPORTED, "conv2d: split of a wave-split tile");
      if (nhwc && hi >= 2 && hi <= 16) return run({c, 1, hi, 2}, true);  // split-K: every tile cut
      if (hi >= 34) return run({c, 1, hi - 32, 1}, true);
      if (hi >= 18) return run({c, 1, hi - 16, 0}, true);
      return run({c, hi > 1 ? hi : 1, 0, 0}, true);
    }
    if (det) return run(best);  // the cost model's whole-K choice: the same in every process
    auto it = g_tuned.find(key);
    if (it != g_tuned.end() && cfg_valid(it->second.cfg, mode, C, va, smallIO, nhwc)) return run(it->second);
    if (g_autotune && !aliased && !fixed) {
      hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
      if (hipStreamIsCapturing(cx->stream, &cs) == hipSuccess && cs == hipStreamCaptureStatusNone) tune = true;
    }
  }
  if (tune) {
    // Time each candidate as it runs in a graph replay (time_graph).  Eager
    // timing would charge a candidate the host's launch cost, which at small
    // sizes exceeds the kernels' own time and penalises split-K's second
    // launch.  The output is rewritten identically by every run (out never
    // aliases x or residual).  Workspaces are grown before any capture.
    constexpr int kReps = 4;
    if (int st = hip_status(hipStreamSynchronize(cx->stream), "hipStreamSynchronize")) return st;
    auto timeCand = [&](const Cand& c, float& ms) -> int {
      return time_graph(cx, [&](hipStream_t s) { return runOn(c, s); }, kReps, ms);
    };
    // times a list of candidates; returns the per-candidate times
    float bestMs = 1e30f;
    auto timeAll = [&](const std::vector<Cand>& list, std::vector<float>& times) -> int {
      int64_t maxWs = 0;
      Cand maxC{0, 1, 0, 0};
      for (const Cand& c : list)
        if (wsFloats(c) > maxWs) maxWs = wsFloats(c), maxC = c;
      if (maxWs > 0) (void)wsFor(maxC);
      times.assign(list.size(), 1e30f);
      // TNH_VERBOSE=2: every candidate's time
      static const bool all = std::getenv("TNH_VERBOSE") && std::atoi(std::getenv("TNH_VERBOSE")) >= 2;
      for (size_t i = 0; i < list.size(); ++i) {
        const Cand& c = list[i];
        if ((c.splits > 1 || c.tail > 0) && !wsFor(c)) continue;
        if (int st = timeCand(c, times[i])) return st;
        if (times[i] < bestMs) bestMs = times[i], best = c;
        if (all)
          std::fprintf(stderr, "[tnh]   candidate cfg %d split %d tail %d%s: %.4f ms\n", c.cfg, c.splits, c.tail,
                       c.slots == 1 ? "/slots" : (c.slots == 2 ? "/all" : ""), times[i]);
      }
      return TNH_OK;
    };
    std::vector<float> times;
    int st = timeAll(cands, times);
    if (!st) {
      // tail splits of the three fastest whole-K lean candidates
      std::vector<size_t> order;
      for (size_t i = 0; i < cands.size(); ++i)
        if (kCfgs[cands[i].cfg].kind == kLean && cands[i].splits == 1 && cands[i].tail == 0) order.push_back(i);
      std::sort(order.begin(), order.end(), [&](size_t x, size_t y) { return times[x] < times[y]; });
      std::vector<Cand> second;
      for (size_t r = 0; r < order.size() && r < 3; ++r) tailCands(cands[order[r]].cfg, second);
      std::vector<float> t2;
      st = timeAll(second, t2);
    }
    if (st) return st;
    std::lock_guard<std::mutex> lk(g_tune_mu);
    g_tuned[key] = best;
    static const bool verbose = std::getenv("TNH_VERBOSE") != nullptr;
    if (verbose)
      std::fprintf(stderr,
                   "[tnh] conv F=%lld N=%lld K=%lld k=%lld s=%lld mode=%d -> cfg %d (%dx%dx%d) split %d tail %d%s "
                   "%.4f ms\n",
                   (long long)F, (long long)N, (long long)K, (long long)kh, (long long)sY, mode, best.cfg,
                   kCfgs[best.cfg].BM, kCfgs[best.cfg].BN, kCfgs[best.cfg].BK, best.splits, best.tail,
                   best.slots ? "/slots" : "", bestMs);
  }
  return run(best);
}

}  // namespace
}  // namespace conv
}  // namespace tnh

using namespace tnh;
using namespace tnh::conv;

namespace {

// Epilogue variant of a channels-last call (ConvArgs::upS / yolo).
struct NhwcEpi {
  int64_t upS = 0;
  float upScale = 1.f;
  float* yolo = nullptr;
  int64_t yoloN = 0, yoloClasses = 0;
};

// tnh_conv2d_fwd_nhwc, its no-allocation variant (noAlloc: split pieces in
// the device's static scratch, no autotuning) and its upsample / yolo
// epilogue variants.
int conv_nhwc_entry(int64_t batch, int64_t C, int64_t H, int64_t W, int64_t F, int64_t kh, int64_t kw, int64_t pH,
                    int64_t pW, int64_t sY, int64_t sX, const float* x, int64_t xOff, int64_t xPix,
                    const float* weights, int64_t wOff, const float* bias, int64_t biasOff, int32_t act,
                    const float* residual, int64_t rOff, int64_t rPix, float* out, int64_t outOff, int64_t outPix,
                    bool noAlloc, const NhwcEpi& epi = NhwcEpi{}) {
  TNH_REQUIRE_CTX(cx);
  float* fixed = nullptr;
  if (noAlloc) {
    fixed = scratch_for(cx->device);
    if (!fixed) return fail(TNH_ERR_NOT_INITIALIZED, "conv2d_nhwc_noalloc: no static scratch on device %d", cx->device);
  }
  TNH_ARG(batch >= 0 && C > 0 && H > 0 && W > 0 && F > 0, "conv2d_nhwc: bad sizes");
  TNH_ARG(kh == kw && (kh == 1 || kh == 3), "conv2d_nhwc: only square 1x1 / 3x3 kernels are supported");
  TNH_ARG(sY > 0 && sX > 0 && pH >= 0 && pW >= 0, "conv2d_nhwc: bad stride/pad");
  TNH_ARG(x && weights && out, "conv2d_nhwc: NULL x/weights/out");
  TNH_ARG(act == TNH_AC_LINEAR || act == TNH_AC_LEAKY || act == TNH_AC_LOGISTIC, "conv2d_nhwc: activation %d", act);
  TNH_ARG(xOff >= 0 && wOff >= 0 && outOff >= 0 && biasOff >= 0 && rOff >= 0, "conv2d_nhwc: negative offset");
  const bool xNchw = xPix == 0;  // the network's NCHW image, few-channel 3x3 only
  TNH_ARG(xNchw ? (kh == 3 && C <= 4) : xPix >= C, "conv2d_nhwc: xPix %lld (C %lld)", (long long)xPix,
          (long long)C);
  TNH_ARG(outPix >= F && (!residual || rPix >= F), "conv2d_nhwc: pixel stride below the filter count");
  const int64_t OH = (H + 2 * pH - kh) / sY + 1, OW = (W + 2 * pW - kw) / sX + 1;
  TNH_ARG(OH > 0 && OW > 0, "conv2d_nhwc: empty output");
  TNH_ARG(kh == 3 || (sY == 1 && sX == 1 && pH == 0 && pW == 0), "conv2d_nhwc: 1x1 needs stride 1, no padding");
  const bool variant = epi.upS > 0 || epi.yolo;
  TNH_ARG(!variant || (!xNchw && !residual), "conv2d_nhwc: an upsampled or yolo output takes no residual and "
                                             "no NCHW image");
  TNH_ARG(epi.upS >= 0 && epi.upS <= 16, "conv2d_nhwc_upsample: stride %lld (1..16)", (long long)epi.upS);
  TNH_ARG(!epi.yolo || (epi.yoloN > 0 && epi.yoloClasses >= 0 && F == epi.yoloN * (epi.yoloClasses + 5)),
          "conv2d_nhwc_yolo: %lld filters for %lld anchors x (5 + %lld classes)", (long long)F, (long long)epi.yoloN,
          (long long)epi.yoloClasses);
  if (batch == 0) return TNH_OK;
  const int64_t K = C * kh * kw, N = batch * OH * OW;
  const int64_t xElems = xNchw ? batch * C * H * W : (batch * H * W - 1) * xPix + C;
  TNH_ARG(xElems * 4 <= kMaxBufBytes, "conv2d_nhwc: input spans more than 2 GiB (split the batch)");
  TNH_ARG(F * K * 4 <= kMaxBufBytes && OH * OW < (int64_t(1) << 31), "conv2d_nhwc: tensor too large");

  ConvArgs a{};
  a.g.x = x + xOff;
  a.g.xBytes = xElems * 4;
  a.g.xBatchStride = xNchw ? C * H * W : H * W * xPix;
  a.g.C = (int)C; a.g.H = (int)H; a.g.W = (int)W; a.g.OW = (int)OW; a.g.OHW = (int)(OH * OW);
  a.g.sY = (int)sY; a.g.sX = (int)sX; a.g.pH = (int)pH; a.g.pW = (int)pW;
  a.g.N = N; a.g.K = K;
  a.w = weights + wOff;
  a.wBytes = F * K * 4;
  a.bias = bias ? bias + biasOff : nullptr;
  a.res = residual ? residual + rOff : nullptr;
  a.out = out + outOff;
  a.F = F;
  a.act = act;
  a.xPix = (int)xPix;
  a.outPix = (int)outPix;
  a.resPix = residual ? (int)rPix : 0;
  a.outBatchStride = OH * OW * outPix;
  a.rBatchStride = residual ? OH * OW * rPix : 0;
  a.outBytes = ((N - 1) * outPix + F) * 4;
  a.resBytes = residual ? ((N - 1) * rPix + F) * 4 : 0;
  if (epi.upS > 0) {  // out is the upsampled image
    a.upS = static_cast<int>(epi.upS);
    a.upScale = epi.upScale;
    a.outBatchStride = OH * OW * epi.upS * epi.upS * outPix;
    a.outBytes = ((N * epi.upS * epi.upS - 1) * outPix + F) * 4;
  }
  if (epi.yolo) {
    a.yolo = epi.yolo;
    a.yoloEntries = static_cast<int>(epi.yoloClasses + 5);
    a.yoloBytes = N * F * 4 <= kMaxBufBytes ? N * F * 4 : 0;
    a.yoloVec = (OH * OW) % 4 == 0 && aligned16(epi.yolo);
  }
  // The network's first layer: on the matrix cores from about 32 blocks of
  // 32 pixels per CU (YOLOv3-416 from batch 2: measured 23.7 against 25.0 us
  // at batch 2, 111 against 135 us at batch 16), else the bit-exact
  // per-pixel kernel, which wins at batch 1 (13.0 against 17.1 us: one
  // block per wave leaves the MFMA kernel's loads exposed) and serves a
  // residual, F > 64 and F % 4 != 0.
  if (xNchw)
    return first_mfma_ok(a) && a.g.N >= int64_t(32) * 32 * cx->cu_count ? launch_first_mfma(a, cx->stream)
                                                                        : launch_smallc<true, true>(a, cx->stream);

  const int mode = kh == 3 ? kTap3 : k1x1;
  const bool va = aligned16(a.w) && K % 4 == 0 && aligned16(a.g.x) && xPix % 4 == 0;
  const bool smallIO = a.outBytes <= kMaxBufBytes && a.resBytes <= kMaxBufBytes;
  TNH_ARG(va && smallIO && C % 4 == 0,
          "conv2d_nhwc: needs C %% 4 == 0, 16-byte aligned x and weights with xPix %% 4 == 0, out within 2 GiB");
  if (C % 32 != 0) return launch_nhwc_any(a, kh == 3 ? kTap3Any : k1x1Any, cx->stream);
  const TuneKey key{F, N, K, C, H, W, (int)kh, (int)sY, mode, va, false, 1, (int)xPix, (int)outPix,
                    residual ? (int)rPix : 0, residual != nullptr, smallIO, epi.upS > 0 ? 1 : (epi.yolo ? 2 : 0)};
  return conv_dispatch(cx, a, mode, va, false, smallIO, true, key, fixed);
}

}  // namespace

extern "C" int32_t tnh_conv2d_fwd_nhwc(int64_t batch, int64_t C, int64_t H, int64_t W, int64_t F, int64_t kh,
                                       int64_t kw, int64_t pH, int64_t pW, int64_t sY, int64_t sX, const float* x,
                                       int64_t xOff, int64_t xPix, const float* weights, int64_t wOff,
                                       const float* bias, int64_t biasOff, int32_t act, const float* residual,
                                       int64_t rOff, int64_t rPix, float* out, int64_t outOff, int64_t outPix) {
  return conv_nhwc_entry(batch, C, H, W, F, kh, kw, pH, pW, sY, sX, x, xOff, xPix, weights, wOff, bias, biasOff, act,
                         residual, rOff, rPix, out, outOff, outPix, false);
}

extern "C" int32_t tnh_conv2d_fwd_nhwc_noalloc(int64_t batch, int64_t C, int64_t H, int64_t W, int64_t F,
                                               int64_t kh, int64_t kw, int64_t pH, int64_t pW, int64_t sY,
                                               int64_t sX, const float* x, int64_t xOff, int64_t xPix,
                                               const float* weights, int64_t wOff, const float* bias,
                                               int64_t biasOff, int32_t act, const float* residual, int64_t rOff,
                                               int64_t rPix, float* out, int64_t outOff, int64_t outPix) {
  return conv_nhwc_entry(batch, C, H, W, F, kh, kw, pH, pW, sY, sX, x, xOff, xPix, weights, wOff, bias, biasOff, act,
                         residual, rOff, rPix, out, outOff, outPix, true);
}

extern "C" int32_t tnh_conv2d_fwd_nhwc_upsample(int64_t batch, int64_t C, int64_t H, int64_t W, int64_t F,
                                                int64_t kh, int64_t kw, int64_t pH, int64_t pW, int64_t sY,
                                                int64_t sX, const float* x, int64_t xOff, int64_t xPix,
                                                const float* weights, int64_t wOff, const float* bias,
                                                int64_t biasOff, int32_t act, int64_t upStride, float upScale,
                                                float* out, int64_t outOff, int64_t outPix) {
  TNH_ARG(upStride >= 1, "conv2d_nhwc_upsample: stride %lld", (long long)upStride);
  NhwcEpi e;
  e.upS = upStride;
  e.upScale = upScale;
  return conv_nhwc_entry(batch, C, H, W, F, kh, kw, pH, pW, sY, sX, x, xOff, xPix, weights, wOff, bias, biasOff, act,
                         nullptr, 0, 0, out, outOff, outPix, false, e);
}

extern "C" int32_t tnh_conv2d_fwd_nhwc_yolo(int64_t batch, int64_t C, int64_t H, int64_t W, int64_t F, int64_t kh,
                                            int64_t kw, int64_t pH, int64_t pW, int64_t sY, int64_t sX,
                                            const float* x, int64_t xOff, int64_t xPix, const float* weights,
                                            int64_t wOff, const float* bias, int64_t biasOff, int32_t act,
                                            float* out, int64_t outOff, int64_t outPix, int64_t n, int64_t classes,
                                            float* yoloOut, int64_t yoloOff) {
  TNH_ARG(yoloOut != nullptr && yoloOff >= 0, "conv2d_nhwc_yolo: NULL head or negative offset");
  NhwcEpi e;
  e.yolo = yoloOut + yoloOff;
  e.yoloN = n;
  e.yoloClasses = classes;
  return conv_nhwc_entry(batch, C, H, W, F, kh, kw, pH, pW, sY, sX, x, xOff, xPix, weights, wOff, bias, biasOff, act,
                         nullptr, 0, 0, out, outOff, outPix, false, e);
}

extern "C" int32_t tnh_conv2d_noalloc_scratch_bytes(int64_t* bytes) {
  TNH_ARG(bytes != nullptr, "conv2d_noalloc_scratch_bytes: NULL");
  *bytes = kNoAllocScratchFloats * 4;
  return TNH_OK;
}

extern "C" int32_t tnh_conv2d_out_dims(int64_t H, int64_t W, int64_t kh, int64_t kw, int64_t pH, int64_t pW,
                                       int64_t sY, int64_t sX, int64_t* OH, int64_t* OW) {
  TNH_ARG(OH && OW, "conv2d_out_dims: NULL output");
  TNH_ARG(kh > 0 && kw > 0 && sY > 0 && sX > 0 && pH >= 0 && pW >= 0, "conv2d_out_dims: bad geometry");
  *OH = (H + 2 * pH - kh) / sY + 1;
  *OW = (W + 2 * pW - kw) / sX + 1;
  return TNH_OK;
}

extern "C" int32_t tnh_conv2d_set_autotune(int32_t enable, int32_t forcedConfig) {
  std::lock_guard<std::mutex> lk(g_tune_mu);
  TNH_ARG(forcedConfig >= -1 && forcedConfig % 64 < kNumCfg && forcedConfig / 64 <= 47 &&
              forcedConfig / 64 != 17 && forcedConfig / 64 != 32 && forcedConfig / 64 != 33,
          "conv2d_set_autotune: config %d", forcedConfig);
  TNH_ARG(forcedConfig < 0 || kCfgs[forcedConfig % 64].kind != kRetired,
          "conv2d_set_autotune: tile %d is retired (ids 6..10)", forcedConfig % 64);
  g_autotune = enable != 0;
  g_forced_cfg = forcedConfig;
  if (!g_autotune) g_tuned.clear();
  return TNH_OK;
}

extern "C" int32_t tnh_conv2d_pack_weights(int64_t F, int64_t C, int64_t kh, int64_t kw, const float* src,
                                           float* dst) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(F > 0 && C > 0 && kh > 0 && kw > 0 && src && dst && src != dst, "conv2d_pack_weights: bad arguments");
  const int64_t blocks = (F * C + 255) / 256;
  hipLaunchKernelGGL(pack_weights_kernel, dim3(static_cast<unsigned>(blocks < 65536 ? blocks : 65536)), dim3(256), 0,
                     cx->stream, F * C, C, kh * kw, src, dst);
  return launch_status("pack_weights_kernel");
}

extern "C" int32_t tnh_conv2d_pack_weights_dgrad(int64_t F, int64_t C, int64_t kh, int64_t kw, const float* src,
                                                 float* tapMajor, float* flipped) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(F > 0 && C > 0 && kh > 0 && kw > 0 && src && flipped && src != flipped && src != tapMajor &&
              tapMajor != flipped,
          "conv2d_pack_weights_dgrad: bad arguments");
  const int64_t blocks = (F * C + 255) / 256;
  hipLaunchKernelGGL(pack_weights_dgrad_kernel, dim3(static_cast<unsigned>(blocks < 65536 ? blocks : 65536)),
                     dim3(256), 0, cx->stream, F, C, kh * kw, src, tapMajor, flipped);
  return launch_status("pack_weights_dgrad_kernel");
}

extern "C" int32_t tnh_conv2d_fwd(int64_t batch, int64_t C, int64_t H, int64_t W, int64_t F, int64_t kh,
                                  int64_t kw, int64_t pH, int64_t pW, int64_t sY, int64_t sX, const float* x,
                                  int64_t xOff, int64_t xBatchStride, const float* weights, int64_t wOff,
                                  int32_t weightLayout, const float* bias, int64_t biasOff, int32_t act,
                                  const float* residual, int64_t rOff, int64_t rBatchStride, float* out,
                                  int64_t outOff, int64_t outBatchStride) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(batch >= 0 && C > 0 && H > 0 && W > 0 && F > 0, "conv2d: bad sizes");
  TNH_ARG(kh >= 1 && kw >= 1 && kh <= 32 && kw <= 32, "conv2d: kernel %lldx%lld (1..32 per side)", (long long)kh,
          (long long)kw);
  TNH_ARG(sY > 0 && sX > 0 && pH >= 0 && pW >= 0, "conv2d: bad stride/pad");
  TNH_ARG(x && weights && out, "conv2d: NULL x/weights/out");
  TNH_ARG(weightLayout == TNH_WEIGHTS_REFERENCE || weightLayout == TNH_WEIGHTS_TAP_MAJOR,
          "conv2d: weight layout %d", weightLayout);
  TNH_ARG(act == TNH_AC_LINEAR || act == TNH_AC_LEAKY || act == TNH_AC_LOGISTIC, "conv2d: activation %d", act);
  TNH_ARG(xOff >= 0 && wOff >= 0 && outOff >= 0 && biasOff >= 0 && rOff >= 0, "conv2d: negative offset");
  const int64_t OH = (H + 2 * pH - kh) / sY + 1, OW = (W + 2 * pW - kw) / sX + 1;
  TNH_ARG(OH > 0 && OW > 0, "conv2d: empty output");
  TNH_ARG(xBatchStride >= C * H * W || batch <= 1, "conv2d: xBatchStride too small");
  TNH_ARG(outBatchStride >= F * OH * OW || batch <= 1, "conv2d: outBatchStride too small");
  TNH_ARG(!residual || rBatchStride >= F * OH * OW || batch <= 1, "conv2d: rBatchStride too small");
  if (batch == 0) return TNH_OK;
  const int64_t K = C * kh * kw, N = batch * OH * OW;
  const int64_t xElems = (batch - 1) * xBatchStride + C * H * W;
  TNH_ARG(xElems * 4 <= kMaxBufBytes, "conv2d: input spans more than 2 GiB (split the batch)");
  TNH_ARG(F * K * 4 <= kMaxBufBytes && OH * OW < (int64_t(1) << 31), "conv2d: tensor too large");

  ConvArgs a{};
  a.g.x = x + xOff;
  a.g.xBytes = xElems * 4;
  a.g.xBatchStride = xBatchStride;
  a.g.C = (int)C; a.g.H = (int)H; a.g.W = (int)W; a.g.OW = (int)OW; a.g.OHW = (int)(OH * OW);
  a.g.sY = (int)sY; a.g.sX = (int)sX; a.g.pH = (int)pH; a.g.pW = (int)pW;
  a.g.N = N; a.g.K = K;
  a.g.kh = (int)kh; a.g.kw = (int)kw;
  a.g.tapW = weightLayout == TNH_WEIGHTS_TAP_MAJOR;
  a.w = weights + wOff;
  a.wBytes = F * K * 4;
  a.bias = bias ? bias + biasOff : nullptr;
  a.res = residual ? residual + rOff : nullptr;
  a.rBatchStride = rBatchStride;
  a.out = out + outOff;
  a.outBatchStride = outBatchStride;
  a.outBytes = ((batch - 1) * outBatchStride + F * OH * OW) * 4;
  a.resBytes = residual ? ((batch - 1) * rBatchStride + F * OH * OW) * 4 : 0;
  a.F = F;
  a.act = act;

  const bool is1x1 = kh == 1 && kw == 1 && sY == 1 && sX == 1 && pH == 0 && pW == 0;
  int mode;
  if (is1x1)
    mode = k1x1;  // both layouts coincide for 1x1
  else if (kh == 1 && kw == 1)
    mode = kGatherRef1;
  else if (kh != 3 || kw != 3)
    mode = kGatherDyn;  // any other kernel size: the LDS-staged tiles with a run-time gather
  else if (weightLayout == TNH_WEIGHTS_TAP_MAJOR)
    mode = C % 16 == 0 ? kTap3 : kGatherTap3;
  else
    mode = kGatherRef3;
  bool forced;
  {
    std::lock_guard<std::mutex> lk(g_tune_mu);
    forced = g_forced_cfg >= 0;
  }
  if (mode == kGatherRef3 && C % 16 == 0 && !forced) {
    // Reference-layout 3x3 weights (as TConvolutionalLayer stores them): the
    // call repacks them tap-major into the stream's packing buffer (one
    // F*K-float read and write, in order before the convolution on the same
    // stream) and runs the tap-major tiles, which read whole 16-channel
    // chunks of one tap per panel.  Nothing is cached, so weights updated
    // between calls need no notice.  Without the buffer (a stream captured
    // before any eager call) the LDS-staged reference-layout tiles run.
    if (float* pk = static_cast<float*>(pack_buffer(cx, static_cast<size_t>(F * K) * 4))) {
      const int64_t blocks = (F * C + 255) / 256;
      hipLaunchKernelGGL(pack_weights_kernel, dim3(static_cast<unsigned>(blocks < 65536 ? blocks : 65536)),
                         dim3(256), 0, cx->stream, F * C, C, kh * kw, a.w, pk);
      if (int st = launch_status("pack_weights_kernel")) return st;
      a.w = pk;
      a.g.tapW = true;
      mode = kTap3;
    }
  }
  const bool va = aligned16(a.w) && K % 4 == 0;
  // the buffer-store epilogue of the lean kernels addresses out, residual and
  // one split's partial sums through 2 GiB buffer resources
  const bool smallIO = a.outBytes <= kMaxBufBytes && a.resBytes <= kMaxBufBytes && F * N * 4 <= kMaxBufBytes;
  const bool vb = is1x1 && aligned16(a.g.x) && (OH * OW) % 4 == 0 && (batch == 1 || xBatchStride % 4 == 0);
  if (mode == kTap3 && !va) mode = kGatherTap3;
  if (kh == 3 && kw == 3 && C <= 4 && N / 256 < INT32_MAX) {
    // few input channels: per-pixel kernel (no tile choice to tune); a forced
    // tile configuration still selects the GEMM path (tests of every tile)
    if (!forced)
      return weightLayout == TNH_WEIGHTS_TAP_MAJOR ? launch_smallc<true, false>(a, cx->stream)
                                                   : launch_smallc<false, false>(a, cx->stream);
  }

  const TuneKey key{F, N, K, C, H, W, (int)kh, (int)sY, mode, va, vb, 0, 0, 0, 0, residual != nullptr, smallIO};
  return conv_dispatch(cx, a, mode, va, vb, smallIO, false, key);
}
