// Row-major fp32 SGEMM on MFMA: C = alpha*op(A)*op(B) + beta*C for the four
// NN/NT/TN/TT variants and strided batches.  Replaces TNNCuda.gemm /
// gemmStridedBatched (nncuda.pas:624, 809) and the CPU cblas_sgemm
// (ntensors.pas:2231-2304).
#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <mutex>
#include <unordered_map>
#include <vector>

#include "common.hpp"
#include "conv_lean.hpp"
#include "conv_wsplit.hpp"
#include "gemm_core.hpp"
#include "wave_panels.hpp"

namespace tnh {
namespace {

struct SgemmArgs {
  const float* A;
  const float* B;
  float* C;
  int64_t M, N, K, lda, ldb, ldc;
  int64_t strideA, strideB, strideC;
  int64_t aBytes, bBytes;  // extent of one batch item of A / B
  int64_t cBytes;          // extent of one batch item of C
  float alpha, beta;
  int tilesM, tilesN;
};

template <class Cfg, bool TA, bool TB, bool VA, bool VB>
__global__ __launch_bounds__(Cfg::NT) void sgemm_kernel(SgemmArgs a) {
  using AL = DenseLoader<!TA, VA, Cfg::BM, Cfg::BK, Cfg::NT>;
  using BL = DenseLoader<TB, VB, Cfg::BN, Cfg::BK, Cfg::NT>;
  using Main = GemmMainloop<Cfg, AL, BL>;
  __shared__ __attribute__((aligned(16))) float smem[Main::LDS_FLOATS];
  lds_t* lds = (lds_t*)smem;

  const int64_t bz = blockIdx.y;
  int tm, tn;
  tile_coords(blockIdx.x, a.tilesM, a.tilesN, tm, tn);
  const int64_t m0 = static_cast<int64_t>(tm) * Cfg::BM, n0 = static_cast<int64_t>(tn) * Cfg::BN;

  AL al;
  al.init(a.A + bz * a.strideA, a.aBytes, a.lda, a.M, a.K, m0, threadIdx.x);
  BL bl;
  bl.init(a.B + bz * a.strideB, a.bBytes, a.ldb, a.N, a.K, n0, threadIdx.x);

  f32x16 acc[Cfg::FM][Cfg::FN];
  Main::exec(al, bl, 0, a.K, lds, acc);

  float* C = a.C + bz * a.strideC;
  const float alpha = a.alpha, beta = a.beta;
  Main::for_each(acc, [&](int row, int col, float v) {
    const int64_t gr = m0 + row, gc = n0 + col;
    if (gr < a.M && gc < a.N) {
      float* p = C + gr * a.ldc + gc;
      float out = alpha * v;
      if (beta != 0.f) out = out + beta * *p;
      *p = out;
    }
  });
}

using Cfg128 = TileCfg<128, 128, 16, 2, 2, 1>;
using Cfg64 = TileCfg<64, 64, 32, 2, 2, 2>;

// Lean SGEMM (conv_lean.hpp's pipeline: swizzled k-contiguous LDS panels,
// per-lane offsets fixed for the whole K loop, one barrier per 32-deep
// panel).  A not transposed and B transposed are k-contiguous operands
// (16-byte loads along k); A transposed and B not transposed are
// row-contiguous (4x4 blocks of 16-byte loads, transposed into LDS).  Needs
// K % 32 == 0, 16-byte aligned operands with ld % 4 == 0, and the extent of
// every row-contiguous operand (M or N) a multiple of 4; C, like every
// operand, within 2 GiB.
// Row-contiguous loader of ROWS rows: 4x4 vector blocks when they tile the
// panel exactly with the workgroup's threads, else one row per thread.
template <class Cfg, int ROWS>
using LeanMN = conv::LeanRowsMN<ROWS, Cfg::BK, Cfg::NT, (Cfg::BK / 4) % (Cfg::NT / (ROWS / 4)) == 0>;

template <class Cfg, bool TA, bool TB>
__global__ __launch_bounds__(Cfg::NT, Cfg::OCC) void sgemm_lean_kernel(SgemmArgs a) {
  using AL = typename std::conditional<TA, LeanMN<Cfg, Cfg::BM>, conv::LeanRowsK<Cfg::BM, Cfg::BK, Cfg::NT>>::type;
  using BL = typename std::conditional<TB, conv::LeanRowsK<Cfg::BN, Cfg::BK, Cfg::NT>, LeanMN<Cfg, Cfg::BN>>::type;
  using Loop = conv::LeanLoop<Cfg, AL, BL>;
  __shared__ __attribute__((aligned(16))) float smem[Loop::LDS_FLOATS];
  lds_t* lds = (lds_t*)smem;

  const int64_t bz = blockIdx.y;
  int tm, tn;
  tile_coords(blockIdx.x, a.tilesM, a.tilesN, tm, tn);
  const int64_t m0 = static_cast<int64_t>(tm) * Cfg::BM, n0 = static_cast<int64_t>(tn) * Cfg::BN;
  AL al;
  al.init(a.A + bz * a.strideA, a.aBytes, a.lda, a.M, m0, threadIdx.x);
  BL bl;
  bl.init(a.B + bz * a.strideB, a.bBytes, a.ldb, a.N, n0, threadIdx.x);
  f32x16 acc[Cfg::FM][Cfg::FN];
  Loop::exec(al, bl, 0, a.K / Cfg::BK, lds, acc);

  // C = alpha*acc (+ beta*C): lane columns n, wave-uniform row offsets in the
  // scalar operand, out-of-range elements at kOOB (dropped); every C load is
  // issued before the first store.
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave / Cfg::WN, wn = wave % Cfg::WN;
  const int64_t m0w = m0 + wm * Cfg::WTM, n0w = n0 + wn * Cfg::WTN;
  const int h = lane >> 5;
  const int rowBase = static_cast<int>(m0w) + 4 * h;
  const bool allRows = m0w + Cfg::FM * 32 <= a.M;
  const uint32_t ldc4 = static_cast<uint32_t>(a.ldc) * 4u;
  const __amdgpu_buffer_rsrc_t cR = make_rsrc(a.C + bz * a.strideC, a.cBytes);
  uint32_t vo[Cfg::FN];
#pragma unroll
  for (int j = 0; j < Cfg::FN; ++j) {
    const int64_t n = n0w + j * 32 + (lane & 31);
    vo[j] = sel_off(n < a.N, static_cast<uint32_t>(rowBase) * ldc4 + static_cast<uint32_t>(n) * 4u);
  }
  auto rowOff = [&](int i, int r) { return static_cast<uint32_t>(i * 32 + 8 * (r >> 2) + (r & 3)); };
  auto off = [&](int i, int j, int r) {
    return allRows || rowBase + static_cast<int>(rowOff(i, r)) < a.M ? vo[j] : kOOB;
  };
  const float alpha = a.alpha, beta = a.beta;
  if (beta != 0.f) {
    float cv[Cfg::FM][Cfg::FN][16];
#pragma unroll
    for (int i = 0; i < Cfg::FM; ++i)
#pragma unroll
      for (int j = 0; j < Cfg::FN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) cv[i][j][r] = buf_ld1s(cR, off(i, j, r), rowOff(i, r) * ldc4);
#pragma unroll
    for (int i = 0; i < Cfg::FM; ++i)
#pragma unroll
      for (int j = 0; j < Cfg::FN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          conv::buf_st1s(cR, alpha * acc[i][j][r] + beta * cv[i][j][r], off(i, j, r), rowOff(i, r) * ldc4);
  } else {
#pragma unroll
    for (int i = 0; i < Cfg::FM; ++i)
#pragma unroll
      for (int j = 0; j < Cfg::FN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) conv::buf_st1s(cR, alpha * acc[i][j][r], off(i, j, r), rowOff(i, r) * ldc4);
  }
}

// Wave-split SGEMM for problems whose lean tiles leave CUs idle (512^3 has
// 64 tiles of 64x64 for 256 CUs): one (32*FM) x (32*FN) tile per workgroup,
// its K range split over the W waves (conv_wsplit.hip's scheme: each wave
// fetches its own panels into its own LDS panel, no barrier in the K loop),
// the W partial tiles summed in wave order through LDS, then alpha / beta.
// Same operand requirements as the lean tiles.
template <class Cfg, bool TA, bool TB>
__global__ __launch_bounds__(Cfg::NT) void sgemm_wsplit_kernel(SgemmArgs a) {
  constexpr int FM = Cfg::FM, FN = Cfg::FN, W = Cfg::W, UNITS = Cfg::UNITS;
  using AL = typename std::conditional<TA, conv::WaveRowsMN<32 * FM>, conv::WaveRowsK<32 * FM>>::type;
  using BL = typename std::conditional<TB, conv::WaveRowsK<32 * FN>, conv::WaveRowsMN<32 * FN>>::type;
  using Pan = conv::LeanCfg<32 * FM, 32 * FN, 32, 1, 1, 1>;
  using Loop = conv::LeanLoop<Pan, AL, BL>;
  constexpr int STAGE = AL::SIZE + BL::SIZE;
  constexpr int LDS = W * STAGE > Cfg::RED_FLOATS ? W * STAGE : Cfg::RED_FLOATS;
  __shared__ __attribute__((aligned(16))) float smem[LDS];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane & 31, h = lane >> 5;
  const int64_t bz = blockIdx.y;
  int tm, tn;
  tile_coords(blockIdx.x, a.tilesM, a.tilesN, tm, tn);
  const int64_t m0 = static_cast<int64_t>(tm) * Cfg::BM, n0 = static_cast<int64_t>(tn) * Cfg::BN;

  AL a0, a1;
  BL b0, b1;
  a0.init(a.A + bz * a.strideA, a.aBytes, a.lda, a.M, m0, lane);
  a1.init(a.A + bz * a.strideA, a.aBytes, a.lda, a.M, m0, lane);
  b0.init(a.B + bz * a.strideB, a.bBytes, a.ldb, a.N, n0, lane);
  b1.init(a.B + bz * a.strideB, a.bBytes, a.ldb, a.N, n0, lane);

  typename Loop::Lanes LN;
#pragma unroll
  for (int c = 0; c < 2; ++c)
#pragma unroll
    for (int e = 0; e < 2; ++e) LN.lo[c][e] = conv::SwzPanel<32, 32>::chunk(r, 4 * c + 2 * h + e);
  LN.aRow = 0;
  LN.bRow = 0;
  f32x16 acc[FM][FN];
  Loop::zero(acc);
  lds_t* panel = (lds_t*)smem + wave * STAGE;
  const int P = static_cast<int>(a.K / 32);
  const int p0 = wave * P / W, np = (wave + 1) * P / W - p0;
  // loads issued unconditionally, clamped to the wave's last panel (a
  // conditional load makes the compiler wait for every load in flight)
  auto kOf = [&](int i) { return 32 * (p0 + min(i, np - 1)); };
  auto multiply = [&]() {
    typename Loop::Frag f0, f1;
    Loop::read(panel, 0, LN, f0);
    Loop::read(panel, 1, LN, f1);
    Loop::mma(f0, acc);
    Loop::mma(f1, acc);
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

  const __amdgpu_buffer_rsrc_t cR = make_rsrc(a.C + bz * a.strideC, a.cBytes);
  const uint32_t ldc4 = static_cast<uint32_t>(a.ldc) * 4u;
  const float alpha = a.alpha, beta = a.beta;
  for (int u = wave; u < UNITS; u += W) {
    const int i = u / (FN * 4), j = (u / 4) % FN, q = u % 4;
    f32x4 p[W];
#pragma unroll
    for (int w = 0; w < W; ++w) p[w] = R[(w * UNITS + u) * 64 + lane];
    f32x4 sum = p[0];
#pragma unroll
    for (int w = 1; w < W; ++w) sum = sum + p[w];
    // lane owns column n; register e of the quad is row m0 + 32i + 8q + 4h + e
    const int64_t n = n0 + 32 * j + r;
    const int64_t mBase = m0 + 32 * i + 8 * q + 4 * h;
    uint32_t vo[4];
#pragma unroll
    for (int e = 0; e < 4; ++e)
      vo[e] = sel_off(n < a.N && mBase + e < a.M,
                      static_cast<uint32_t>(mBase + e) * ldc4 + static_cast<uint32_t>(n) * 4u);
    float cv[4] = {0.f, 0.f, 0.f, 0.f};
    if (beta != 0.f) {
#pragma unroll
      for (int e = 0; e < 4; ++e) cv[e] = buf_ld1s(cR, vo[e], 0);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e)
      conv::buf_st1s(cR, beta != 0.f ? alpha * sum[e] + beta * cv[e] : alpha * sum[e], vo[e], 0);
  }
}

template <class Cfg>
int launch_wsplit(const SgemmArgs& a0, int64_t batch, bool ta, bool tb, hipStream_t s) {
  SgemmArgs a = a0;
  const int64_t tm = (a.M + Cfg::BM - 1) / Cfg::BM, tn = (a.N + Cfg::BN - 1) / Cfg::BN;
  if (tm * tn > INT32_MAX || batch > 65535)
    return fail(TNH_ERR_UNSUPPORTED, "sgemm: grid too large (%lld tiles, batch %lld)",
                (long long)(tm * tn), (long long)batch);
  a.tilesM = static_cast<int>(tm);
  a.tilesN = static_cast<int>(tn);
  const dim3 grid(static_cast<unsigned>(tm * tn), static_cast<unsigned>(batch));
  if (!ta && !tb)
    hipLaunchKernelGGL((sgemm_wsplit_kernel<Cfg, false, false>), grid, dim3(Cfg::NT), 0, s, a);
  else if (!ta)
    hipLaunchKernelGGL((sgemm_wsplit_kernel<Cfg, false, true>), grid, dim3(Cfg::NT), 0, s, a);
  else if (!tb)
    hipLaunchKernelGGL((sgemm_wsplit_kernel<Cfg, true, false>), grid, dim3(Cfg::NT), 0, s, a);
  else
    hipLaunchKernelGGL((sgemm_wsplit_kernel<Cfg, true, true>), grid, dim3(Cfg::NT), 0, s, a);
  return launch_status("sgemm_wsplit_kernel");
}

using Lean128x128 = conv::LeanCfg<128, 128, 32, 4, 2, 2>;
using Lean128x64 = conv::LeanCfg<128, 64, 32, 2, 2, 3>;
using Lean64x128 = conv::LeanCfg<64, 128, 32, 2, 2, 3>;
using Lean64x64 = conv::LeanCfg<64, 64, 32, 2, 2, 4>;

template <class Cfg, bool TA, bool TB, bool VA, bool VB>
int launch_one(const SgemmArgs& a0, int64_t batch, hipStream_t s) {
  SgemmArgs a = a0;
  const int64_t tm = (a.M + Cfg::BM - 1) / Cfg::BM, tn = (a.N + Cfg::BN - 1) / Cfg::BN;
  if (tm * tn > INT32_MAX || batch > 65535)
    return fail(TNH_ERR_UNSUPPORTED, "sgemm: grid too large (%lld tiles, batch %lld)",
                (long long)(tm * tn), (long long)batch);
  a.tilesM = static_cast<int>(tm);
  a.tilesN = static_cast<int>(tn);
  dim3 grid(static_cast<unsigned>(tm * tn), static_cast<unsigned>(batch));
  hipLaunchKernelGGL((sgemm_kernel<Cfg, TA, TB, VA, VB>), grid, dim3(Cfg::NT), 0, s, a);
  return launch_status("sgemm_kernel");
}

template <class Cfg, bool TA, bool TB>
int launch_vec(const SgemmArgs& a, int64_t batch, bool va, bool vb, hipStream_t s) {
  if (va && vb) return launch_one<Cfg, TA, TB, true, true>(a, batch, s);
  if (va) return launch_one<Cfg, TA, TB, true, false>(a, batch, s);
  if (vb) return launch_one<Cfg, TA, TB, false, true>(a, batch, s);
  return launch_one<Cfg, TA, TB, false, false>(a, batch, s);
}

template <class Cfg>
int launch_cfg(const SgemmArgs& a, int64_t batch, bool ta, bool tb, bool va, bool vb, hipStream_t s) {
  if (!ta && !tb) return launch_vec<Cfg, false, false>(a, batch, va, vb, s);
  if (!ta && tb) return launch_vec<Cfg, false, true>(a, batch, va, vb, s);
  if (ta && !tb) return launch_vec<Cfg, true, false>(a, batch, va, vb, s);
  return launch_vec<Cfg, true, true>(a, batch, va, vb, s);
}

template <class Cfg>
int launch_lean(const SgemmArgs& a0, int64_t batch, bool ta, bool tb, hipStream_t s) {
  SgemmArgs a = a0;
  const int64_t tm = (a.M + Cfg::BM - 1) / Cfg::BM, tn = (a.N + Cfg::BN - 1) / Cfg::BN;
  if (tm * tn > INT32_MAX || batch > 65535)
    return fail(TNH_ERR_UNSUPPORTED, "sgemm: grid too large (%lld tiles, batch %lld)",
                (long long)(tm * tn), (long long)batch);
  a.tilesM = static_cast<int>(tm);
  a.tilesN = static_cast<int>(tn);
  const dim3 grid(static_cast<unsigned>(tm * tn), static_cast<unsigned>(batch));
  if (!ta && !tb)
    hipLaunchKernelGGL((sgemm_lean_kernel<Cfg, false, false>), grid, dim3(Cfg::NT), 0, s, a);
  else if (!ta)
    hipLaunchKernelGGL((sgemm_lean_kernel<Cfg, false, true>), grid, dim3(Cfg::NT), 0, s, a);
  else if (!tb)
    hipLaunchKernelGGL((sgemm_lean_kernel<Cfg, true, false>), grid, dim3(Cfg::NT), 0, s, a);
  else
    hipLaunchKernelGGL((sgemm_lean_kernel<Cfg, true, true>), grid, dim3(Cfg::NT), 0, s, a);
  return launch_status("sgemm_lean_kernel");
}

// Tile configurations: 0, 1 the general kernel (any K, alignment or size),
// 2..5 lean (see sgemm_lean_kernel for their requirements), 6..8 wave-split
// (32x32 with 4 or 8 waves, 32x64 with 4; the lean tiles' requirements).
enum SgemmCfg {
  kG128 = 0,
  kG64,
  kL128x128,
  kL128x64,
  kL64x128,
  kL64x64,
  kW32x32x4,
  kW32x32x8,
  kW32x64x4,
  kNumSgemmCfg
};

int launch_sgemm(int cfg, const SgemmArgs& a, int64_t batch, bool ta, bool tb, bool va, bool vb, hipStream_t s) {
  switch (cfg) {
    case kG128: return launch_cfg<Cfg128>(a, batch, ta, tb, va, vb, s);
    case kG64: return launch_cfg<Cfg64>(a, batch, ta, tb, va, vb, s);
    case kL128x128: return launch_lean<Lean128x128>(a, batch, ta, tb, s);
    case kL128x64: return launch_lean<Lean128x64>(a, batch, ta, tb, s);
    case kL64x128: return launch_lean<Lean64x128>(a, batch, ta, tb, s);
    case kL64x64: return launch_lean<Lean64x64>(a, batch, ta, tb, s);
    case kW32x32x4: return launch_wsplit<conv::WsCfg<1, 1, 4>>(a, batch, ta, tb, s);
    case kW32x32x8: return launch_wsplit<conv::WsCfg<1, 1, 8>>(a, batch, ta, tb, s);
    default: return launch_wsplit<conv::WsCfg<1, 2, 4>>(a, batch, ta, tb, s);
  }
}

struct SgemmKey {
  int64_t M, N, K, lda, ldb, ldc, batch;
  int ta, tb, lean;
  bool operator==(const SgemmKey& o) const {
    return M == o.M && N == o.N && K == o.K && lda == o.lda && ldb == o.ldb && ldc == o.ldc && batch == o.batch &&
           ta == o.ta && tb == o.tb && lean == o.lean;
  }
};
struct SgemmKeyHash {
  size_t operator()(const SgemmKey& t) const {
    size_t h = 1469598103934665603ull;
    for (int64_t v : {t.M, t.N, t.K, t.lda, t.ldb, t.ldc, t.batch, (int64_t)t.ta, (int64_t)t.tb, (int64_t)t.lean})
      h = (h ^ static_cast<size_t>(v)) * 1099511628211ull;
    return h;
  }
};
std::mutex g_sgemm_mu;
std::unordered_map<SgemmKey, int, SgemmKeyHash> g_sgemm_tuned;
bool g_sgemm_autotune = true;
int g_sgemm_forced = -1;

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// 16-byte loads of an operand are legal when every vector starts aligned and
// lies entirely inside or outside the contiguous extent.
bool vec_ok(const float* p, int64_t ld, int64_t contigExtent, int64_t stride, int64_t batch) {
  return aligned16(p) && ld % 4 == 0 && contigExtent % 4 == 0 && (batch == 1 || stride % 4 == 0);
}

int sgemm_impl(int32_t transA, int32_t transB, int64_t M, int64_t N, int64_t K, float alpha, const float* A,
               int64_t aOff, int64_t lda, int64_t strideA, const float* B, int64_t bOff, int64_t ldb,
               int64_t strideB, float beta, float* C, int64_t cOff, int64_t ldc, int64_t strideC, int64_t batch) {
  TNH_REQUIRE_CTX(cx);
  TNH_ARG(M >= 0 && N >= 0 && K >= 0 && batch >= 0, "sgemm: negative size");
  if (M == 0 || N == 0 || batch == 0) return TNH_OK;
  TNH_ARG(C != nullptr, "sgemm: C is NULL");
  TNH_ARG(ldc >= N, "sgemm: ldc %lld < N %lld", (long long)ldc, (long long)N);
  const bool ta = transA != 0, tb = transB != 0;
  if (K > 0) {
    TNH_ARG(A != nullptr && B != nullptr, "sgemm: A or B is NULL");
    TNH_ARG(lda >= (ta ? M : K), "sgemm: lda %lld too small", (long long)lda);
    TNH_ARG(ldb >= (tb ? K : N), "sgemm: ldb %lld too small", (long long)ldb);
  }
  TNH_ARG(aOff >= 0 && bOff >= 0 && cOff >= 0, "sgemm: negative offset");
  TNH_ARG(strideA >= 0 && strideB >= 0 && strideC >= 0, "sgemm: negative stride");
  TNH_ARG(K < (int64_t(1) << 31), "sgemm: K too large");
  // operand extents as addressed by the kernel (one batch item)
  const int64_t aElems = K == 0 ? 0 : (ta ? (K - 1) * lda + M : (M - 1) * lda + K);
  const int64_t bElems = K == 0 ? 0 : (tb ? (N - 1) * ldb + K : (K - 1) * ldb + N);
  TNH_ARG(aElems * 4 <= kMaxBufBytes && bElems * 4 <= kMaxBufBytes,
          "sgemm: an operand spans more than 2 GiB (split the call)");

  SgemmArgs a{};
  a.A = A ? A + aOff : nullptr;
  a.B = B ? B + bOff : nullptr;
  a.C = C + cOff;
  a.M = M; a.N = N; a.K = K; a.lda = lda; a.ldb = ldb; a.ldc = ldc;
  a.strideA = strideA; a.strideB = strideB; a.strideC = strideC;
  a.alpha = alpha; a.beta = beta;
  a.aBytes = aElems * 4;
  a.bBytes = bElems * 4;
  const int64_t cElems = (M - 1) * ldc + N;
  a.cBytes = cElems * 4;
  // A operand: contiguous along k when not transposed, along m when transposed.
  const bool va = K > 0 && vec_ok(a.A, lda, ta ? M : K, strideA, batch);
  const bool vb = K > 0 && vec_ok(a.B, ldb, tb ? K : N, strideB, batch);
  // the lean tiles need whole 32-deep panels, 16-byte operands and C within 2 GiB
  const bool lean = K % 32 == 0 && va && vb && a.cBytes <= kMaxBufBytes;
  // Untuned choice: large problems use 128x128 tiles; small ones 64x64 to
  // fill the 256 CUs.
  const int64_t tiles128 = ((M + 127) / 128) * ((N + 127) / 128) * batch;
  const bool big = tiles128 >= 2 * cx->cu_count;
  int cfg = lean ? (big ? kL128x128 : kL64x64) : (big ? kG128 : kG64);
  const SgemmKey key{M, N, K, lda, ldb, ldc, batch, ta, tb, lean};
  bool tune = false;
  {
    std::lock_guard<std::mutex> lk(g_sgemm_mu);
    auto it = g_sgemm_tuned.find(key);
    if (g_sgemm_forced >= 0) {
      if (g_sgemm_forced < kL128x128 || lean) cfg = g_sgemm_forced;
    } else if (deterministic()) {
      // the untuned choice from the shape alone
    } else if (it != g_sgemm_tuned.end()) {
      cfg = it->second;
    } else if (g_sgemm_autotune) {
      hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
      tune = hipStreamIsCapturing(cx->stream, &cs) == hipSuccess && cs == hipStreamCaptureStatusNone;
    }
  }
  if (tune) {
    // First call for this shape: time every valid configuration as a graph
    // replay (time_graph), writing a scratch copy of C so the caller's C is
    // untouched (beta != 0 reads it).  Every whole-K configuration sums k in
    // the same order; the wave-split tiles (timed only where the 64x64 tiles
    // number under two per CU) sum per-wave partials, so their pick can
    // change the last bits (the deterministic mode never times them).
    const size_t cBytesAll = static_cast<size_t>((batch - 1) * strideC + cElems) * 4;
    void* scratch = nullptr;
    if (int st = hip_status(hipStreamSynchronize(cx->stream), "hipStreamSynchronize")) return st;
    if (hipMalloc(&scratch, cBytesAll) == hipSuccess) {
      SgemmArgs t = a;
      t.C = static_cast<float*>(scratch);
      float bestMs = 1e30f;
      int bestCfg = cfg;
      int st = TNH_OK;
      const int64_t tiles64 = ((M + 63) / 64) * ((N + 63) / 64) * batch;
      for (int c = 0; c < kNumSgemmCfg && !st; ++c) {
        if (c >= kL128x128 && !lean) continue;
        if (c >= kW32x32x4 && tiles64 >= 2 * static_cast<int64_t>(cx->cu_count)) continue;
        float ms = 0.f;
        st = time_graph(cx, [&](hipStream_t s) { return launch_sgemm(c, t, batch, ta, tb, va, vb, s); }, 3, ms);
        if (!st && ms < bestMs) bestMs = ms, bestCfg = c;
      }
      (void)hipFree(scratch);
      if (st) return st;
      cfg = bestCfg;
      std::lock_guard<std::mutex> lk(g_sgemm_mu);
      g_sgemm_tuned[key] = cfg;
      static const bool verbose = std::getenv("TNH_VERBOSE") != nullptr;
      if (verbose)
        std::fprintf(stderr, "[tnh] sgemm %c%c M=%lld N=%lld K=%lld batch=%lld -> cfg %d %.4f ms\n", ta ? 'T' : 'N',
                     tb ? 'T' : 'N', (long long)M, (long long)N, (long long)K, (long long)batch, cfg, bestMs);
    } else {
      (void)hipGetLastError();
    }
  }
  return launch_sgemm(cfg, a, batch, ta, tb, va, vb, cx->stream);
}

}  // namespace
}  // namespace tnh

extern "C" int32_t tnh_sgemm_set_autotune(int32_t enable, int32_t forcedConfig) {
  TNH_ARG(forcedConfig >= -1 && forcedConfig < tnh::kNumSgemmCfg, "sgemm_set_autotune: config %d", forcedConfig);
  std::lock_guard<std::mutex> lk(tnh::g_sgemm_mu);
  tnh::g_sgemm_autotune = enable != 0;
  tnh::g_sgemm_forced = forcedConfig;
  if (!tnh::g_sgemm_autotune) tnh::g_sgemm_tuned.clear();
  return TNH_OK;
}

extern "C" int32_t tnh_sgemm(int32_t transA, int32_t transB, int64_t M, int64_t N, int64_t K, float alpha,
                             const float* A, int64_t aOff, int64_t lda, const float* B, int64_t bOff, int64_t ldb,
                             float beta, float* C, int64_t cOff, int64_t ldc) {
  return tnh::sgemm_impl(transA, transB, M, N, K, alpha, A, aOff, lda, 0, B, bOff, ldb, 0, beta, C, cOff, ldc, 0, 1);
}

extern "C" int32_t tnh_sgemm_strided_batched(int32_t transA, int32_t transB, int64_t M, int64_t N, int64_t K,
                                             float alpha, const float* A, int64_t aOff, int64_t lda,
                                             int64_t strideA, const float* B, int64_t bOff, int64_t ldb,
                                             int64_t strideB, float beta, float* C, int64_t cOff, int64_t ldc,
                                             int64_t strideC, int64_t batch) {
  return tnh::sgemm_impl(transA, transB, M, N, K, alpha, A, aOff, lda, strideA, B, bOff, ldb, strideB, beta, C, cOff,
                         ldc, strideC, batch);
}
