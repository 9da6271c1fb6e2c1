// Row-major fp32 SGEMM on MFMA: C = alpha*op(A)*op(B) + beta*C for the four
// NN/NT/TN/TT variants and strided batches.  Replaces TNNCuda.gemm /
// gemmStridedBatched (nncuda.pas:624, 809) and the CPU cblas_sgemm
// (ntensors.pas:2231-2304).
#include "common.hpp"
#include "gemm_core.hpp"

namespace tnh {
namespace {

struct SgemmArgs {
  const float* A;
  const float* B;
  float* C;
  int64_t M, N, K, lda, ldb, ldc;
  int64_t strideA, strideB, strideC;
  int64_t aBytes, bBytes;  // extent of one batch item of A / B
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
  // A operand: contiguous along k when not transposed, along m when transposed.
  const bool va = K > 0 && vec_ok(a.A, lda, ta ? M : K, strideA, batch);
  const bool vb = K > 0 && vec_ok(a.B, ldb, tb ? K : N, strideB, batch);
  // Large problems use 128x128 tiles; small ones 64x64 to fill the 256 CUs.
  const int64_t tiles128 = ((M + 127) / 128) * ((N + 127) / 128) * batch;
  if (tiles128 >= 2 * cx->cu_count) return launch_cfg<Cfg128>(a, batch, ta, tb, va, vb, cx->stream);
  return launch_cfg<Cfg64>(a, batch, ta, tb, va, vb, cx->stream);
}

}  // namespace
}  // namespace tnh

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
