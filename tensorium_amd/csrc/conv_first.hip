// The network's first convolution (3x3 over an NCHW image with C <= 4
// channels, channels-last output) on the matrix cores.
//
// The layer writes F outputs per 9*C inputs, so it is store-bound; on the
// vector ALU its 27-term dot products alone take longer than the stores
// (there is no packed fp32 here).  Here one wave computes 32 output pixels x
// 32 filters per v_mfma_f32_32x32x2_f32 chain:
//   * A = the weights: lane (f, h) supplies W[f][k = 2s + h] at step s, held
//     in registers for the whole kernel (k = tap*C + c over the tap-major
//     weights, zero past K = 9C);
//   * B = the pixels' windows, gathered per lane: lane (n, h) loads input
//     value k = 2s + h of output pixel n straight from the NCHW image (32
//     consecutive pixels per half-wave: coalesced), padding taps masked to
//     kOOB (reads 0);
//   * D[f][pixel]: a lane holds 16 filters of one pixel in groups of four
//     consecutive channels; bias + activation are applied in registers and
//     the 32 x 32 block passes through the wave's LDS tile (rows of eight
//     16-byte chunks, chunk c of row r at c ^ ((r / 2) % 8): conflict-free
//     both ways) so that 8 consecutive lanes store one pixel's 128
//     contiguous bytes (a store instruction covers 8 whole pixel rows rather
//     than 32 bytes of 32 rows).
// K = 27 takes 14 MFMA steps per 32x32 block.  A wave walks blocks of 32
// pixels with the next block's gather in flight while the current one is
// multiplied and stored.  The sums run in MFMA order, not the reference's
// sequential chain: results match the oracle within the per-tensor 1e-5 of
// every convolution (the NCHW entry point keeps the bit-exact kernel).
#include "common.hpp"
#include "conv_first.hpp"
#include "gemm_core.hpp"

namespace tnh {
namespace conv {
namespace {

template <int C, int NF, int ACT>
__global__ __launch_bounds__(256) void conv_first_mfma_kernel(ConvArgs a) {
  constexpr int K = 9 * C, S = (K + 1) / 2;  // MFMA steps: step s pairs k = 2s (lanes 0-31), 2s + 1 (32-63)
  __shared__ f32x4 tile[4][32 * 8];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n = lane & 31, h = lane >> 5;
  const int F = static_cast<int>(a.F);
  const int H = a.g.H, W = a.g.W, OW = a.g.OW, OHW = a.g.OHW;
  const int M = static_cast<int>(a.g.N);

  // this lane's weights (A operand) and biases; per step its tap bit and the
  // offset of its input value relative to the output pixel's centre tap
  float wA[NF][S], bv[NF][4][4];
  int rel[S], tb[S];
#pragma unroll
  for (int s = 0; s < S; ++s) {
    const int k = 2 * s + h, kk = k < K ? k : K - 1;
    const int tap = kk / C, c = kk - tap * C;
    const int ky = tap / 3, kx = tap - ky * 3;
    rel[s] = c * H * W + (ky - 1) * W + (kx - 1);
    tb[s] = k < K ? tap : 31;  // bit 31 of a tap mask is never set: k past K reads 0
#pragma unroll
    for (int j = 0; j < NF; ++j) {
      const int f = 32 * j + n;
      wA[j][s] = (f < F && k < K) ? a.w[f * K + k] : 0.f;
    }
  }
#pragma unroll
  for (int j = 0; j < NF; ++j)
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int f = 32 * j + 8 * q + 4 * h + e;
        bv[j][q][e] = a.bias && f < F ? a.bias[f] : -0.f;  // -0.0: the exact additive identity
      }

  const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.g.x, a.g.xBytes);
  const int xbs = static_cast<int>(a.g.xBatchStride);
  const int nBlocks = (M + 31) / 32;
  const int stride = gridDim.x * 4;
  const int OH = OHW / OW;
  // The input values of block blk (pixel blk*32 + n) for this lane's k.  The
  // block's first pixel is split into (image, row, column) once per wave
  // (scalar); with OW >= 32 a lane's pixel is at most one row further.
  auto gather = [&](int blk, float (&xs)[S]) {
    const int p0 = blk * 32;
    const int P = p0 + n;
    const bool valid = P < M;
    int b, oy, ox;
    if (OW >= 32) {
      const int b0 = p0 / OHW, r0 = p0 - b0 * OHW;
      const int oy0 = r0 / OW;
      b = b0;
      oy = oy0;
      ox = r0 - oy0 * OW + n;
      if (ox >= OW) {
        ox -= OW;
        if (++oy == OH) oy = 0, ++b;
      }
    } else {
      const int PP = valid ? P : 0;
      b = PP / OHW;
      const int p = PP - b * OHW;
      oy = p / OW;
      ox = p - oy * OW;
    }
    const int iy = oy * a.g.sY - a.g.pH + 1, ix = ox * a.g.sX - a.g.pW + 1;  // the centre tap
    uint32_t mask = 0;
#pragma unroll
    for (int ky = 0; ky < 3; ++ky)
#pragma unroll
      for (int kx = 0; kx < 3; ++kx) {
        const bool in = static_cast<unsigned>(iy + ky - 1) < static_cast<unsigned>(H) &&
                        static_cast<unsigned>(ix + kx - 1) < static_cast<unsigned>(W);
        mask |= (valid && in ? 1u : 0u) << (ky * 3 + kx);
      }
    const int base = b * xbs + iy * W + ix;
#pragma unroll
    for (int s = 0; s < S; ++s)
      xs[s] = buf_ld1(xr, sel_off((mask >> tb[s]) & 1u, static_cast<uint32_t>(base + rel[s]) * 4u));
  };
  // Multiplies block blk and stores it (bias, activation, 16-byte stores of
  // whole pixel rows through the wave's LDS tile).
  f32x4* t = tile[wave];
  const int rq = lane & 7;  // the 16-byte chunk a lane stores
  auto finish = [&](int blk, const float (&xs)[S]) {
    const int p0 = blk * 32;
#pragma unroll
    for (int j = 0; j < NF; ++j) {
      f32x16 acc;
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[e] = 0.f;
#pragma unroll
      for (int s = 0; s < S; ++s) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(wA[j][s], xs[s], acc, 0, 0, 0);
      // lane (n, h), quad q: channels 8q + 4h .. +3 of pixel n = chunk 2q + h of row n
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        f32x4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = apply_act(acc[4 * q + e] + bv[j][q][e], ACT);
        t[n * 8 + ((2 * q + h) ^ ((n >> 1) & 7))] = v;
      }
      __builtin_amdgcn_wave_barrier();
      // lanes 8i .. 8i+7 store pixel row 8*it + i, chunk lane & 7; the stores
      // are non-temporal (the output, 354 MB at batch 16, is far larger than
      // the caches: 12-15 us less per batch-16 layer in the network than
      // plain stores)
      const int fq = 32 * j + 4 * rq;
#pragma unroll
      for (int it = 0; it < 4; ++it) {
        const int row = it * 8 + (lane >> 3);
        const f32x4 v = t[row * 8 + (rq ^ ((row >> 1) & 7))];
        const int P = p0 + row;
        if (P < M && fq + 4 <= F)  // F % 4 == 0: a chunk is whole or absent
          __builtin_nontemporal_store(v, reinterpret_cast<f32x4*>(a.out + static_cast<int64_t>(P) * a.outPix + fq));
      }
      __builtin_amdgcn_wave_barrier();
    }
  };

  // Blocks gw, gw + stride, ...: the waves together sweep the output front
  // to back, so the stores stream through a moving window of HBM.  Two
  // register sets in rotation: the gather of the next block is issued
  // before the current one is multiplied; the loads are unconditional
  // (clamped to the last block) so that the compiler waits only for the set
  // it multiplies.  Neighbouring blocks run on different XCDs, so the image
  // is fetched about 4.4 times (146 MB at batch 16), against 354 MB of
  // stores; renumbering the workgroups XCD-contiguously brought the fetch to
  // 1.07x but made the kernel slower (126 against 111-116 us), and so did
  // contiguous block ranges per wave (122 us).
  const int gw = blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(wave);  // uniform: block origins stay scalar
  if (gw >= nBlocks) return;
  float x0[S], x1[S];
  gather(gw, x0);
  for (int blk = gw; blk < nBlocks; blk += 2 * stride) {
    gather(min(blk + stride, nBlocks - 1), x1);
    finish(blk, x0);
    gather(min(blk + 2 * stride, nBlocks - 1), x0);
    if (blk + stride < nBlocks) finish(blk + stride, x1);
  }
}

template <int C, int NF>
void launch_act(const ConvArgs& a, unsigned grid, hipStream_t s) {
  auto go = [&](auto actTag) {
    constexpr int ACT = decltype(actTag)::value;
    hipLaunchKernelGGL((conv_first_mfma_kernel<C, NF, ACT>), dim3(grid), dim3(256), 0, s, a);
  };
  if (a.act == TNH_AC_LEAKY)
    go(std::integral_constant<int, TNH_AC_LEAKY>{});
  else if (a.act == TNH_AC_LOGISTIC)
    go(std::integral_constant<int, TNH_AC_LOGISTIC>{});
  else
    go(std::integral_constant<int, TNH_AC_LINEAR>{});
}

}  // namespace

bool first_mfma_ok(const ConvArgs& a) {
  return a.g.C >= 1 && a.g.C <= 4 && a.F <= 64 && a.F % 4 == 0 && !a.res && a.outPix % 4 == 0 &&
         (reinterpret_cast<uintptr_t>(a.out) & 15) == 0 && a.g.N < (int64_t(1) << 30) &&
         a.g.xBytes < (int64_t(1) << 31) && a.upS == 0 && !a.yolo;
}

int launch_first_mfma(const ConvArgs& a, hipStream_t s) {
  if (!first_mfma_ok(a)) return fail(TNH_ERR_UNSUPPORTED, "conv2d: first-layer MFMA kernel: unsupported call");
  const int64_t blocks = (a.g.N + 31) / 32;
  // about eight blocks of 32 pixels per wave when the layer is large, one
  // when it is small (four waves per workgroup)
  const int64_t grid = std::max<int64_t>(1, std::min<int64_t>((blocks + 3) / 4, 2048));
  auto go = [&](auto cTag) {
    constexpr int C = decltype(cTag)::value;
    if (a.F <= 32)
      launch_act<C, 1>(a, static_cast<unsigned>(grid), s);
    else
      launch_act<C, 2>(a, static_cast<unsigned>(grid), s);
  };
  switch (a.g.C) {
    case 1: go(std::integral_constant<int, 1>{}); break;
    case 2: go(std::integral_constant<int, 2>{}); break;
    case 3: go(std::integral_constant<int, 3>{}); break;
    default: go(std::integral_constant<int, 4>{}); break;
  }
  return launch_status("conv_first_mfma_kernel");
}

}  // namespace conv
}  // namespace tnh
