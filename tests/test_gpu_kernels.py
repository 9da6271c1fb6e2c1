"""GPU parity tests: every kernel through the C ABI against the CPU oracle on
identical seeded inputs.  Bit-exact for im2col/col2im, maxpool (values and
int64 indices), upsample, bias, activations, copies and the YOLO head;
per-tensor max|g - r| / max|r| <= 1e-5 for GEMM and convolution, and exact
equality for GEMMs on integer-valued data (every partial sum exact)."""
import numpy as np
import pytest
import torch

from oracle import refcpu as R
from tensorium_amd import synth
from tensorium_amd.nnhip import CONV_NCHW_CFGS, CONV_RETIRED_CFGS, CONV_SPLIT_UNIT, CONV_TAIL_BASE, CONV_TAIL_SLOT_BASE, CONV_WSPLIT_CFGS, NUM_SGEMM_CFGS, WEIGHTS_TAP_MAJOR, TNHError, acLEAKY, acLINEAR, acLOGISTIC

pytestmark = pytest.mark.gpu
TOL = 1e-5


def D(a):
    t = torch.from_numpy(np.ascontiguousarray(a)).cuda()
    torch.cuda.synchronize()
    return t


def H(t, hip):
    hip.finish()
    torch.cuda.synchronize()
    return t.cpu().numpy()


def case(msg):
    print(f"[case] {msg}", flush=True)


def op(X, t):
    return X.T if t else X


# ---------------------------------------------------------------- SGEMM ----
SHAPES = [(1, 1, 1), (7, 5, 3), (33, 65, 17), (64, 64, 16), (128, 128, 64), (129, 257, 100), (300, 200, 500),
          (16, 5000, 27)]


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("M,N,K", SHAPES)
def test_sgemm_exact_integer(hip, ta, tb, M, N, K):
    case(f"sgemm int ta={ta} tb={tb} {M}x{N}x{K}")
    rng = np.random.default_rng(M * 1000 + N + K)
    A = rng.integers(-4, 5, (K, M) if ta else (M, K)).astype(np.float32)
    B = rng.integers(-4, 5, (N, K) if tb else (K, N)).astype(np.float32)
    C0 = rng.integers(-9, 10, (M, N)).astype(np.float32)
    dA, dB, dC = D(A), D(B), D(C0)
    hip.gemm(ta, tb, M, N, K, 1.0, dA, 0, A.shape[1], dB, 0, B.shape[1], 1.0, dC, 0, N)
    ref = op(A, ta).astype(np.int64) @ op(B, tb).astype(np.int64) + C0.astype(np.int64)
    assert np.array_equal(H(dC, hip), ref.astype(np.float32))


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("M,N,K", [(256, 256, 256), (512, 512, 512), (100, 300, 1000), (64, 10816, 288)])
def test_sgemm_vs_oracle(hip, ta, tb, M, N, K):
    case(f"sgemm rand ta={ta} tb={tb} {M}x{N}x{K}")
    A = synth.uniform(11, (K, M) if ta else (M, K), -1, 1)
    B = synth.uniform(12, (N, K) if tb else (K, N), -1, 1)
    C = np.zeros((M, N), np.float32)
    dA, dB, dC = D(A), D(B), D(C)
    hip.gemm(ta, tb, M, N, K, 1.0, dA, 0, A.shape[1], dB, 0, B.shape[1], 0.0, dC, 0, N)
    R.sgemm(ta, tb, M, N, K, 1.0, A, A.shape[1], B, B.shape[1], 0.0, C, N)
    assert R.rel_err(H(dC, hip), C) <= TOL


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_sgemm_full_size_exact(hip, ta, tb):
    """BASELINE config 2 at 4096^3 (the tuned lean kernels at their benchmark
    size): integer operands in [-4, 4] make every partial sum exact in fp32,
    so the result equals a float64 product bit for bit."""
    M = N = K = 4096
    case(f"sgemm full size int ta={ta} tb={tb} {M}x{N}x{K}")
    rng = np.random.default_rng(4096 + 2 * ta + tb)
    A = rng.integers(-4, 5, (K, M) if ta else (M, K)).astype(np.float32)
    B = rng.integers(-4, 5, (N, K) if tb else (K, N)).astype(np.float32)
    dA, dB = D(A), D(B)
    dC = torch.full((M, N), 3.0, dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    hip.gemm(ta, tb, M, N, K, 1.0, dA, 0, A.shape[1], dB, 0, B.shape[1], 0.0, dC, 0, N)
    ref = op(A, ta).astype(np.float64) @ op(B, tb).astype(np.float64)
    assert np.array_equal(H(dC, hip), ref.astype(np.float32))


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_sgemm_8192_exact(hip, ta, tb):
    """BASELINE config 2's largest square size in all four variants (the
    bench's 8192^3 lines): integer operands in [-2, 2] keep every partial sum
    below 2^24, so the product is exact in fp32 and must equal a float64
    product bit for bit."""
    M = N = K = 8192
    case(f"sgemm 8192^3 int ta={ta} tb={tb}")
    g = torch.Generator(device="cuda").manual_seed(8192 + 2 * ta + tb)
    dA = torch.randint(-2, 3, (M, K), generator=g, device="cuda").float()
    dB = torch.randint(-2, 3, (K, N), generator=g, device="cuda").float()
    dC = torch.full((M, N), 5.0, dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    hip.gemm(ta, tb, M, N, K, 1.0, dA, 0, dA.shape[1], dB, 0, dB.shape[1], 0.0, dC, 0, N)
    hip.finish()
    a64 = dA.double().T if ta else dA.double()
    b64 = dB.double().T if tb else dB.double()
    ref = (a64 @ b64).float()
    assert torch.equal(dC, ref)


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("n", [1024, 2048])
def test_sgemm_mid_square_exact(hip, n, ta, tb):
    """The bench's 1024^3 and 2048^3 lines in all four variants (the sizes
    where the wave-split tiles compete with the lean ones): integer operands
    in [-4, 4] keep every partial sum exact in fp32, so the product equals a
    float64 product bit for bit; then U[-1, 1) operands against the oracle on
    16 sampled rows of C (the oracle's per-row chains do not depend on the
    other rows of A)."""
    M = N = K = n
    case(f"sgemm {n}^3 int ta={ta} tb={tb}")
    g = torch.Generator(device="cuda").manual_seed(n + 2 * ta + tb)
    dA = torch.randint(-4, 5, (M, K), generator=g, device="cuda").float()
    dB = torch.randint(-4, 5, (K, N), generator=g, device="cuda").float()
    dC = torch.full((M, N), 7.0, dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    hip.gemm(ta, tb, M, N, K, 1.0, dA, 0, n, dB, 0, n, 0.0, dC, 0, N)
    hip.finish()
    a64 = dA.double().T if ta else dA.double()
    b64 = dB.double().T if tb else dB.double()
    assert torch.equal(dC, (a64 @ b64).float())
    del dA, dB, dC
    case(f"sgemm {n}^3 rand ta={ta} tb={tb} vs oracle (16 rows)")
    A = synth.uniform(41 + n, (n, n), -1, 1)
    B = synth.uniform(42 + n, (n, n), -1, 1)
    dA, dB = D(A), D(B)
    dC = torch.zeros((M, N), dtype=torch.float32, device="cuda")
    hip.gemm(ta, tb, M, N, K, 1.0, dA, 0, n, dB, 0, n, 0.0, dC, 0, N)
    got = H(dC, hip)
    rows = np.linspace(0, M - 1, 16).astype(np.int64)
    # rows r of op(A): A[r, :] for NN/NT, column r of A (row r of A^T) for TN/TT
    Ar = np.ascontiguousarray(A.T[rows] if ta else A[rows])
    ref = np.zeros((16, N), np.float32)
    R.sgemm(0, tb, 16, N, K, 1.0, Ar, K, B, n, 0.0, ref, N)
    assert R.rel_err(got[rows], ref) <= TOL


# the conv-shaped skinny GEMMs of BASELINE config 2 (M = F, N = OH*OW*16,
# K = 9*C): the bench times all five
SKINNY = [(64, 692224, 288), (128, 173056, 576), (256, 43264, 1152), (512, 10816, 2304), (1024, 2704, 4608)]


@pytest.mark.parametrize("M,N,K", SKINNY)
def test_sgemm_skinny_bench_shapes(hip, M, N, K):
    """The bench's skinny shapes, NN: exact on integer operands at full size,
    and random U[-1, 1) operands against the oracle (16 rows of A: the
    oracle's per-row FMA chains do not depend on the other rows)."""
    case(f"sgemm skinny int {M}x{N}x{K}")
    g = torch.Generator(device="cuda").manual_seed(M + N + K)
    dA = torch.randint(-2, 3, (M, K), generator=g, device="cuda").float()
    dB = torch.randint(-2, 3, (K, N), generator=g, device="cuda").float()
    dC = torch.zeros((M, N), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    hip.gemm(0, 0, M, N, K, 1.0, dA, 0, K, dB, 0, N, 0.0, dC, 0, N)
    hip.finish()
    assert torch.equal(dC, (dA.double() @ dB.double()).float())
    del dA, dB, dC
    case(f"sgemm skinny rand {M}x{N}x{K} vs oracle")
    A = synth.uniform(31, (M, K), -1, 1)
    B = synth.uniform(32, (K, N), -1, 1)
    dA, dB = D(A), D(B)
    dC = torch.zeros((M, N), dtype=torch.float32, device="cuda")
    hip.gemm(0, 0, M, N, K, 1.0, dA, 0, K, dB, 0, N, 0.0, dC, 0, N)
    got = H(dC, hip)
    rows = np.linspace(0, M - 1, 16).astype(np.int64)
    ref = np.zeros((16, N), np.float32)
    R.sgemm(0, 0, 16, N, K, 1.0, np.ascontiguousarray(A[rows]), K, B, N, 0.0, ref, N)
    assert R.rel_err(got[rows], ref) <= TOL


@pytest.mark.parametrize("ta,tb", [(0, 0), (1, 1)])
def test_sgemm_alpha_half_beta_one_full_size(hip, ta, tb):
    """The config-2 beta = 1 / alpha = 0.5 run at 4096^3: integer operands, so
    0.5 * sum + C is exact whatever the order (the reference scales A by
    alpha first, ntensors.pas:2136-2206)."""
    M = N = K = 4096
    case(f"sgemm alpha 0.5 beta 1 int ta={ta} tb={tb} 4096^3")
    g = torch.Generator(device="cuda").manual_seed(77 + ta + tb)
    dA = torch.randint(-3, 4, (M, K), generator=g, device="cuda").float()
    dB = torch.randint(-3, 4, (K, N), generator=g, device="cuda").float()
    C0 = torch.randint(-50, 51, (M, N), generator=g, device="cuda").float()
    dC = C0.clone()
    torch.cuda.synchronize()
    hip.gemm(ta, tb, M, N, K, 0.5, dA, 0, K, dB, 0, N, 1.0, dC, 0, N)
    hip.finish()
    a64 = dA.double().T if ta else dA.double()
    b64 = dB.double().T if tb else dB.double()
    assert torch.equal(dC, (0.5 * (a64 @ b64) + C0.double()).float())


def test_sgemm_alpha_beta_offsets_ld(hip):
    case("sgemm alpha/beta, offsets, padded ld")
    rng = np.random.default_rng(5)
    M, N, K, lda, ldb, ldc = 45, 70, 33, 40, 77, 81
    A = rng.uniform(-1, 1, 3 + M * lda).astype(np.float32)
    B = rng.uniform(-1, 1, 5 + K * ldb).astype(np.float32)
    C = rng.uniform(-1, 1, 7 + M * ldc).astype(np.float32)
    dA, dB, dC = D(A), D(B), D(C)
    hip.gemm(0, 0, M, N, K, 0.5, dA, 3, lda, dB, 5, ldb, 2.0, dC, 7, ldc)
    ref = C.copy()
    Cv = ref[7:].reshape(M, ldc)
    Cv2 = np.ascontiguousarray(Cv)
    R.sgemm(0, 0, M, N, K, 0.5, A[3:].reshape(M, lda), lda, B[5:].reshape(K, ldb), ldb, 2.0, Cv2, ldc)
    ref[7:] = Cv2.ravel()
    got = H(dC, hip)
    assert np.array_equal(got[:7], C[:7])                      # untouched prefix
    g2, r2 = got[7:].reshape(M, ldc), ref[7:].reshape(M, ldc)
    assert np.array_equal(g2[:, N:], r2[:, N:])                # untouched ld padding
    assert R.rel_err(g2[:, :N], r2[:, :N]) <= TOL


@pytest.mark.parametrize("cfg", range(NUM_SGEMM_CFGS))
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("M,N,K", [(100, 300, 96), (36, 68, 32), (260, 132, 320)])
def test_sgemm_forced_configs(hip, cfg, ta, tb, M, N, K):
    """Every SGEMM tile configuration on shapes with edge tiles, padded leading
    dimensions and beta = 1 (integer data: the sums are exact)."""
    case(f"sgemm cfg{cfg} ta={ta} tb={tb} {M}x{N}x{K}")
    rng = np.random.default_rng(cfg * 7919 + M + N + K + 2 * ta + tb)
    lda, ldb, ldc = (M if ta else K) + 4, (K if tb else N) + 8, N + 4
    A = rng.integers(-4, 5, (K if ta else M, lda)).astype(np.float32)
    B = rng.integers(-4, 5, (N if tb else K, ldb)).astype(np.float32)
    C0 = rng.integers(-9, 10, (M, ldc)).astype(np.float32)
    dA, dB, dC = D(A), D(B), D(C0)
    hip.setSgemmAutotune(True, cfg)
    try:
        hip.gemm(ta, tb, M, N, K, 1.0, dA, 0, lda, dB, 0, ldb, 1.0, dC, 0, ldc)
    finally:
        hip.setSgemmAutotune(True, -1)
    a = A[:, :M].T if ta else A[:, :K]
    b = B[:, :K].T if tb else B[:, :N]
    ref = C0.astype(np.int64)
    ref[:, :N] += a.astype(np.int64) @ b.astype(np.int64)
    assert np.array_equal(H(dC, hip), ref.astype(np.float32))


@pytest.mark.parametrize("cfg", range(2, NUM_SGEMM_CFGS))
def test_sgemm_lean_batched_alpha_beta(hip, cfg):
    """Lean tiles through gemmStridedBatched with alpha, beta and a shared A."""
    case(f"sgemm lean batched cfg{cfg}")
    M, N, K, batch = 72, 200, 64, 3
    A = synth.uniform(31, (M, K), -1, 1)
    B = synth.uniform(32, (batch, K, N), -1, 1)
    C = synth.uniform(33, (batch, M, N), -1, 1)
    dA, dB, dC = D(A), D(B), D(C)
    hip.setSgemmAutotune(True, cfg)
    try:
        hip.gemmStridedBatched(0, 0, M, N, K, 0.5, dA, 0, K, 0, dB, 0, N, K * N, 2.0, dC, 0, N, M * N, batch)
    finally:
        hip.setSgemmAutotune(True, -1)
    got = H(dC, hip)
    for i in range(batch):
        ref = C[i].copy()
        R.sgemm(0, 0, M, N, K, 0.5, A, K, np.ascontiguousarray(B[i]), N, 2.0, ref, N)
        assert R.rel_err(got[i], ref) <= TOL


def test_sgemm_beta_zero_overwrites(hip):
    case("sgemm beta=0 ignores NaN in C")
    A = np.ones((8, 4), np.float32)
    B = np.ones((4, 8), np.float32)
    dC = D(np.full((8, 8), np.nan, np.float32))
    hip.gemm(0, 0, 8, 8, 4, 1.0, D(A), 0, 4, D(B), 0, 8, 0.0, dC, 0, 8)
    assert np.all(H(dC, hip) == 4.0)


@pytest.mark.parametrize("ta,tb", [(0, 0), (1, 0), (0, 1)])
def test_sgemm_strided_batched(hip, ta, tb):
    case(f"sgemm strided batched ta={ta} tb={tb}")
    M, N, K, batch = 40, 90, 50, 3
    A = synth.uniform(21, (K, M) if ta else (M, K), -1, 1)  # shared: strideA = 0
    B = synth.uniform(22, (batch,) + ((N, K) if tb else (K, N)), -1, 1)
    C = np.zeros((batch, M, N), np.float32)
    dC = D(C)
    hip.gemmStridedBatched(ta, tb, M, N, K, 1.0, D(A), 0, A.shape[1], 0, D(B), 0, B.shape[2], N * K, 0.0, dC, 0, N,
                           M * N, batch)
    R.sgemm_strided_batched(ta, tb, M, N, K, 1.0, A, A.shape[1], 0, B, B.shape[2], N * K, 0.0, C, N, M * N, batch)
    assert R.rel_err(H(dC, hip), C) <= TOL


# ------------------------------------------------------- im2col/col2im ----
GEOMS = [((1, 3, 416, 416), 3, 1, 1), ((2, 8, 33, 31), 3, 1, 2), ((2, 5, 20, 20), 1, 0, 1), ((1, 4, 13, 13), 3, 1, 1),
         ((3, 2, 10, 12), 3, 2, 3)]


@pytest.mark.parametrize("shape,k,p,s", GEOMS)
def test_im2col_bit_exact(hip, shape, k, p, s):
    case(f"im2col {shape} k{k} p{p} s{s}")
    x = synth.uniform(31, shape)
    B, Cc, Hh, W = shape
    ref = R.im2col(x, k, k, p, p, s, s)
    dcol = torch.empty(ref.shape, dtype=torch.float32, device="cuda")
    hip.im2colStridedBatched(Cc, Hh, W, k, k, p, p, s, s, 1, 1, D(x), Cc * Hh * W, 0, dcol, ref[0].size, 0, B)
    assert np.array_equal(H(dcol, hip), ref)


def test_im2col_dilation(hip):
    case("im2col dilation 2")
    x = synth.uniform(32, (1, 3, 15, 14))
    ref = R.im2col(x, 3, 3, 2, 2, 1, 1, 2, 2)
    dcol = torch.empty(ref.shape, dtype=torch.float32, device="cuda")
    hip.im2col(3, 15, 14, 3, 3, 2, 2, 1, 1, 2, 2, D(x), 0, dcol, 0)
    assert np.array_equal(H(dcol, hip), ref)


@pytest.mark.parametrize("shape,k,p,s", GEOMS[1:])
def test_col2im_bit_exact_accumulates(hip, shape, k, p, s):
    case(f"col2im {shape} k{k} p{p} s{s}")
    B, Cc, Hh, W = shape
    OH, OW = R.conv_out(Hh, k, p, s), R.conv_out(W, k, p, s)
    col = synth.normal(33, (B, Cc * k * k, OH * OW))
    im0 = synth.normal(34, shape)
    ref = R.col2im(col, im0.copy(), k, k, p, p, s, s)
    dim = D(im0)
    hip.col2imStridedBatched(Cc, Hh, W, k, k, p, p, s, s, 1, 1, D(col), col[0].size, 0, dim, Cc * Hh * W, 0, B)
    assert np.array_equal(H(dim, hip), ref)


# ----------------------------------------------------------- convolution ----
CONVS = [  # batch, C, H, F, k, s, p, act
    (1, 3, 416, 16, 3, 1, 1, acLEAKY),    # config 1
    (2, 32, 52, 64, 3, 2, 1, acLEAKY),
    (2, 64, 26, 32, 1, 1, 0, acLEAKY),
    (3, 128, 13, 255, 1, 1, 0, acLINEAR),  # odd HW (169): scalar 1x1 path
    (2, 256, 13, 512, 3, 1, 1, acLEAKY),
    (1, 27, 30, 130, 3, 1, 1, acLEAKY),    # K = 243, F not a tile multiple
]


@pytest.mark.parametrize("B,Cc,Hh,F,k,s,p,act", CONVS)
def test_conv_forward_vs_oracle(hip, B, Cc, Hh, F, k, s, p, act):
    case(f"conv B{B} C{Cc} H{Hh} F{F} k{k} s{s} p{p} act{act}")
    x = synth.uniform(41, (B, Cc, Hh, Hh))
    Wt = synth.normal(42, (F, Cc * k * k), 0.05 if Cc == 3 else (2.0 / (Cc * k * k)) ** 0.5)
    b = synth.normal(43, (F,), 0.1)
    ref = R.conv_forward(x, Wt, b, k, s, p, act)
    dout = torch.empty(ref.shape, dtype=torch.float32, device="cuda")
    hip.conv2dForward(B, Cc, Hh, Hh, F, k, s, p, D(x), 0, D(Wt), D(b), act, dout, 0)
    assert R.rel_err(H(dout, hip), ref) <= TOL


@pytest.mark.parametrize("B,Cc,Hh,F,s,res", [(2, 64, 20, 96, 1, False), (3, 32, 17, 64, 2, False),
                                             (1, 128, 13, 256, 1, True)])
def test_conv_reference_layout_repacks(hip, B, Cc, Hh, F, s, res):
    """A 3x3 call with reference-layout weights ([F][C][3][3], as the layer
    stores them) repacks them tap-major for the call and runs the tap-major
    tiles: bit-identical to a call with weights packed by packConvWeights
    (same kernel, same tuned tile), within the bound of the oracle, and the
    caller's weights are left as they were.  A second call after the weights
    change sees the new weights (nothing is cached)."""
    case(f"conv reference layout repacked B{B} C{Cc} H{Hh} F{F} s{s} residual={res}")
    x = synth.uniform(47, (B, Cc, Hh, Hh))
    Wt = synth.normal(48, (F, Cc * 9), (2.0 / (Cc * 9)) ** 0.5)
    b = synth.normal(49, (F,), 0.1)
    ref = R.conv_forward(x, Wt, b, 3, s, 1, acLEAKY)
    OH = ref.shape[2]
    r = synth.uniform(50, ref.shape, -1, 1) if res else None
    if res:
        ref = (ref + r).astype(np.float32)
    dx, dW, db = D(x), D(Wt), D(b)
    dr = D(r) if res else None
    packed = torch.empty_like(dW)
    hip.packConvWeights(F, Cc, 3, dW, packed)
    outs = []
    for w, layout in ((packed, WEIGHTS_TAP_MAJOR), (dW, 0)):
        dout = torch.empty(ref.shape, dtype=torch.float32, device="cuda")
        hip.conv2dForward(B, Cc, Hh, Hh, F, 3, s, 1, dx, 0, w, db, acLEAKY, dout, 0, weightLayout=layout,
                          residual=dr)
        outs.append(H(dout, hip))
    assert np.array_equal(outs[0], outs[1])
    assert R.rel_err(outs[1], ref) <= TOL
    assert np.array_equal(H(dW, hip), Wt)
    W2 = (Wt * np.float32(-0.5)).astype(np.float32)
    dW.copy_(torch.from_numpy(W2))
    dout = torch.empty(ref.shape, dtype=torch.float32, device="cuda")
    hip.conv2dForward(B, Cc, Hh, Hh, F, 3, s, 1, dx, 0, dW, db, acLEAKY, dout, 0, weightLayout=0, residual=dr)
    ref2 = R.conv_forward(x, W2, b, 3, s, 1, acLEAKY)
    if res:
        ref2 = (ref2 + r).astype(np.float32)
    assert R.rel_err(H(dout, hip), ref2) <= TOL
    assert OH > 0


@pytest.mark.parametrize("cfg", CONV_NCHW_CFGS)
@pytest.mark.parametrize("B,Cc,Hh,F,k,s,p,act", [(2, 32, 26, 64, 3, 1, 1, acLEAKY), (1, 64, 13, 96, 3, 2, 1, acLEAKY),
                                                 (2, 48, 11, 40, 3, 1, 1, acLINEAR), (1, 3, 20, 16, 3, 1, 1, acLEAKY),
                                                 (2, 40, 9, 70, 1, 1, 0, acLEAKY), (3, 64, 13, 300, 1, 1, 0, acLEAKY),
                                                 (2, 16, 7, 33, 3, 2, 1, acLEAKY)])
def test_conv_packed_every_config(hip, cfg, B, Cc, Hh, F, k, s, p, act):
    """Tap-major packed weights through each tile configuration (pinned)."""
    case(f"conv packed cfg{cfg} B{B} C{Cc} H{Hh} F{F} k{k} s{s}")
    x = synth.uniform(44, (B, Cc, Hh, Hh))
    Wt = synth.normal(45, (F, Cc * k * k), (2.0 / (Cc * k * k)) ** 0.5)
    b = synth.normal(46, (F,), 0.1)
    ref = R.conv_forward(x, Wt, b, k, s, p, act)
    dW = D(Wt)
    packed = torch.empty_like(dW)
    hip.packConvWeights(F, Cc, k, dW, packed)
    got = H(packed, hip).reshape(F, k, k, Cc)
    assert np.array_equal(got, Wt.reshape(F, Cc, k, k).transpose(0, 2, 3, 1))
    dout = torch.empty(ref.shape, dtype=torch.float32, device="cuda")
    hip.setConvAutotune(True, cfg)
    try:
        hip.conv2dForward(B, Cc, Hh, Hh, F, k, s, p, D(x), 0, packed, D(b), act, dout, 0,
                          weightLayout=WEIGHTS_TAP_MAJOR if k > 1 else 0)
        got = H(dout, hip)
    finally:
        hip.setConvAutotune(True, -1)
    assert R.rel_err(got, ref) <= TOL


# (B, C, H, F, k, stride, residual): ragged pixel and filter counts, stride 2,
# 1x1 with HW % 4 != 0 (scalar pixel loads) and == 0 (16-byte pixel
# vectors), K = 32 over up to 8 waves (some waves get no panel), and
# YOLOv3's 13x13 batch-1 3x3 shape
WSPLIT_NCHW_SHAPES = [
    (1, 64, 13, 96, 3, 1, True),
    (2, 32, 10, 40, 3, 2, False),
    (1, 32, 9, 70, 1, 1, True),
    (3, 96, 8, 33, 1, 1, False),
    (2, 64, 12, 40, 1, 1, True),
    (1, 512, 13, 1024, 3, 1, False),
]


@pytest.mark.parametrize("cfg", CONV_WSPLIT_CFGS)
@pytest.mark.parametrize("shape", WSPLIT_NCHW_SHAPES)
def test_conv_nchw_wsplit_integer(hip, cfg, shape):
    """Every wave-split tile through tnh_conv2d_fwd (rows = filters, columns =
    output pixels) on integer data, so every partial sum is exact and the
    result equals the oracle bit for bit; input, output and residual at
    offsets with batch strides wider than one image (route slices), the
    rest of the output untouched."""
    B, Cc, Hh, F, k, s, with_res = shape
    p = k // 2
    case(f"conv nchw wsplit cfg{cfg} {shape}")
    OH = (Hh + 2 * p - k) // s + 1
    rng = np.random.default_rng(cfg * 1000 + Cc + F)
    x = rng.integers(-3, 4, (B, Cc, Hh, Hh)).astype(np.float32)
    Wt = rng.integers(-2, 3, (F, Cc * k * k)).astype(np.float32)
    b = rng.integers(-5, 6, F).astype(np.float32)
    ref = R.conv_forward(x, Wt, b, k, s, p, acLEAKY)
    xs, os_, rs = Cc * Hh * Hh + 12, F * OH * OH + 20, F * OH * OH + 8
    xin = np.zeros(8 + B * xs, np.float32)
    for i in range(B):
        xin[8 + i * xs:8 + i * xs + Cc * Hh * Hh] = x[i].ravel()
    res = rin = None
    if with_res:
        res = rng.integers(-5, 6, (B, F, OH, OH)).astype(np.float32)
        ref = R.addvv(ref, res)
        rin = np.zeros(4 + B * rs, np.float32)
        for i in range(B):
            rin[4 + i * rs:4 + i * rs + F * OH * OH] = res[i].ravel()
    dout = D(np.full(16 + B * os_, 7.0, np.float32))
    wt = Wt.reshape(F, Cc, k, k).transpose(0, 2, 3, 1).reshape(F, -1) if k > 1 else Wt
    hip.setConvAutotune(True, cfg)
    try:
        hip.conv2dForward(B, Cc, Hh, Hh, F, k, s, p, D(xin), 8, D(np.ascontiguousarray(wt)), D(b), acLEAKY, dout, 16,
                          inBatchStride=xs, outBatchStride=os_, residual=None if rin is None else D(rin),
                          resOffset=4, resBatchStride=rs, weightLayout=WEIGHTS_TAP_MAJOR if k > 1 else 0)
    finally:
        hip.setConvAutotune(True, -1)
    got = H(dout, hip)
    mask = np.ones(got.shape, bool)
    for i in range(B):
        seg = got[16 + i * os_:16 + i * os_ + F * OH * OH].reshape(F, OH, OH)
        assert np.array_equal(seg, ref[i]), f"image {i}"
        mask[16 + i * os_:16 + i * os_ + F * OH * OH] = False
    assert np.all(got[mask] == 7.0)


@pytest.mark.parametrize("cfg", CONV_WSPLIT_CFGS)
@pytest.mark.parametrize("act", [acLEAKY, acLINEAR, acLOGISTIC])
def test_conv_nchw_wsplit_vs_oracle(hip, cfg, act):
    """Wave-split tiles through tnh_conv2d_fwd on YOLOv3's batch-1 26x26 3x3
    layer (C 256 -> 512), random data: per tensor within 1e-5 of the oracle.
    The fused logistic is TNNCuda's 1/(1 + exp(-x)) (cuda_sgemm.cu:305-309),
    held against the float64 sigmoid of the oracle's linear output."""
    B, Cc, Hh, F, k = 1, 256, 26, 512, 3
    case(f"conv nchw wsplit cfg{cfg} act{act} vs oracle")
    x = synth.uniform(95 + cfg, (B, Cc, Hh, Hh))
    Wt = synth.normal(96, (F, Cc * k * k), (2.0 / (Cc * k * k)) ** 0.5)
    b = synth.normal(97, (F,), 0.1)
    if act == acLOGISTIC:
        ref = 1.0 / (1.0 + np.exp(-R.conv_forward(x, Wt, b, k, 1, 1, acLINEAR).astype(np.float64)))
    else:
        ref = R.conv_forward(x, Wt, b, k, 1, 1, act)
    wt = np.ascontiguousarray(Wt.reshape(F, Cc, k, k).transpose(0, 2, 3, 1).reshape(F, -1))
    dout = torch.empty((B, F, Hh, Hh), dtype=torch.float32, device="cuda")
    hip.setConvAutotune(True, cfg)
    try:
        hip.conv2dForward(B, Cc, Hh, Hh, F, k, 1, 1, D(x), 0, D(wt), D(b), act, dout, 0,
                          weightLayout=WEIGHTS_TAP_MAJOR)
    finally:
        hip.setConvAutotune(True, -1)
    assert R.rel_err(H(dout, hip), ref) <= TOL


@pytest.mark.parametrize("B,Cc,Hh,F,s,tap,act,resid", [(1, 3, 416, 16, 1, False, acLEAKY, False),
                                                       (2, 3, 37, 32, 1, True, acLEAKY, True),
                                                       (1, 1, 9, 5, 2, False, acLINEAR, False),
                                                       (3, 4, 20, 7, 1, True, acLEAKY, False),
                                                       (2, 2, 15, 9, 2, True, acLINEAR, True),
                                                       (1, 3, 50, 12, 2, True, acLINEAR, True),
                                                       (2, 3, 33, 64, 1, False, acLEAKY, False),
                                                       (1, 3, 24, 35, 1, True, acLINEAR, True)])
def test_conv_few_channels_bit_exact(hip, B, Cc, Hh, F, s, tap, act, resid):
    """C <= 4 3x3 layers (the RGB input layer; config 1 at full size) run the
    per-pixel kernel, whose sequential FMA chain in the reference k order is
    the reference CPU arithmetic: equal bit for bit to the oracle.  32 and
    more filters over few pixels split into filter groups (64: four groups
    of 16; 35: groups of 20 and 15)."""
    case(f"conv few-channel B{B} C{Cc} H{Hh} F{F} s{s} tap{tap} act{act} res{resid}")
    x = synth.uniform(51, (B, Cc, Hh, Hh))
    Wt = synth.normal(52, (F, Cc * 9), 0.05)
    b = synth.normal(53, (F,), 0.1)
    ref = R.conv_forward(x, Wt, b, 3, s, 1, act)
    res = synth.normal(54, ref.shape) if resid else None
    if resid:
        ref = R.addvv(ref, res)
    dW = D(Wt)
    if tap:
        packed = torch.empty_like(dW)
        hip.packConvWeights(F, Cc, 3, dW, packed)
        dW = packed
    dout = torch.empty(ref.shape, dtype=torch.float32, device="cuda")
    hip.conv2dForward(B, Cc, Hh, Hh, F, 3, s, 1, D(x), 0, dW, D(b), act, dout, 0,
                      residual=D(res) if resid else None, weightLayout=WEIGHTS_TAP_MAJOR if tap else 0)
    assert np.array_equal(H(dout, hip), ref)


@pytest.mark.parametrize("cfg", [0, 1, 11, 13])
@pytest.mark.parametrize("splits", [2, 4, 16])
@pytest.mark.parametrize("B,Cc,Hh,F,k,s", [(1, 512, 13, 1024, 3, 1), (1, 256, 13, 255, 1, 1), (2, 64, 9, 96, 3, 2)])
def test_conv_splitk(hip, cfg, splits, B, Cc, Hh, F, k, s):
    """Split-K partial sums reduced in fixed order, then the epilogue."""
    case(f"conv split-K {splits} cfg{cfg} B{B} C{Cc} H{Hh} F{F} k{k} s{s}")
    p = k // 2
    x = synth.uniform(47, (B, Cc, Hh, Hh))
    Wt = synth.normal(48, (F, Cc * k * k), (2.0 / (Cc * k * k)) ** 0.5)
    b = synth.normal(49, (F,), 0.1)
    res = synth.normal(50, (B, F, (Hh + 2 * p - k) // s + 1, (Hh + 2 * p - k) // s + 1))
    ref = R.addvv(R.conv_forward(x, Wt, b, k, s, p, acLEAKY), res)
    dW = D(Wt)
    packed = torch.empty_like(dW)
    hip.packConvWeights(F, Cc, k, dW, packed)
    dout = torch.empty(ref.shape, dtype=torch.float32, device="cuda")
    hip.setConvAutotune(True, CONV_SPLIT_UNIT * splits + cfg)
    try:
        hip.conv2dForward(B, Cc, Hh, Hh, F, k, s, p, D(x), 0, packed, D(b), acLEAKY, dout, 0, residual=D(res),
                          weightLayout=WEIGHTS_TAP_MAJOR if k > 1 else 0)
        got = H(dout, hip)
    finally:
        hip.setConvAutotune(True, -1)
    assert R.rel_err(got, ref) <= TOL


_TAIL_REFS = {}


@pytest.mark.parametrize("base", [CONV_TAIL_BASE, CONV_TAIL_SLOT_BASE])
@pytest.mark.parametrize("cfg", [11, 13, 17])
@pytest.mark.parametrize("pieces", [2, 3, 8])
@pytest.mark.parametrize("B,Cc,Hh,F,k,s", [(4, 32, 184, 128, 3, 1), (4, 64, 184, 128, 1, 1), (4, 32, 368, 128, 3, 2)])
def test_conv_tail_split(hip, base, cfg, pieces, B, Cc, Hh, F, k, s):
    """Tail split: whole rounds of tiles (one per CU, or one per resident
    workgroup slot), the remainder cut into K pieces summed in K order by a
    second kernel, then the epilogue."""
    case(f"conv tail split {pieces} base {base} cfg{cfg} B{B} C{Cc} H{Hh} F{F} k{k} s{s}")
    p = k // 2
    OH = (Hh + 2 * p - k) // s + 1
    bm, bn = {11: (64, 64), 13: (128, 64), 17: (128, 64)}[cfg]
    tiles = -(-F // bm) * -(-(B * OH * OH) // bn)
    # more tiles than 8 workgroup slots per CU, and a partial last round for
    # every round size up to that, so the tail is cut in both modes
    assert tiles > 8 * hip.cuCount() and all(tiles % (o * hip.cuCount()) != 0 for o in range(1, 9))
    key = (B, Cc, Hh, F, k, s)
    if key not in _TAIL_REFS:
        x = synth.uniform(61, (B, Cc, Hh, Hh))
        Wt = synth.normal(62, (F, Cc * k * k), (2.0 / (Cc * k * k)) ** 0.5)
        b = synth.normal(63, (F,), 0.1)
        res = synth.normal(64, (B, F, OH, OH))
        _TAIL_REFS[key] = (x, Wt, b, res, R.addvv(R.conv_forward(x, Wt, b, k, s, p, acLEAKY), res))
    x, Wt, b, res, ref = _TAIL_REFS[key]
    dW = D(Wt)
    packed = torch.empty_like(dW)
    hip.packConvWeights(F, Cc, k, dW, packed)
    dout = torch.empty(ref.shape, dtype=torch.float32, device="cuda")
    hip.setConvAutotune(True, cfg + CONV_SPLIT_UNIT * (base + pieces))
    try:
        hip.conv2dForward(B, Cc, Hh, Hh, F, k, s, p, D(x), 0, packed, D(b), acLEAKY, dout, 0, residual=D(res),
                          weightLayout=WEIGHTS_TAP_MAJOR if k > 1 else 0)
        got = H(dout, hip)
    finally:
        hip.setConvAutotune(True, -1)
    assert R.rel_err(got, ref) <= TOL


def oracle_conv_any(x, Wt, b, kh, kw, s, pH, pW, act):
    """Conv2D (ntensors.pas:8252-8345) for any kernel shape through the
    oracle's im2col and per-image NN SGEMM, then bias and activation."""
    B = x.shape[0]
    F = Wt.shape[0]
    col = R.im2col(x, kh, kw, pH, pW, s, s)
    L = col.shape[2]
    out = np.zeros((B, F, L), np.float32)
    for i in range(B):
        R.sgemm(0, 0, F, L, col.shape[1], 1.0, Wt, Wt.shape[1], np.ascontiguousarray(col[i]), L, 0.0, out[i], L)
    out = R.forward_bias(out, b, B)
    return R.activate(out, act)


@pytest.mark.parametrize("B,Cc,Hh,Ww,F,kh,kw,s,pH,pW,tap", [(2, 8, 21, 21, 24, 5, 5, 1, 2, 2, False),
                                                           (1, 16, 30, 30, 40, 7, 7, 2, 3, 3, True),
                                                           (2, 5, 12, 16, 9, 2, 2, 2, 0, 0, False),
                                                           (2, 12, 14, 9, 20, 1, 3, 1, 0, 1, True),
                                                           (1, 32, 11, 13, 64, 3, 5, 1, 1, 2, False),
                                                           (2, 3, 33, 33, 16, 5, 5, 1, 2, 2, True)])
def test_conv_any_kernel_size(hip, B, Cc, Hh, Ww, F, kh, kw, s, pH, pW, tap):
    """Kernel sizes beyond 1x1 / 3x3 (5x5, 7x7, even, non-square) through
    tnh_conv2d_fwd in both weight layouts, against the oracle's im2col +
    SGEMM path; every LDS-staged tile configuration once."""
    case(f"conv any kernel B{B} C{Cc} {Hh}x{Ww} F{F} k{kh}x{kw} s{s} p{pH},{pW} tap{tap}")
    x = synth.uniform(150, (B, Cc, Hh, Ww))
    Wt = synth.normal(151, (F, Cc * kh * kw), (2.0 / (Cc * kh * kw)) ** 0.5)
    b = synth.normal(152, (F,), 0.1)
    ref = oracle_conv_any(x, Wt, b, kh, kw, s, pH, pW, acLEAKY)
    OH, OW = (Hh + 2 * pH - kh) // s + 1, (Ww + 2 * pW - kw) // s + 1
    dW = D(Wt)
    if tap:
        packed = torch.empty_like(dW)
        hip.packConvWeights(F, Cc, kh, dW, packed, kernelWidth=kw)
        dW = packed
    for cfg in (-1, 0, 1, 2, 3, 4, 5):
        dout = torch.empty((B, F, OH, OW), dtype=torch.float32, device="cuda")
        hip.setConvAutotune(True, cfg)
        try:
            call = dict(weightLayout=WEIGHTS_TAP_MAJOR if tap else 0, kernelWidth=kw, padWidth=pW)
            hip.conv2dForward(B, Cc, Hh, Ww, F, kh, s, pH, D(x), 0, dW, D(b), acLEAKY, dout, 0, **call)
            got = H(dout, hip)
        finally:
            hip.setConvAutotune(True, -1)
        assert R.rel_err(got.reshape(B, F, -1), ref) <= TOL, cfg


def test_conv_golden_fixture(hip):
    case("conv golden fixture (torch fp64)")
    import os

    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "conv_small.npz"))
    dout = torch.empty(g["y64"].shape, dtype=torch.float32, device="cuda")
    hip.conv2dForward(1, 3, 16, 16, 8, 3, 1, 1, D(g["x"]), 0, D(g["W"]), D(g["b"]), acLEAKY, dout, 0)
    assert R.rel_err(H(dout, hip), g["y64"]) <= TOL


def test_conv_fused_shortcut_and_strided_io(hip):
    """residual fused after the activation (== conv then addvv) and output
    written into a channel slice of a wider (route) buffer."""
    case("conv + fused shortcut + strided output")
    B, Cc, Hh, F = 2, 64, 26, 128
    x = synth.uniform(51, (B, Cc, Hh, Hh))
    Wt = synth.normal(52, (F, Cc * 9), (2.0 / (Cc * 9)) ** 0.5)
    b = synth.normal(53, (F,), 0.1)
    res = synth.normal(54, (B, F, Hh, Hh))
    y = R.conv_forward(x, Wt, b, 3, 1, 1, acLEAKY)
    ref = R.addvv(y, res)
    wide = torch.zeros((B, F + 32, Hh, Hh), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    hip.conv2dForward(B, Cc, Hh, Hh, F, 3, 1, 1, D(x), 0, D(Wt), D(b), acLEAKY, wide, 32 * Hh * Hh,
                      outBatchStride=(F + 32) * Hh * Hh, residual=D(res))
    got = H(wide, hip)
    assert np.all(got[:, :32] == 0)
    assert R.rel_err(got[:, 32:], ref) <= TOL
    # the fused add itself is one fp32 add: exact w.r.t. the GPU conv result
    plain = torch.empty((B, F, Hh, Hh), dtype=torch.float32, device="cuda")
    hip.conv2dForward(B, Cc, Hh, Hh, F, 3, 1, 1, D(x), 0, D(Wt), D(b), acLEAKY, plain, 0)
    assert np.array_equal(got[:, 32:], H(plain, hip) + res)


def test_conv_tuned_dense_then_output_beyond_2gib(hip):
    """A shape tuned with a dense output, then called with an output batch
    stride that puts image 1 beyond 2 GiB: the lean kernels cannot address
    that output, so the cached choice must not be reused (integer data: every
    tiling gives the same exact sums, so both outputs are compared bit for
    bit)."""
    case("conv tuned dense, then output beyond 2 GiB")
    B, Cc, Hh, F = 2, 64, 26, 64
    rng = np.random.default_rng(2024)
    x = rng.integers(-3, 4, (B, Cc, Hh, Hh)).astype(np.float32)
    Wt = rng.integers(-2, 3, (F, Cc * 9)).astype(np.float32)
    b = rng.integers(-5, 6, F).astype(np.float32)
    dx, dW, db = D(x), D(Wt), D(b)
    packed = torch.empty_like(dW)
    hip.packConvWeights(F, Cc, 3, dW, packed)
    dense = torch.empty((B, F, Hh, Hh), dtype=torch.float32, device="cuda")
    hip.conv2dForward(B, Cc, Hh, Hh, F, 3, 1, 1, dx, 0, packed, db, acLINEAR, dense, 0,
                      weightLayout=WEIGHTS_TAP_MAJOR)
    want = H(dense, hip)
    stride = (1 << 29) + 64  # floats: image 1 starts 2 GiB + 256 B into the buffer
    big = torch.zeros(stride + F * Hh * Hh, dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    hip.conv2dForward(B, Cc, Hh, Hh, F, 3, 1, 1, dx, 0, packed, db, acLINEAR, big, 0, outBatchStride=stride,
                      weightLayout=WEIGHTS_TAP_MAJOR)
    hip.finish()
    img0 = big[:F * Hh * Hh].cpu().numpy().reshape(F, Hh, Hh)
    img1 = big[stride:].cpu().numpy().reshape(F, Hh, Hh)
    assert np.array_equal(img0, want[0])
    assert np.array_equal(img1, want[1])
    ref = R.conv_forward(x, Wt, b, 3, 1, 1, acLINEAR)
    assert np.array_equal(want, ref)


def test_deterministic_mode_ignores_tuning_state(hip):
    """tnh_set_deterministic: the same bits whatever the tuner cached before
    (here a batch-1 13x13 layer whose tuned tiling usually cuts K), for the
    NCHW and channels-last convs and the SGEMM; results within the bound."""
    case("deterministic mode")
    B, Cc, Hh, F = 1, 512, 13, 1024
    x = synth.uniform(140, (B, Cc, Hh, Hh))
    Wt = synth.normal(141, (F, Cc * 9), (2.0 / (Cc * 9)) ** 0.5)
    b = synth.normal(142, (F,), 0.1)
    ref = R.conv_forward(x, Wt, b, 3, 1, 1, acLEAKY)
    dx, dW, db = D(x), D(Wt), D(b)
    packed = torch.empty_like(dW)
    hip.packConvWeights(F, Cc, 3, dW, packed)
    xn = D(np.ascontiguousarray(x.transpose(0, 2, 3, 1)))
    A = synth.uniform(143, (1024, 2304), -1, 1)
    Bm = synth.uniform(144, (2304, 169), -1, 1)
    dA, dB = D(A), D(Bm)

    def run():
        o = torch.empty(ref.shape, dtype=torch.float32, device="cuda")
        hip.conv2dForward(B, Cc, Hh, Hh, F, 3, 1, 1, dx, 0, packed, db, acLEAKY, o, 0, weightLayout=WEIGHTS_TAP_MAJOR)
        on = torch.empty((B, Hh, Hh, F), dtype=torch.float32, device="cuda")
        hip.conv2dForwardNHWC(B, Cc, Hh, Hh, F, 3, 1, 1, xn, 0, packed, db, acLEAKY, on, 0)
        oc = torch.empty((1024, 169), dtype=torch.float32, device="cuda")
        hip.gemm(False, False, 1024, 169, 2304, 1.0, dA, 0, 2304, dB, 0, 169, 0.0, oc, 0, 169)
        return [H(t, hip) for t in (o, on, oc)]

    run()  # the tuner caches its (possibly K-cutting) choices
    try:
        hip.setDeterministic(True)
        first = run()
        hip.setConvAutotune(False, -1)  # clears the caches, as in a fresh process
        hip.setSgemmAutotune(False, -1)
        hip.setConvAutotune(True, -1)
        hip.setSgemmAutotune(True, -1)
        second = run()
    finally:
        hip.setDeterministic(False)
    for u, v in zip(first, second):
        assert np.array_equal(u, v)
    assert R.rel_err(first[0], ref) <= TOL
    assert R.rel_err(first[1].transpose(0, 3, 1, 2), ref) <= TOL
    C = np.zeros((1024, 169), np.float32)
    R.sgemm(0, 0, 1024, 169, 2304, 1.0, A, 2304, Bm, 169, 0.0, C, 169)
    assert R.rel_err(first[2], C) <= TOL


# ------------------------------------------------------- pool / upsample ----
@pytest.mark.parametrize("size,stride,pad,shape", [(2, 2, 0, (2, 5, 19, 16)), (3, 2, 0, (2, 5, 19, 16)),
                                                   (2, 1, 1, (2, 5, 19, 16)), (3, 1, 2, (2, 5, 19, 16)),
                                                   (5, 1, 4, (2, 5, 19, 16)), (2, 2, 0, (3, 4, 10, 18)),
                                                   (2, 2, 1, (2, 3, 12, 12)), (2, 2, 0, (2, 3, 9, 7)),
                                                   (2, 2, 0, (128, 32, 32, 32))])
def test_maxpool_forward_backward_bit_exact(hip, size, stride, pad, shape):
    """Values, int64 indices and the backward scatter-add, bit-exact; the
    2x2/2 shapes cover the paired kernels (16- and 8-byte input loads, the
    config-3 layer) and the general kernel (odd width)."""
    case(f"maxpool size{size} stride{stride} pad{pad} {shape}")
    B, Cc, Hh, W = shape
    x = synth.normal(61, (B, Cc, Hh, W))
    x[0, 0, :4, :4] = 1.0  # ties
    x[-1, -1, :2, :2] = -np.inf  # a window of -inf: -MaxSingle, index -1
    x[0, -1, 2, 3] = np.nan
    out, idx = R.maxpool_fwd(x, size, stride, stride, pad)
    _, _, OH, OW = out.shape
    dout = torch.empty(out.shape, dtype=torch.float32, device="cuda")
    didx = torch.empty(out.shape, dtype=torch.int64, device="cuda")
    hip.forwardMaxPool(B, Cc, OH, OW, D(x), Cc, Hh, W, stride, stride, pad, size, didx, dout)
    assert np.array_equal(H(dout, hip), out)
    assert np.array_equal(H(didx, hip), idx)
    delta = synth.normal(62, out.shape)
    dIn0 = synth.normal(63, x.shape)
    ref = R.maxpool_bwd(idx, delta, dIn0.copy())
    ddIn = D(dIn0)
    hip.backwardMaxPool(B, Cc, OH, OW, ddIn, didx, D(delta))  # TNNCuda's 7 arguments
    assert np.array_equal(H(ddIn, hip), ref)
    # the same indexes in a buffer no forward wrote: with the geometry given
    # (tnh_maxpool_bwd_geom), and, where windows do not overlap, without it
    # (the scatter)
    other = torch.empty(out.shape, dtype=torch.int64, device="cuda")
    other.copy_(didx)
    ddIn = D(dIn0)
    hip.backwardMaxPool(B, Cc, OH, OW, ddIn, other, D(delta), geometry=(Hh, W, stride, stride, pad, size))
    assert np.array_equal(H(ddIn, hip), ref)
    if size <= stride:
        hip.forwardMaxPool(B, Cc, OH, OW, D(x), Cc, Hh, W, stride, stride, pad, size, other, dout)
        H(other, hip)
        del other  # forget nothing: the buffer of a fresh allocation below may reuse the address
        fresh = torch.empty(out.shape, dtype=torch.int64, device="cuda")
        fresh.copy_(didx)
        ddIn = D(dIn0)
        hip.backwardMaxPool(B, Cc, OH, OW, ddIn, fresh, D(delta))
        assert np.array_equal(H(ddIn, hip), ref)


@pytest.mark.parametrize("c,outC", [(64, 4), (30, 7), (3, 5)])
def test_maxpool_depth_bit_exact(hip, c, outC):
    """maxpool_depth (outC != c, the image size kept): values and int64
    indices against the oracle bit for bit (NaN, -inf and ties included;
    outC > c leaves empty groups), and TNNCuda's 7-argument backward
    scatters through them."""
    case(f"maxpool_depth c{c} outC{outC}")
    B, Hh, W = 2, 9, 13
    x = synth.normal(65, (B, c, Hh, W))
    x[0, :, 0, 0] = 1.0
    x[1, :, 2, 3] = -np.inf
    x[0, 0, 4, 4] = np.nan
    out, idx = R.maxpool_depth_fwd(x, outC)
    dout = torch.empty(out.shape, dtype=torch.float32, device="cuda")
    didx = torch.empty(out.shape, dtype=torch.int64, device="cuda")
    hip.forwardMaxPool(B, outC, Hh, W, D(x), c, Hh, W, 1, 1, 0, 1, didx, dout)
    assert np.array_equal(H(dout, hip), out)
    assert np.array_equal(H(didx, hip), idx)
    delta = synth.normal(66, out.shape)
    dIn0 = synth.normal(67, x.shape)
    ref = R.maxpool_bwd(idx, delta, dIn0.copy())
    ddIn = D(dIn0)
    hip.backwardMaxPool(B, outC, Hh, W, ddIn, didx, D(delta))
    assert np.array_equal(H(ddIn, hip), ref)
    with pytest.raises(TNHError, match="maxpool_depth"):
        hip.forwardMaxPool(B, outC, Hh - 1, W, D(x), c, Hh, W, 1, 1, 0, 1, didx, dout)


def test_maxpool_inference_no_indexes(hip):
    case("maxpool without indexes")
    x = synth.normal(64, (2, 3, 8, 8))
    out, _ = R.maxpool_fwd(x, 2, 2, 2, 0, with_idx=False)
    dout = torch.empty(out.shape, dtype=torch.float32, device="cuda")
    hip.forwardMaxPool(2, 3, 4, 4, D(x), 3, 8, 8, 2, 2, 0, 2, None, dout)
    assert np.array_equal(H(dout, hip), out)


@pytest.mark.parametrize("stride,scale", [(2, 1.0), (2, 0.5), (3, 1.0)])
def test_upsample_bit_exact(hip, stride, scale):
    case(f"upsample stride{stride} scale{scale}")
    B, Cc, h, w = 2, 7, 13, 11
    x = synth.normal(71, (B, Cc, h, w))
    ref = R.upsample_fwd(x, stride, scale)
    dout = torch.empty(ref.shape, dtype=torch.float32, device="cuda")
    hip.upSample(B, Cc, h, w, D(x), stride, 1, scale, dout)
    assert np.array_equal(H(dout, hip), ref)
    d = synth.normal(72, ref.shape)
    dIn0 = synth.normal(73, x.shape)
    refb = R.upsample_bwd(dIn0.copy(), d, stride, scale)
    ddIn = D(dIn0)
    hip.upSample(B, Cc, h, w, ddIn, stride, 0, scale, D(d))
    assert np.array_equal(H(ddIn, hip), refb)


# ------------------------------------------------------------ element-wise ----
def test_bias_scale_activation_bit_exact(hip):
    case("forward_bias / forward_scale / activate / derive")
    B, F, P = 3, 17, 50
    x = synth.normal(81, (B, F, P))
    b = synth.normal(82, (F,))
    dx = D(x)
    hip.forwardBias(x.size, dx, 0, F, D(b), 1, B)
    ref = R.forward_bias(x.copy(), b, B)
    assert np.array_equal(H(dx, hip), ref)
    hip.forwardScale(x.size, dx, 0, F, D(b), 1, B)
    ref = R.forward_scale(ref, b, B)
    assert np.array_equal(H(dx, hip), ref)
    v = np.concatenate([x.ravel(), np.array([0.0, -0.0, np.nan, -np.inf, np.inf, -1e-40], np.float32)])
    dv = D(v)
    hip.ActivateArray(v.size, dv, 0, acLEAKY)
    refv = R.activate(v.copy(), acLEAKY)
    assert np.array_equal(H(dv, hip).view(np.uint32), refv.view(np.uint32))
    delta = synth.normal(83, v.shape)
    dd = D(delta)
    hip.DeriveArray(v.size, D(refv), 0, acLEAKY, dd)
    assert np.array_equal(H(dd, hip), R.derive(refv, acLEAKY, delta.copy()))


def test_copy_fill_axpy_addvv_route(hip):
    case("copy / fill / axpy / addvv / route")
    a = synth.normal(91, (1000,))
    b = synth.normal(92, (1000,))
    da, db = D(a), D(b)
    dc = torch.empty(1000, dtype=torch.float32, device="cuda")
    hip.addvv(1000, da, 0, 1, db, 0, 1, dc, 0, 1)
    assert np.array_equal(H(dc, hip), a + b)
    hip.addvv(333, da, 1, 3, db, 0, 3, dc, 0, 3)  # strided
    got = H(dc, hip)
    assert np.array_equal(got[0:999:3], a[1::3][:333] + b[0:999:3])
    hip.axpy(1000, 0.25, da, 0, 1, db, 0, 1)
    assert np.array_equal(H(db, hip), b + np.float32(0.25) * a)
    hip.fill(500, dc, 1, 7.0, 2)
    got = H(dc, hip)
    assert np.all(got[1:1000:2] == 7.0)
    # contiguous: 16-byte stores when aligned (offset 4), single ones when not
    # (offset 1, and 998 elements); the elements around the range stay
    for off, n in ((4, 992), (1, 996), (0, 998)):
        hip.copy(1000, da, 0, 1, dc, 0, 1)
        hip.fill(n, dc, off, -2.5, 1)
        want = a.copy()
        want[off:off + n] = -2.5
        assert np.array_equal(H(dc, hip), want), (off, n)
    hip.copy(1000, da, 0, 1, dc, 0, 1)
    assert np.array_equal(H(dc, hip), a)
    hip.scale(1000, 3.0, dc, 1)
    assert np.array_equal(H(dc, hip), np.float32(3.0) * a)
    s0, s1 = synth.normal(93, (2, 3, 4)), synth.normal(94, (2, 5, 4))
    dst = torch.empty((2, 8, 4), dtype=torch.float32, device="cuda")
    hip.concat(2, [D(s0), D(s1)], [12, 20], dst)
    assert np.array_equal(H(dst, hip), np.concatenate([s0, s1], axis=1))


def test_yolo_head_bit_exact(hip):
    case("yolo head logistic")
    x = synth.normal(95, (2, 3 * 85, 13, 13), 3.0)
    ref = R.yolo_fwd(x, 3, 80, exact=True)
    dout = torch.empty(x.shape, dtype=torch.float32, device="cuda")
    hip.yoloForward(2, 3, 80, 13, 13, D(x), dout)
    assert np.array_equal(H(dout, hip), ref)


def test_yolo_logistic_pinned_values(hip):
    """The yolo kernels (NCHW and channels-last) on the committed exact-mode
    logistic table (hand-derivable cases, the clamps, +-inf, fraction-1/2
    points; test_oracle_logistic.py) and NaN: bit for bit."""
    from tests.test_oracle_logistic import TABLE, from_bits

    case("yolo logistic pinned values")
    vals = np.array([from_bits(xb) for xb, _ in TABLE] + [np.nan], np.float32)
    P = vals.size
    x = np.zeros((1, 6, 1, P), np.float32)  # one anchor, one class: entries 0, 1, 4, 5 get the logistic
    for e in (0, 1, 4, 5):
        x[0, e, 0] = vals
    want = np.array([yb for _, yb in TABLE], np.uint32)
    dout = torch.empty(x.shape, dtype=torch.float32, device="cuda")
    hip.yoloForward(1, 1, 1, 1, P, D(x), dout)
    got = H(dout, hip)
    xn = np.ascontiguousarray(x.transpose(0, 2, 3, 1))  # [1][1][P][6] channels-last
    dout2 = torch.empty(x.shape, dtype=torch.float32, device="cuda")
    hip.yoloForwardNHWC(1, 1, 1, 1, P, D(xn), 0, 6, dout2)
    got2 = H(dout2, hip)
    for g in (got, got2):
        for e in (0, 1, 4, 5):
            assert np.array_equal(g[0, e, 0, :-1].view(np.uint32), want), e
            assert np.isnan(g[0, e, 0, -1])
        assert np.array_equal(g[0, 2:4], x[0, 2:4])


def test_bn_normalize_vs_oracle_exact(hip):
    case("bn normalize (exact division)")
    B, F, P = 2, 6, 40
    x = synth.normal(96, (B, F, P))
    mean = synth.normal(97, (F,))
    var = synth.uniform(98, (F,), 0.1, 3.0)
    var[2] = 0.0
    dx = D(x)
    hip.blockNormalize(x.size, dx, 0, F, D(mean), D(var), B)
    assert np.array_equal(H(dx, hip), R.bn_normalize(x.copy(), mean, var, B, exact=True))


@pytest.mark.parametrize("B,F,P", [(2, 6, 40), (3, 5, 1), (2, 7, 9), (4, 16, 64)])
def test_normalize_tnncuda_signature(hip, B, F, P):
    """TNNCuda.normalize's argument list (srcSize = channels, dstSize,
    groups = batch, strided statistics, destination offset) with the CPU
    clamps, bit-exact against the oracle: blocks of one element clamp the
    variance, longer blocks the standard deviation; NaN and zero variances."""
    case(f"normalize (TNNCuda signature) B{B} F{F} P{P}")
    x = synth.normal(120, (B, F, P))
    mean = synth.normal(121, (2 * F,))
    var = synth.uniform(122, (3 * F,), 0.1, 3.0)
    var[0], var[3] = 0.0, np.nan
    ref = R.bn_normalize(x.copy(), np.ascontiguousarray(mean[::2]), np.ascontiguousarray(var[::3]), B)
    buf = np.concatenate([np.full(5, 9.0, np.float32), x.ravel()])
    dbuf = D(buf)
    hip.normalize(F, x.size, B, D(mean), 2, D(var), 3, dbuf, 5)
    got = H(dbuf, hip)
    assert np.array_equal(got[:5], buf[:5])
    assert np.array_equal(got[5:].reshape(x.shape), ref, equal_nan=True)


@pytest.mark.parametrize("B,F,P", [(2, 6, 40), (3, 5, 1), (1, 7, 9)])
def test_forward_scale_add_bit_exact(hip, B, F, P):
    """TNNCuda.forwardScaleAdd = the CPU's forwardScale then forwardBias."""
    case(f"forward scale add B{B} F{F} P{P}")
    x = synth.normal(123, (B, F, P))
    sc = synth.normal(124, (F,))
    bi = synth.normal(125, (F,))
    ref = R.forward_bias(R.forward_scale(x.copy(), sc, B), bi, B)
    dx = D(x)
    hip.forwardScaleAdd(x.size, dx, 0, F, D(sc), D(bi), 1, B)
    assert np.array_equal(H(dx, hip), ref)


@pytest.mark.parametrize("B,F,P,act,norm", [(4, 32, 1024, acLEAKY, True), (3, 5, 7, acLEAKY, True),
                                            (2, 10, 1, acLINEAR, False), (2, 64, 64, acLOGISTIC, True)])
def test_bn_forward_equals_the_reference_sequence(hip, B, F, P, act, norm):
    """tnh_bn_forward == copy, blockNormalize, copy, forwardScale,
    forwardBias, activate (nbaselayer.pas:335-368 + the layer activation) on
    the GPU, bit for bit, and == the oracle's normalize / scale / bias /
    activation."""
    case(f"bn forward B{B} F{F} P{P} act{act} xnorm{norm}")
    x = synth.normal(126, (B, F, P))
    mean = synth.normal(127, (F,))
    var = synth.uniform(128, (F,), 0.1, 3.0)
    var[0] = 0.0
    sc, bi = synth.normal(129, (F,)), synth.normal(130, (F,))
    xn_ref = R.bn_normalize(x.copy(), mean, var, B)
    out_ref = R.activate(R.forward_bias(R.forward_scale(xn_ref.copy(), sc, B), bi, B), act)
    dx, dm, dv, ds, db = D(x), D(mean), D(var), D(sc), D(bi)
    dxn = torch.empty_like(dx) if norm else None
    dout = torch.empty_like(dx)
    hip.bnForward(x.size, F, B, dx, dxn, dout, dm, dv, ds, db, act)
    seq = dx.clone()
    hip.blockNormalize(x.size, seq, 0, F, dm, dv, B)
    seqn = seq.clone()
    hip.forwardScale(x.size, seq, 0, F, ds, 1, B)
    hip.forwardBias(x.size, seq, 0, F, db, 1, B)
    hip.ActivateArray(x.size, seq, 0, act)
    got = H(dout, hip)
    assert np.array_equal(got, H(seq, hip))
    if act != acLOGISTIC:  # the oracle's logistic is the reference polynomial, the layer activation is expf
        assert np.array_equal(got, out_ref)
    if norm:
        assert np.array_equal(H(dxn, hip), xn_ref)
        assert np.array_equal(H(dxn, hip), H(seqn, hip))


# --------------------------------------------------------------- errors ----
def test_invalid_arguments_raise(hip):
    case("argument checks")
    for c in CONV_RETIRED_CFGS:  # retired tile ids are refused, not silently replaced
        with pytest.raises(TNHError):
            hip.setConvAutotune(True, c)
    hip.setConvAutotune(True, -1)
    dx = D(np.zeros(16, np.float32))
    with pytest.raises(TNHError):
        hip.gemm(0, 0, 4, 4, 4, 1.0, dx, 0, 2, dx, 0, 4, 0.0, dx, 0, 4)  # lda < K
    with pytest.raises(TNHError):
        hip.conv2dForward(1, 1, 4, 4, 1, 33, 1, 16, dx, 0, dx, None, acLEAKY, dx, 0)  # kernel above 32
    with pytest.raises(TNHError):
        hip.ActivateArray(4, dx, 0, 123)
    with pytest.raises(TNHError):
        hip.forwardMaxPool(1, 1, 3, 3, dx, 1, 4, 4, 2, 2, 0, 2, None, dx)  # wrong out dims
    hip.finish()  # the context stays usable after rejected calls
