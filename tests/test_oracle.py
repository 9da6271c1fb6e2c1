"""Pins the CPU oracle (oracle/refcpu.c) against what the mathematics and
independent library routines fix.  The reference ships no tests, fixtures or
golden vectors for this path (it is Free Pascal and cannot be built here), so
every expected value below is either (a) exact integer arithmetic, (b) a
hand-derived value for an input built so that a plausible mistake (sequential
instead of 8-lane dot, mul+add instead of FMA, wrong accumulation order, wrong
window offset) gives a different answer, (c) a library routine (numpy fp64
matmul, torch unfold/fold/max_pool2d/interpolate/conv2d), or (d) a committed
golden fixture under tests/golden/ made by tests/golden/make_golden.py from
library routines.
"""
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as Fn

from oracle import refcpu as R

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
TOL = 1e-5  # per-tensor max|g - r| / max|r| for GEMM / conv


def op(X, t):
    return X.T if t else X


def rand_gemm(rng, ta, tb, M, N, K, lo=-1.0, hi=1.0):
    A = rng.uniform(lo, hi, (K, M) if ta else (M, K)).astype(np.float32)
    B = rng.uniform(lo, hi, (N, K) if tb else (K, N)).astype(np.float32)
    return A, B


# ---------------------------------------------------------------- SGEMM ----
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_sgemm_exact_integer(ta, tb):
    """Small integers with every partial sum < 2^24: any order is exact."""
    rng = np.random.default_rng(1)
    M, N, K = 23, 41, 37
    A = rng.integers(-8, 9, (K, M) if ta else (M, K)).astype(np.float32)
    B = rng.integers(-8, 9, (N, K) if tb else (K, N)).astype(np.float32)
    C0 = rng.integers(-50, 51, (M, N)).astype(np.float32)
    C = C0.copy()
    R.sgemm(ta, tb, M, N, K, 2.0, A, A.shape[1], B, B.shape[1], 3.0, C, N)
    ref = 2 * op(A, ta).astype(np.int64) @ op(B, tb).astype(np.int64) + 3 * C0.astype(np.int64)
    assert np.array_equal(C, ref.astype(np.float32))


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_sgemm_vs_fp64(ta, tb):
    rng = np.random.default_rng(2)
    M, N, K = 64, 97, 300
    A, B = rand_gemm(rng, ta, tb, M, N, K)
    C = np.zeros((M, N), np.float32)
    R.sgemm(ta, tb, M, N, K, 1.0, A, A.shape[1], B, B.shape[1], 0.0, C, N)
    ref = op(A, ta).astype(np.float64) @ op(B, tb).astype(np.float64)
    assert R.rel_err(C, ref) < TOL


def test_sgemm_nn_uses_fma():
    """C = (-1-2^-11)*1 + (1+2^-12)^2 = 2^-24 exactly; a fused multiply-add
    chain (saxpy_avx2's vfmadd231ps) returns it, mul-then-add returns 0."""
    a0, e = -1 - 2.0 ** -11, 1 + 2.0 ** -12
    for ta in (0, 1):
        A = np.array([[a0, e]], np.float32)
        if ta:
            A = A.T.copy()
        B = np.array([[1.0], [e]], np.float32)
        C = np.zeros((1, 1), np.float32)
        R.sgemm(ta, 0, 1, 1, 2, 1.0, A, A.shape[1], B, 1, 0.0, C, 1)
        assert C[0, 0] == np.float32(2.0 ** -24)


def test_sgemm_nt_eight_lane_dot():
    """sdot_avx2 keeps 8 lane accumulators and reduces (l, l+4) pairs first.
    Case 1: a = [2^24, 1x7, -2^24, 0x7]: lanes give the exact 7, a sequential
    dot gives 0.  Case 2: lane values [2^24,1,1,1,-2^24,1,1,1]: the (l,l+4)
    then (t0+t1)+(t2+t3) reduction gives 6, sequential 3, adjacent-pair hadd 5."""
    b = np.ones((1, 16), np.float32)
    a = np.zeros((1, 16), np.float32)
    a[0, 0], a[0, 1:8], a[0, 8] = 2.0 ** 24, 1.0, -(2.0 ** 24)
    C = np.zeros((1, 1), np.float32)
    R.sgemm(0, 1, 1, 1, 16, 1.0, a, 16, b, 16, 0.0, C, 1)
    assert C[0, 0] == 7.0
    a2 = np.array([[2.0 ** 24, 1, 1, 1, -(2.0 ** 24), 1, 1, 1]], np.float32)
    C[:] = 0
    R.sgemm(0, 1, 1, 1, 8, 1.0, a2, 8, np.ones((1, 8), np.float32), 8, 0.0, C, 1)
    assert C[0, 0] == 6.0


def test_sgemm_nt_masked_tail():
    """K = 11: the 3 tail elements land in lanes 0-2 (vmaskmovps), giving
    acc = [2^24+1 -> 2^24 ...]; exact-integer tail check against fp64."""
    rng = np.random.default_rng(3)
    A = rng.integers(-5, 6, (3, 11)).astype(np.float32)
    B = rng.integers(-5, 6, (4, 11)).astype(np.float32)
    C = np.zeros((3, 4), np.float32)
    R.sgemm(0, 1, 3, 4, 11, 1.0, A, 11, B, 11, 0.0, C, 4)
    assert np.array_equal(C, (A.astype(np.int64) @ B.T.astype(np.int64)).astype(np.float32))


def test_sgemm_alpha_beta_closed_forms():
    rng = np.random.default_rng(4)
    M, N, K = 9, 13, 5
    A, B = rand_gemm(rng, 0, 0, M, N, K)
    C0 = rng.standard_normal((M, N)).astype(np.float32)
    # alpha = 0: C = beta*C exactly (fma(0*a, b, beta*c) = beta*c)
    C = C0.copy()
    R.sgemm(0, 0, M, N, K, 0.0, A, K, B, N, 0.5, C, N)
    assert np.array_equal(C, (np.float32(0.5) * C0).astype(np.float32))
    # K = 1, beta = 0: C = fl(fl(alpha*a) * b)
    C = C0.copy()
    R.sgemm(0, 0, M, N, 1, 3.0, A[:, :1].copy(), 1, B[:1].copy(), N, 0.0, C, N)
    assert np.array_equal(C, (np.float32(3.0) * A[:, :1]) * B[:1])


def test_sgemm_thread_count_independent():
    rng = np.random.default_rng(5)
    A, B = rand_gemm(rng, 0, 0, 33, 70, 19)
    outs = []
    for p in (1, 3, 8):
        R.set_threads(p)
        C = np.zeros((33, 70), np.float32)
        R.sgemm(0, 0, 33, 70, 19, 1.0, A, 19, B, 70, 0.0, C, 70)
        outs.append(C)
    R.set_threads(0)
    assert all(np.array_equal(outs[0], o) for o in outs[1:])


def test_sgemm_golden_fixture():
    """Committed fixture: float64 products of seeded inputs (make_golden.py)."""
    g = np.load(os.path.join(GOLDEN, "sgemm_small.npz"))
    for v in ("nn", "nt", "tn", "tt"):
        ta, tb = int(v[0] == "t"), int(v[1] == "t")
        A, B, ref = g[f"{v}_A"], g[f"{v}_B"], g[f"{v}_C64"]
        M, N = ref.shape
        C = np.zeros((M, N), np.float32)
        R.sgemm(ta, tb, M, N, A.shape[0] if ta else A.shape[1], 1.0, A, A.shape[1], B, B.shape[1], 0.0, C, N)
        assert R.rel_err(C, ref) < TOL


# -------------------------------------------------------------- im2col ----
def test_im2col_literal():
    """3x3 image 1..9, 3x3 kernel, pad 1, stride 1: hand-written rows."""
    x = np.arange(1, 10, dtype=np.float32).reshape(1, 1, 3, 3)
    col = R.im2col(x, 3, 3, 1, 1, 1, 1)[0]
    assert col.shape == (9, 9)
    assert col[0].tolist() == [0, 0, 0, 0, 1, 2, 0, 4, 5]  # (ky,kx) = (0,0)
    assert col[4].tolist() == list(range(1, 10))           # centre tap
    assert col[8].tolist() == [5, 6, 0, 8, 9, 0, 0, 0, 0]  # (2,2)
    col2 = R.im2col(x, 3, 3, 1, 1, 2, 2)[0]                 # stride 2 -> 2x2 outputs
    assert col2[0].tolist() == [0, 0, 0, 5]
    assert col2[8].tolist() == [5, 0, 0, 0]


@pytest.mark.parametrize("shape,k,p,s,d", [((2, 3, 11, 13), 3, 1, 1, 1), ((1, 4, 12, 10), 3, 1, 2, 1),
                                           ((2, 2, 9, 9), 3, 2, 1, 2), ((1, 5, 8, 8), 1, 0, 1, 1),
                                           ((1, 3, 7, 6), 5, 2, 3, 1)])
def test_im2col_vs_torch_unfold(shape, k, p, s, d):
    rng = np.random.default_rng(6)
    x = rng.standard_normal(shape).astype(np.float32)
    got = R.im2col(x, k, k, p, p, s, s, d, d)
    ref = Fn.unfold(torch.from_numpy(x), k, dilation=d, padding=p, stride=s).numpy()
    assert np.array_equal(got, ref)


# -------------------------------------------------------------- col2im ----
@pytest.mark.parametrize("shape,k,p,s", [((2, 3, 9, 7), 3, 1, 1), ((1, 4, 10, 8), 3, 1, 2), ((3, 2, 6, 6), 1, 0, 1)])
def test_col2im_adjoint_and_fold(shape, k, p, s):
    """<im2col x, y> == <x, col2im y> exactly on small integers, and
    col2im(y) == torch fold(y) (library)."""
    rng = np.random.default_rng(7)
    x = rng.integers(-4, 5, shape).astype(np.float32)
    col = R.im2col(x, k, k, p, p, s, s)
    y = rng.integers(-4, 5, col.shape).astype(np.float32)
    im = np.zeros(shape, np.float32)
    R.col2im(y, im, k, k, p, p, s, s)
    lhs = int((col.astype(np.int64) * y.astype(np.int64)).sum())
    rhs = int((x.astype(np.int64) * im.astype(np.int64)).sum())
    assert lhs == rhs
    ref = Fn.fold(torch.from_numpy(y), shape[2:], k, padding=p, stride=s).numpy()
    assert np.array_equal(im, ref)


def test_col2im_accumulation_order():
    """One pixel with existing value 2^24 receiving +1, +1, -2^24 (in kernel
    tap order): the reference adds into the image value first, so the result
    is ((2^24+1)+1)-2^24 = 0 in fp32 (ties to even), not 2 (sum-then-add)."""
    # 1 channel, 1x3 image, 1x3 kernel, pad 1, stride 1 -> OW = 3; pixel x=1
    # receives col[kx][ox] with ox = 1 - (kx - 1) = 2 - kx: taps kx=0,1,2.
    im = np.array([[[[0.0, 2.0 ** 24, 0.0]]]], np.float32)
    col = np.zeros((1, 3, 3), np.float32)
    col[0, 0, 2], col[0, 1, 1], col[0, 2, 0] = 1.0, 1.0, -(2.0 ** 24)
    R.col2im(col, im, 1, 3, 0, 1, 1, 1)
    assert im[0, 0, 0, 1] == 0.0


# ------------------------------------------------------ bias / leaky ------
def test_bias_scale_leaky_closed_forms():
    rng = np.random.default_rng(8)
    x = rng.standard_normal((2, 3, 4, 5)).astype(np.float32)
    b = rng.standard_normal(3).astype(np.float32)
    got = R.forward_bias(x.copy(), b, 2)
    assert np.array_equal(got, x + b[None, :, None, None])
    got = R.forward_scale(x.copy(), b, 2)
    assert np.array_equal(got, x * b[None, :, None, None])
    v = np.array([-1.0, 0.0, -0.0, 2.5, np.nan, -3e-39, -np.inf], np.float32)
    out = R.activate(v.copy(), 9)  # acLEAKY
    assert out[0] == np.float32(-0.1)                     # 0.1f * -1
    assert out[0].view(np.uint32) == np.uint32(0xBDCCCCCD)
    assert out[1] == 0 and np.signbit(out[2])             # -0 passes through
    assert out[3] == 2.5 and np.isnan(out[4])
    assert out[5] == np.float32(0.1) * np.float32(-3e-39)
    assert out[6] == -np.inf
    d = np.ones(4, np.float32)
    R.derive(np.array([-1, 0, 1, 2], np.float32), 9, d)
    assert d.tolist() == [np.float32(0.1), np.float32(0.1), 1.0, 1.0]


# ----------------------------------------------------------- maxpool ------
def to_global(idx_plane, B, C, H, W):
    """torch per-plane flat index -> the reference's global flat index."""
    planes = np.arange(B * C).reshape(B, C, 1, 1)
    return idx_plane + planes * H * W


@pytest.mark.parametrize("size,stride", [(2, 2), (3, 2), (3, 3)])
def test_maxpool_vs_torch(size, stride):
    rng = np.random.default_rng(9)
    B, C, H, W = 2, 3, 12, 10
    x = rng.standard_normal((B, C, H, W)).astype(np.float32)
    out, idx = R.maxpool_fwd(x, size, stride, stride, 0)
    rv, ri = Fn.max_pool2d(torch.from_numpy(x), size, stride, return_indices=True)
    assert np.array_equal(out, rv.numpy())
    assert np.array_equal(idx, to_global(ri.numpy(), B, C, H, W))


def test_maxpool_pad_offset():
    """size 2, stride 1, pad 1 (darknet tiny style): offset -1 div 2 = 0 and
    OH = (H + 1 - 2) + 1 = H, i.e. windows hang over the bottom/right edge:
    equals torch max_pool2d on the input padded with -inf on bottom/right."""
    rng = np.random.default_rng(10)
    B, C, H, W = 1, 2, 6, 7
    x = rng.standard_normal((B, C, H, W)).astype(np.float32)
    out, idx = R.maxpool_fwd(x, 2, 1, 1, 1)
    xp = Fn.pad(torch.from_numpy(x), (0, 1, 0, 1), value=-np.inf)
    rv, ri = Fn.max_pool2d(xp, 2, 1, return_indices=True)
    assert out.shape == (B, C, H, W) and np.array_equal(out, rv.numpy())
    ri = ri.numpy()
    ry, rx = ri // (W + 1), ri % (W + 1)
    assert np.array_equal(idx, to_global(ry * W + rx, B, C, H, W))


def test_maxpool_ties_and_empty_window():
    """Ties keep the first maximum in scan order (strict '>'); a window of
    -inf yields -MaxSingle and index -1 (nMaxPoolLayer.pas:294-312)."""
    x = np.array([[[[1, 1], [1, 1]]]], np.float32)
    out, idx = R.maxpool_fwd(x, 2, 2, 2, 0)
    assert out[0, 0, 0, 0] == 1 and idx[0, 0, 0, 0] == 0
    x = np.full((1, 1, 2, 2), -np.inf, np.float32)
    out, idx = R.maxpool_fwd(x, 2, 2, 2, 0)
    assert out[0, 0, 0, 0] == -np.finfo(np.float32).max and idx[0, 0, 0, 0] == -1


def test_maxpool_backward_skips_empty_windows():
    """An index of -1 (a window with no tap above -MaxSingle) contributes
    nothing: the reference's loop would add into element -1, outside the
    tensor.  The guard in front of the oracle's buffer stays untouched."""
    x = np.full((1, 1, 4, 4), -np.inf, np.float32)
    x[0, 0, 2:, 2:] = 1.0
    _, idx = R.maxpool_fwd(x, 2, 2, 2, 0)
    assert (idx == -1).sum() == 3
    buf = np.zeros(1 + x.size, np.float32)
    buf[0] = 7.0  # element -1 of the view below
    dIn = buf[1:]
    R.maxpool_bwd(idx, np.full(idx.shape, 2.0, np.float32), dIn)
    assert buf[0] == 7.0
    assert dIn.sum() == 2.0 and dIn[idx[0, 0, 1, 1]] == 2.0


def test_maxpool_backward_scatter():
    rng = np.random.default_rng(11)
    x = rng.standard_normal((2, 2, 6, 6)).astype(np.float32)
    _, idx = R.maxpool_fwd(x, 3, 1, 1, 0)  # overlapping windows: collisions
    d = rng.integers(-5, 6, idx.shape).astype(np.float32)
    dIn = np.zeros(x.shape, np.float32)
    R.maxpool_bwd(idx, d, dIn)
    ref = np.zeros(x.size, np.int64)
    np.add.at(ref, idx.ravel(), d.ravel().astype(np.int64))
    assert np.array_equal(dIn.ravel(), ref.astype(np.float32))


def _maxpool_depth_brute(x, outC):
    """nMaxPoolLayer.pas:372-399 as written: loops over b, i, j, g, then
    k = g, g + outC, ... < c with a strict '>' from -MaxSingle."""
    B, c, h, w = x.shape
    flat = x.ravel()
    out = np.zeros((B, outC, h, w), np.float32)
    idx = np.zeros((B, outC, h, w), np.int64)
    for b in range(B):
        for i in range(h):
            for j in range(w):
                for g in range(outC):
                    m, mi, k = -np.finfo(np.float32).max, -1, g
                    while k < c:
                        ii = j + w * (i + h * (k + c * b))
                        if flat[ii] > m:
                            m, mi = flat[ii], ii
                        k += outC
                    out[b, g, i, j], idx[b, g, i, j] = m, mi
    return out, idx


@pytest.mark.parametrize("c,outC", [(8, 1), (8, 3), (6, 2), (2, 4)])
def test_maxpool_depth_vs_loops_and_torch(c, outC):
    """maxpool_depth: against the layer's loops run literally on a small
    input (ties from integer values keep the first channel; outC > c leaves
    groups with no channel at -MaxSingle / -1), and, for outC dividing c,
    the values against torch's max over the channel groups."""
    rng = np.random.default_rng(c * 10 + outC)
    x = rng.integers(-3, 4, (2, c, 3, 5)).astype(np.float32)
    x[0, 0, 0, 0] = np.nan  # never beats anything ('>' is false)
    out, idx = R.maxpool_depth_fwd(x, outC)
    ref, ridx = _maxpool_depth_brute(x, outC)
    assert np.array_equal(out, ref) and np.array_equal(idx, ridx)
    if c % outC == 0:
        t = torch.from_numpy(np.nan_to_num(x, nan=-np.inf)).reshape(2, c // outC, outC, 3, 5).amax(1)
        assert np.array_equal(out, t.numpy())
    # backward through the depth indices: every input receives at most one delta
    d = rng.integers(-5, 6, idx.shape).astype(np.float32)
    dIn = np.zeros(x.shape, np.float32)
    R.maxpool_bwd(idx, d, dIn)
    ref = np.zeros(x.size, np.float32)
    for o, k in zip(range(idx.size), idx.ravel()):
        if k >= 0:
            ref[k] += d.ravel()[o]
    assert np.array_equal(dIn.ravel(), ref)


# ---------------------------------------------------------- upsample ------
def test_upsample_vs_torch():
    rng = np.random.default_rng(12)
    x = rng.standard_normal((2, 3, 5, 4)).astype(np.float32)
    got = R.upsample_fwd(x, 2)
    ref = Fn.interpolate(torch.from_numpy(x), scale_factor=2, mode="nearest").numpy()
    assert np.array_equal(got, ref)
    got3 = R.upsample_fwd(x, 3, 0.5)
    ref3 = np.float32(0.5) * Fn.interpolate(torch.from_numpy(x), scale_factor=3, mode="nearest").numpy()
    assert np.array_equal(got3, ref3)


def test_upsample_backward_integers():
    rng = np.random.default_rng(13)
    d = rng.integers(-9, 10, (2, 3, 8, 6)).astype(np.float32)
    dIn = rng.integers(-9, 10, (2, 3, 4, 3)).astype(np.float32)
    ref = dIn + d.reshape(2, 3, 4, 2, 3, 2).sum(axis=(3, 5))
    R.upsample_bwd(dIn, d, 2)
    assert np.array_equal(dIn, ref)


# ----------------------------------------------------------------- BN ------
def test_bn_normalize_and_fuse():
    rng = np.random.default_rng(14)
    x = rng.standard_normal((2, 4, 3, 3)).astype(np.float32)
    mean = rng.standard_normal(4).astype(np.float32)
    var = rng.uniform(0.5, 2.0, 4).astype(np.float32)
    var[1] = 0.0  # clamp: max(sqrt(0), 1e-6)
    got = R.bn_normalize(x.copy(), mean, var, 2, exact=True)
    d = np.maximum(np.sqrt(var.astype(np.float64)), 1e-6)
    ref = (x - mean[None, :, None, None].astype(np.float64)) / d[None, :, None, None]
    assert np.max(np.abs(got - ref) / np.maximum(np.abs(ref), 1e-30)) < 2 ** -22
    # NaN variance: Pascal's Max(d, eps) = d > eps ? d : eps gives eps
    xn = np.ones((1, 2, 2, 2), np.float32)
    got_nan = R.bn_normalize(xn.copy(), np.zeros(2, np.float32), np.array([np.nan, 4.0], np.float32), 1)
    assert np.all(got_nan[0, 0] == np.float32(1e6)) and np.all(got_nan[0, 1] == np.float32(0.5))
    faithful = R.bn_normalize(x.copy(), mean, var, 2, exact=False)  # rcpss: ~12 bits
    assert np.max(np.abs(faithful - ref) / np.maximum(np.abs(ref), 1)) < 1.5 * 2 ** -12 * 4
    # folding: conv(W') + b' == BN(conv(W) + b) within the per-tensor tolerance
    xin = rng.uniform(0, 1, (1, 3, 8, 8)).astype(np.float32)
    W = rng.normal(0, 0.2, (4, 27)).astype(np.float32)
    b = rng.normal(0, 0.1, 4).astype(np.float32)
    scales = rng.uniform(0.5, 1.5, 4).astype(np.float32)
    var = rng.uniform(0.5, 2.0, 4).astype(np.float32)
    y = R.conv_forward(xin, W, np.zeros(4, np.float32), 3, 1, 1, 4)
    y = R.bn_normalize(y, mean, var, 1)
    y = R.forward_scale(y, scales, 1)
    y = R.forward_bias(y, b, 1)
    Wf, bf = R.fuse_bn(W, b, scales, mean, var)  # b' = b - m*g', W' = W*g'
    yf = R.conv_forward(xin, Wf, bf, 3, 1, 1, 4)
    ref = y.astype(np.float64)
    assert R.rel_err(yf, ref) < 1e-5


# --------------------------------------------------------- conv layer ------
@pytest.mark.parametrize("C,F,H,k,s,p,act", [(3, 16, 20, 3, 1, 1, 9), (8, 12, 15, 3, 2, 1, 9), (16, 8, 9, 1, 1, 0, 4)])
def test_conv_forward_vs_torch_fp64(C, F, H, k, s, p, act):
    rng = np.random.default_rng(15)
    x = rng.uniform(0, 1, (2, C, H, H)).astype(np.float32)
    W = rng.normal(0, 0.05, (F, C * k * k)).astype(np.float32)
    b = rng.normal(0, 0.1, F).astype(np.float32)
    got = R.conv_forward(x, W, b, k, s, p, act)
    ref = Fn.conv2d(torch.from_numpy(x).double(), torch.from_numpy(W.reshape(F, C, k, k)).double(),
                    torch.from_numpy(b).double(), stride=s, padding=p)
    if act == 9:
        ref = torch.where(ref < 0, 0.1 * ref, ref)
    assert R.rel_err(got, ref.numpy()) < TOL


def test_logistic_exact_mode_error():
    """The reference's degree-2 exp polynomial is ~1.7e-3 relative; the exact
    mode (IEEE reciprocal) must sit within that of the true sigmoid."""
    x = np.linspace(-20, 20, 4001).astype(np.float32)
    got = R.activate(x.copy(), 0, exact=True)
    ref = 1.0 / (1.0 + np.exp(-x.astype(np.float64)))
    assert np.max(np.abs(got - ref) / ref) < 2e-3
    fa = R.activate(x.copy(), 0, exact=False)
    assert np.max(np.abs(fa - got) / got) < 1.5 * 2 ** -12 * 2


def test_yolo_head_entries():
    rng = np.random.default_rng(16)
    x = rng.standard_normal((2, 3 * 7, 4, 5)).astype(np.float32)  # 3 anchors, 2 classes
    out = R.yolo_fwd(x, 3, 2)
    xr = x.reshape(2, 3, 7, 4, 5)
    o = out.reshape(2, 3, 7, 4, 5)
    assert np.array_equal(o[:, :, 2:4], xr[:, :, 2:4])  # w, h untouched
    sig = R.activate(xr[:, :, [0, 1, 4, 5, 6]].copy(), 0)
    assert np.array_equal(o[:, :, [0, 1, 4, 5, 6]], sig)


# ------------------------------------------------------------ route -------
_ROUTE_CFG = """[net]
height=6
width=6
channels=2
[convolutional]
filters=3
size=3
pad=1
activation=leaky
[convolutional]
filters=2
size=1
activation=linear
[route]
layers=-1,-2
"""


def test_netref_reference_route_is_whole_tensor_concat():
    """TConcatLayer.forward -> TTensor.concat (nconcatlayer.pas:115,
    ntensors.pas:12045-12058): each input's whole batched tensor is copied
    at the running offset, so with inputs of n0 and n1 floats per image the
    first element of input 1 lands at flat offset B*n0, and image b of the
    route output (as [B, C, H, W]) holds floats [b*(n0+n1), (b+1)*(n0+n1))
    of that stream.  At batch 1 this is the per-image concat."""
    from oracle import netref
    from tensorium_amd import darknet

    _, layers = darknet.parse_cfg(_ROUTE_CFG)
    W = darknet.synthetic_weights(layers, seed=3)
    B = 3
    x = np.random.default_rng(40).uniform(0, 1, (B, 2, 6, 6)).astype(np.float32)
    ref = netref.forward(layers, W, x, route_mode="reference")
    img = netref.forward(layers, W, x, route_mode="image")
    src0, src1 = ref[1], ref[0]  # layers=-1,-2 from layer 2: layer 1, then layer 0
    n0, n1 = src0[0].size, src1[0].size
    flat = ref[2].ravel()
    assert ref[2].shape == (B, 5, 6, 6)
    assert flat[B * n0] == src1.ravel()[0]
    assert np.array_equal(flat[:B * n0], src0.ravel()) and np.array_equal(flat[B * n0:], src1.ravel())
    for b in range(B):  # image b's slice of the stream
        assert np.array_equal(ref[2][b].ravel(), flat[b * (n0 + n1):(b + 1) * (n0 + n1)])
    # per-image concat: image b = [src0[b] | src1[b]]; differs at B > 1
    for b in range(B):
        assert np.array_equal(img[2][b].ravel(), np.concatenate([src0[b].ravel(), src1[b].ravel()]))
    assert not np.array_equal(img[2], ref[2])
    one_r = netref.forward(layers, W, x[:1], route_mode="reference")
    one_i = netref.forward(layers, W, x[:1], route_mode="image")
    assert np.array_equal(one_r[2], one_i[2])


def test_bn_normalize_one_element_per_channel_clamps_the_variance():
    """blockNormalize with blockSize 1 (a connected layer's batch norm) goes
    through _snormvv (ntensors.pas:4338): (x - m) / sqrt(max(v, 1e-6)), where
    longer blocks clamp the standard deviation.  With v = 0 the two differ by
    a factor 1000: 1/sqrt(1e-6f) against 1/1e-6f."""
    x = np.ones((3, 4, 1, 1), np.float32)
    mean = np.zeros(4, np.float32)
    var = np.array([0.0, 4.0, np.nan, 1e-7], np.float32)
    got = R.bn_normalize(x.copy(), mean, var, 3).reshape(3, 4)
    d_eps = np.sqrt(np.float32(1e-6))
    want = np.array([np.float32(1) / d_eps, np.float32(0.5), np.float32(1) / d_eps, np.float32(1) / d_eps],
                    np.float32)
    assert np.array_equal(got, np.tile(want, (3, 1)))
    assert want[0] != np.float32(1e6)
    blk = R.bn_normalize(np.ones((1, 4, 1, 2), np.float32), mean, var, 1)
    assert blk[0, 0, 0, 0] == np.float32(1) / np.float32(1e-6)
