"""numpy interface to the CPU oracle librefcpu.so (TEST INFRASTRUCTURE ONLY).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module.  Each function forwards to the C restatement in refcpu.c, which
cites the reference routine it follows.
"""
import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "librefcpu.so")

i32, i64, f32 = C.c_int32, C.c_int64, C.c_float
P = C.c_void_p

_PROTOS = {
    "ref_set_threads": ([i32], None),
    "ref_get_threads": ([], i32),
    "ref_axpy": ([i64, f32, P, P], None),
    "ref_sgemm": ([i32, i32, i64, i64, i64, f32, P, i64, P, i64, f32, P, i64], None),
    "ref_sgemm_strided_batched": ([i32, i32, i64, i64, i64, f32, P, i64, i64, P, i64, i64, f32, P, i64, i64,
                                   i64], None),
    "ref_im2col_batched": ([i64] * 11 + [P, i64, P, i64, i64], None),
    "ref_col2im_batched": ([i64] * 11 + [P, i64, P, i64, i64], None),
    "ref_forward_bias": ([P, i64, i64, P, i64], None),
    "ref_forward_scale": ([P, i64, i64, P, i64], None),
    "ref_activate": ([P, i64, i32, i32], None),
    "ref_derive": ([P, i64, i32, P], None),
    "ref_maxpool_fwd": ([i64] * 8 + [P, P, P], None),
    "ref_maxpool_bwd": ([i64, P, P, P], None),
    "ref_upsample": ([P, i64, i64, i64, i64, i64, i32, f32, P], None),
    "ref_addvv": ([i64, P, P, P], None),
    "ref_bn_normalize": ([P, i64, i64, P, P, i64, i32], None),
    "ref_yolo_fwd": ([i64] * 5 + [P, P, i32], None),
    "ref_fuse_bn": ([i64, i64, P, P, P, P, P], None),
    "ref_conv_forward": ([i64] * 8 + [P, P, P, i32, P, P], None),
    "ref_means_vars": ([P, i64, i64, i64, P, P, i32], None),
    "ref_means_vars_delta": ([P, P, P, P, i64, i64, i64, P, P, i32], None),
    "ref_add_dots": ([P, P, P, i64, i64, i64, i32], None),
    "ref_softmax_rows": ([P, i64, i64, f32, P], None),
}

_lib = None


def build():
    subprocess.run([os.path.join(_HERE, "build.sh")], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        for n, (a, r) in _PROTOS.items():
            f = getattr(L, n)
            f.argtypes = a
            f.restype = r
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data


def _f32(a):
    a = np.ascontiguousarray(a, dtype=np.float32)
    return a


def set_threads(p):
    lib().ref_set_threads(p)


def get_threads():
    return lib().ref_get_threads()


def axpy(y, a, x):
    """Returns y + a*x with one fused multiply-add per element (saxpy_avx2)."""
    y = _f32(y).copy()
    x = _f32(x)
    lib().ref_axpy(y.size, a, _p(x), _p(y))
    return y


def sgemm(transA, transB, M, N, K, alpha, A, lda, B, ldb, beta, Cm, ldc):
    """cblas_sgemm on numpy arrays; Cm is updated in place and returned."""
    A, B = _f32(A), _f32(B)
    assert Cm.dtype == np.float32 and Cm.flags.c_contiguous
    lib().ref_sgemm(int(transA), int(transB), M, N, K, alpha, _p(A), lda, _p(B), ldb, beta, _p(Cm), ldc)
    return Cm


def sgemm_strided_batched(transA, transB, M, N, K, alpha, A, lda, strideA, B, ldb, strideB, beta, Cm, ldc,
                          strideC, batch):
    A, B = _f32(A), _f32(B)
    assert Cm.dtype == np.float32 and Cm.flags.c_contiguous
    lib().ref_sgemm_strided_batched(int(transA), int(transB), M, N, K, alpha, _p(A), lda, strideA, _p(B), ldb,
                                    strideB, beta, _p(Cm), ldc, strideC, batch)
    return Cm


def conv_out(H, k, p, s, d=1):
    return (H + 2 * p - (d * (k - 1) + 1)) // s + 1


def im2col(x, kh, kw, pH, pW, sY, sX, dY=1, dX=1):
    """x: [B, C, H, W] -> col [B, C*kh*kw, OH*OW] (sim2colStridedBatched)."""
    x = _f32(x)
    B, Cc, H, W = x.shape
    OH, OW = conv_out(H, kh, pH, sY, dY), conv_out(W, kw, pW, sX, dX)
    col = np.empty((B, Cc * kh * kw, OH * OW), np.float32)
    lib().ref_im2col_batched(Cc, H, W, kh, kw, pH, pW, sY, sX, dY, dX, _p(x), Cc * H * W, _p(col),
                             col[0].size, B)
    return col


def col2im(col, im, kh, kw, pH, pW, sY, sX, dY=1, dX=1):
    """Accumulates col [B, C*kh*kw, OH*OW] into im [B, C, H, W] in place."""
    col = _f32(col)
    assert im.dtype == np.float32 and im.flags.c_contiguous
    B, Cc, H, W = im.shape
    lib().ref_col2im_batched(Cc, H, W, kh, kw, pH, pW, sY, sX, dY, dX, _p(col), col[0].size, _p(im),
                             Cc * H * W, B)
    return im


def forward_bias(x, bias, batch):
    """x [batch, nb, ...] += bias[nb] broadcast (vsAddB)."""
    assert x.dtype == np.float32 and x.flags.c_contiguous
    bias = _f32(bias)
    nb = bias.size
    lib().ref_forward_bias(_p(x), nb, x.size // (nb * batch), _p(bias), batch)
    return x


def forward_scale(x, scale, batch):
    assert x.dtype == np.float32 and x.flags.c_contiguous
    scale = _f32(scale)
    nb = scale.size
    lib().ref_forward_scale(_p(x), nb, x.size // (nb * batch), _p(scale), batch)
    return x


def activate(x, act, exact=True):
    assert x.dtype == np.float32 and x.flags.c_contiguous
    lib().ref_activate(_p(x), x.size, act, 1 if exact else 0)
    return x


def derive(x, act, delta):
    x = _f32(x)
    assert delta.dtype == np.float32 and delta.flags.c_contiguous
    lib().ref_derive(_p(x), x.size, act, _p(delta))
    return delta


def maxpool_fwd(x, size, strideX, strideY, pad, with_idx=True):
    x = _f32(x)
    B, Cc, H, W = x.shape
    OH = (H + pad - size) // strideY + 1
    OW = (W + pad - size) // strideX + 1
    out = np.empty((B, Cc, OH, OW), np.float32)
    idx = np.empty((B, Cc, OH, OW), np.int64) if with_idx else None
    lib().ref_maxpool_fwd(B, Cc, H, W, size, strideX, strideY, pad, _p(x), _p(out), _p(idx))
    return out, idx


def maxpool_depth_fwd(x, outC, with_idx=True):
    """maxpool_depth (TMaxPoolLayer.forwardMaxPool's first branch,
    nMaxPoolLayer.pas:372-399): out[b, g, i, j] = max over input channels
    k = g, g + outC, ... < c of x[b, k, i, j], scanned in ascending k with a
    strict '>' from -MaxSingle; the index is the input's global offset
    j + w*(i + h*(k + c*b)), -1 when nothing beats the start value."""
    x = _f32(x)
    B, Cc, H, W = x.shape
    out = np.full((B, outC, H, W), -np.finfo(np.float32).max, np.float32)
    idx = np.full((B, outC, H, W), -1, np.int64)
    base = (np.arange(B, dtype=np.int64)[:, None, None] * Cc * H * W
            + np.arange(H * W, dtype=np.int64).reshape(1, H, W))
    for g in range(outC):
        for k in range(g, Cc, outC):
            v = x[:, k]
            hit = v > out[:, g]
            out[:, g] = np.where(hit, v, out[:, g])
            idx[:, g] = np.where(hit, base + k * H * W, idx[:, g])
    return out, (idx if with_idx else None)


def maxpool_bwd(idx, dOut, dIn):
    assert dIn.dtype == np.float32 and dIn.flags.c_contiguous
    idx = np.ascontiguousarray(idx, np.int64)
    dOut = _f32(dOut)
    lib().ref_maxpool_bwd(idx.size, _p(idx), _p(dOut), _p(dIn))
    return dIn


def upsample_fwd(x, stride, scale=1.0):
    x = _f32(x)
    B, Cc, h, w = x.shape
    out = np.empty((B, Cc, h * stride, w * stride), np.float32)
    lib().ref_upsample(_p(x), w, h, Cc, B, stride, 1, scale, _p(out))
    return out


def upsample_bwd(dIn, dOut, stride, scale=1.0):
    """dIn [B,C,h,w] += scale * dOut gathered (upsample backward)."""
    assert dIn.dtype == np.float32 and dIn.flags.c_contiguous
    dOut = _f32(dOut)
    B, Cc, h, w = dIn.shape
    lib().ref_upsample(_p(dIn), w, h, Cc, B, stride, 0, scale, _p(dOut))
    return dIn


def addvv(a, b):
    a, b = _f32(a), _f32(b)
    out = np.empty_like(a)
    lib().ref_addvv(a.size, _p(a), _p(b), _p(out))
    return out


def yolo_fwd(x, n, classes, exact=True):
    x = _f32(x)
    B = x.shape[0]
    h, w = x.shape[-2], x.shape[-1]
    out = np.empty_like(x)
    lib().ref_yolo_fwd(B, n, classes, h, w, _p(x), _p(out), 1 if exact else 0)
    return out


def bn_normalize(x, mean, var, batch, exact=True):
    assert x.dtype == np.float32 and x.flags.c_contiguous
    mean, var = _f32(mean), _f32(var)
    nb = mean.size
    lib().ref_bn_normalize(_p(x), nb, x.size // (nb * batch), _p(mean), _p(var), batch, 1 if exact else 0)
    return x


def fuse_bn(W, bias, scales, mean, var):
    """Returns (W', b') folded as fuseBatchNorm does; W is [F, ...]."""
    W = _f32(W).copy()
    bias = _f32(bias).copy()
    F = W.shape[0]
    lib().ref_fuse_bn(F, W.size // F, _p(W), _p(bias), _p(_f32(scales)), _p(_f32(mean)), _p(_f32(var)))
    return W, bias


def conv_forward(x, Wt, bias, k, stride, pad, act):
    """TConvolutionalLayer.forward (BN folded): returns out [B, F, OH, OW]."""
    x = _f32(x)
    Wt = _f32(Wt)
    bias = _f32(bias)
    B, Cc, H, W = x.shape
    F = Wt.shape[0]
    OH = (H + 2 * pad - k) // stride + 1
    OW = (W + 2 * pad - k) // stride + 1
    # zero-filled: cblas_sgemm implements beta = 0 as C *= 0 (ntensors.pas:2259),
    # so NaN garbage in an uninitialised C would survive
    out = np.zeros((B, F, OH, OW), np.float32)
    ws = None
    if k != 1 or stride != 1:
        ws = np.empty(B * Cc * k * k * OH * OW, np.float32)
    lib().ref_conv_forward(B, Cc, H, W, F, k, stride, pad, _p(x), _p(Wt), _p(bias), act, _p(out), _p(ws))
    return out


def rel_err(got, ref):
    """Per-tensor error max|g - r| / max|r| (the GEMM/conv parity metric)."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    den = np.max(np.abs(ref))
    if den == 0:
        return float(np.max(np.abs(got)))
    return float(np.max(np.abs(got - ref)) / den)


def means_vars(x, nch, groups, avx2=False):
    """TTensor.MeansAndVars over x viewed as [groups][nch][block]; avx2: the
    AVX2 host's routines (srss drops lanes 4..7 of blocks whose length is a
    multiple of 8), else the Pascal loops (the parity target)."""
    x = _f32(x)
    block = x.size // (nch * groups)
    m, v = np.empty(nch, np.float32), np.empty(nch, np.float32)
    lib().ref_means_vars(_p(x), nch, block, groups, _p(m), _p(v), int(avx2))
    return m, v


def means_vars_delta(delta, x, mean, var, groups, avx2=False):
    """sMeanAndVarianceDelta: (mean_delta, variance_delta) per channel."""
    delta, x, mean, var = _f32(delta), _f32(x), _f32(mean), _f32(var)
    nch = mean.size
    block = delta.size // (nch * groups)
    md, vd = np.empty(nch, np.float32), np.empty(nch, np.float32)
    lib().ref_means_vars_delta(_p(delta), _p(x), _p(mean), _p(var), nch, block, groups, _p(md), _p(vd), int(avx2))
    return md, vd


def add_dots(dst, a, b, groups, avx2=False):
    """TTensor.addDots: dst + the per-channel dots of a and b (a new array)."""
    out = _f32(dst).copy()
    a, b = _f32(a), _f32(b)
    nch = out.size
    block = a.size // (nch * groups)
    lib().ref_add_dots(_p(out), _p(a), _p(b), nch, block, groups, int(avx2))
    return out


def softmax_rows(x, temp=1.0):
    """softmax of each row of a 2-D array."""
    x = _f32(x)
    out = np.empty_like(x)
    lib().ref_softmax_rows(_p(x), x.shape[0], x.shape[1], float(temp), _p(out))
    return out
