"""Channels-last (NHWC) convolution through the C ABI against the CPU oracle
(NCHW) on identical seeded inputs: the oracle's tensors are transposed to
channels-last on the host.  Per-tensor max|g - r| / max|r| <= 1e-5 (fp32
summation order; the first layer on the matrix cores too), exact for the
per-pixel first-layer kernel, and exact equality on integer-valued data;
pixel strides that make a tensor a channel slice of a wider buffer leave the
rest of the buffer untouched."""
import numpy as np
import pytest
import torch

from oracle import refcpu as R
from tensorium_amd import synth
from tensorium_amd.nnhip import (CONV_LEAN_CFGS, CONV_SPLIT_UNIT, CONV_TAIL_BASE, CONV_TAIL_SLOT_BASE,
                                  CONV_WSPLIT_CFGS, TNHError, acLEAKY, acLINEAR, acLOGISTIC)

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


def nhwc(x):
    return np.ascontiguousarray(x.transpose(0, 2, 3, 1))


def tap_major(Wt, F, C, k):
    return np.ascontiguousarray(Wt.reshape(F, C, k, k).transpose(0, 2, 3, 1).reshape(F, k * k * C))


CONVS = [  # batch, C, H, F, k, s, p, act, residual
    (2, 32, 52, 64, 3, 2, 1, acLEAKY, False),
    (2, 64, 26, 32, 1, 1, 0, acLEAKY, True),
    (3, 128, 13, 255, 1, 1, 0, acLINEAR, False),
    (2, 256, 13, 512, 3, 1, 1, acLEAKY, True),
    (1, 64, 30, 130, 3, 1, 1, acLOGISTIC, False),
    (2, 32, 17, 96, 3, 2, 1, acLEAKY, False),
    # C % 32 != 0 (one fixed tile, K tail): YOLOv3-tiny's 16-channel layer,
    # C = 8 with stride 2, C = 4 read channels-last, C = 48 / 80 (panels that
    # cross a tap), 1x1 with C = 20 and 100
    (2, 16, 52, 32, 3, 1, 1, acLEAKY, False),
    (2, 8, 33, 48, 3, 2, 1, acLEAKY, True),
    (1, 4, 40, 70, 3, 1, 1, acLINEAR, False),
    (2, 48, 21, 64, 3, 1, 1, acLEAKY, True),
    (2, 80, 13, 40, 3, 1, 1, acLEAKY, False),
    (2, 20, 19, 24, 1, 1, 0, acLEAKY, False),
    (1, 100, 15, 130, 1, 1, 0, acLOGISTIC, False),
]


@pytest.mark.parametrize("B,Cc,Hh,F,k,s,p,act,resid", CONVS)
def test_conv_nhwc_vs_oracle(hip, B, Cc, Hh, F, k, s, p, act, resid):
    case(f"conv nhwc B{B} C{Cc} H{Hh} F{F} k{k} s{s} p{p} act{act} res{resid}")
    x = synth.uniform(71, (B, Cc, Hh, Hh))
    Wt = synth.normal(72, (F, Cc * k * k), (2.0 / (Cc * k * k)) ** 0.5)
    b = synth.normal(73, (F,), 0.1)
    OH = (Hh + 2 * p - k) // s + 1
    if act == acLOGISTIC:
        # the oracle's logistic is the reference's approximation (within 2e-3);
        # the device computes 1 / (1 + exp(-x)): compare against the exact one
        lin = R.conv_forward(x, Wt, b, k, s, p, acLINEAR).astype(np.float64)
        ref = (1.0 / (1.0 + np.exp(-lin))).astype(np.float32)
    else:
        ref = R.conv_forward(x, Wt, b, k, s, p, act)
    res = None
    if resid:
        res = synth.normal(74, ref.shape)
        ref = R.addvv(ref, res)
    dout = torch.empty((B, OH, OH, F), dtype=torch.float32, device="cuda")
    hip.conv2dForwardNHWC(B, Cc, Hh, Hh, F, k, s, p, D(nhwc(x)), 0, D(tap_major(Wt, F, Cc, k)), D(b), act, dout, 0,
                          residual=None if res is None else D(nhwc(res)))
    got = H(dout, hip).transpose(0, 3, 1, 2)
    assert R.rel_err(got, ref) <= TOL


# The matrix-core kernel serves layers of at least 32 x 32 x (CU count)
# output pixels (262 144 on 256 CUs); smaller ones run the per-pixel kernel.
@pytest.mark.parametrize("B,Cc,Hh,F,s,act,bias,pad", [
    (2, 3, 416, 32, 1, acLEAKY, True, 0),    # YOLOv3 layer 0 at batch 2
    (2, 3, 517, 44, 1, acLEAKY, True, 4),    # two filter blocks, the second ragged (12), a 16-byte aligned slice
    (3, 1, 604, 4, 1, acLINEAR, False, 0),   # one store quad, no bias, a ragged last block of pixels
    (8, 4, 186, 64, 1, acLEAKY, True, 8),    # two whole blocks, C = 4, rows of 186 pixels (blocks cross rows)
    (6, 2, 420, 16, 2, acLINEAR, True, 0),   # half a block, stride 2
])
def test_conv_nhwc_first_layer_mfma(hip, B, Cc, Hh, F, s, act, bias, pad):
    """C <= 4 image read as NCHW, output channels-last, F % 4 == 0, no
    residual, 16-byte aligned output, at least 262 144 output pixels: the
    first layer on the matrix cores (32 filters x 32 pixels per MFMA chain),
    within 1e-5 of the oracle per tensor; a channel slice of a wider output
    leaves the other channels untouched."""
    case(f"conv nhwc first layer mfma B{B} C{Cc} H{Hh} F{F} s{s} act{act} bias{bias} pad{pad}")
    x = synth.uniform(75, (B, Cc, Hh, Hh))
    Wt = synth.normal(76, (F, Cc * 9), (2.0 / (9 * Cc)) ** 0.5)
    b = synth.normal(77, (F,), 0.1) if bias else np.zeros(F, np.float32)
    ref = R.conv_forward(x, Wt, b, 3, s, 1, act)
    OH = ref.shape[2]
    outPix = F + 2 * pad
    dout = D(np.full((B, OH, OH, outPix), 7.0, np.float32))
    hip.conv2dForwardNHWC(B, Cc, Hh, Hh, F, 3, s, 1, D(x), 0, D(tap_major(Wt, F, Cc, 3)), D(b) if bias else None,
                          act, dout, pad, outPix=outPix, nchwInput=True)
    got = H(dout, hip)
    assert R.rel_err(got[..., pad:pad + F].transpose(0, 3, 1, 2), ref) <= TOL
    assert np.all(got[..., :pad] == 7.0) and np.all(got[..., pad + F:] == 7.0)


@pytest.mark.parametrize("B,Cc,Hh,F,s,act,resid,bias,pad", [
    (2, 3, 416, 32, 1, acLEAKY, True, True, 0),    # YOLOv3 layer 0 with a residual
    (2, 3, 37, 45, 1, acLEAKY, True, True, 4),     # ragged last chunk (13 filters), residual, channel slice
    (2, 3, 21, 45, 1, acLEAKY, False, True, 3),    # unaligned channel slice: scalar stores
    (1, 1, 9, 5, 2, acLINEAR, False, False, 0),    # no bias, fewer filters than one store quad
    (3, 4, 20, 7, 1, acLEAKY, False, True, 1),     # unaligned slice, one ragged quad
    (2, 2, 15, 64, 2, acLINEAR, True, True, 0),    # two whole chunks, stride 2
])
def test_conv_nhwc_first_layer_bit_exact(hip, B, Cc, Hh, F, s, act, resid, bias, pad):
    """C <= 4 image read as NCHW, output channels-last, in the cases the
    matrix-core kernel leaves to the per-pixel kernel (a residual, F % 4 != 0,
    an output slice that is not 16-byte aligned): the reference's sequential
    FMA chain, bit-exact against the oracle; a channel slice of a wider
    output leaves the other channels untouched."""
    case(f"conv nhwc few-channel B{B} C{Cc} H{Hh} F{F} s{s} act{act} res{resid} bias{bias} pad{pad}")
    x = synth.uniform(75, (B, Cc, Hh, Hh))
    Wt = synth.normal(76, (F, Cc * 9), (2.0 / (9 * Cc)) ** 0.5)
    b = synth.normal(77, (F,), 0.1) if bias else np.zeros(F, np.float32)
    ref = R.conv_forward(x, Wt, b, 3, s, 1, act)
    OH = ref.shape[2]
    res = None
    if resid:
        res = synth.normal(78, ref.shape)
        ref = R.addvv(ref, res)
    outPix = (F + pad + 3) // 4 * 4
    dout = D(np.full((B, OH, OH, outPix), 7.0, np.float32))
    hip.conv2dForwardNHWC(B, Cc, Hh, Hh, F, 3, s, 1, D(x), 0, D(tap_major(Wt, F, Cc, 3)), D(b) if bias else None,
                          act, dout, pad, outPix=outPix, nchwInput=True,
                          residual=None if res is None else D(nhwc(res)))
    got = H(dout, hip)
    assert np.array_equal(got[..., pad:pad + F].transpose(0, 3, 1, 2), ref)
    assert np.all(got[..., :pad] == 7.0) and np.all(got[..., pad + F:] == 7.0)


@pytest.mark.parametrize("k,s", [(3, 1), (3, 2), (1, 1)])
def test_conv_nhwc_channel_slices(hip, k, s):
    """Input, residual and output as channel slices of wider buffers (the
    route/concat case): only the slice is written."""
    case(f"conv nhwc slices k{k} s{s}")
    B, Cc, Hh, F = 2, 64, 26, 96
    p = k // 2
    OH = (Hh + 2 * p - k) // s + 1
    rng = np.random.default_rng(k * 10 + s)
    x = rng.integers(-3, 4, (B, Cc, Hh, Hh)).astype(np.float32)
    Wt = rng.integers(-2, 3, (F, Cc * k * k)).astype(np.float32)
    b = rng.integers(-5, 6, F).astype(np.float32)
    res = rng.integers(-5, 6, (B, F, OH, OH)).astype(np.float32)
    ref = R.addvv(R.conv_forward(x, Wt, b, k, s, p, acLINEAR), res)
    xin = np.zeros((B, Hh, Hh, Cc + 32), np.float32)
    xin[..., 16:16 + Cc] = nhwc(x)
    rin = np.zeros((B, OH, OH, F + 8), np.float32)
    rin[..., 4:4 + F] = nhwc(res)
    outbuf = np.full((B, OH, OH, F + 64), 7.0, np.float32)
    dout = D(outbuf)
    hip.conv2dForwardNHWC(B, Cc, Hh, Hh, F, k, s, p, D(xin), 16, D(tap_major(Wt, F, Cc, k)), D(b), acLINEAR, dout, 32,
                          inPix=Cc + 32, outPix=F + 64, residual=D(rin), resOffset=4, resPix=F + 8)
    got = H(dout, hip)
    assert np.array_equal(got[..., 32:32 + F].transpose(0, 3, 1, 2), ref)
    assert np.all(got[..., :32] == 7.0) and np.all(got[..., 32 + F:] == 7.0)


@pytest.mark.parametrize("Cc,k,s,F", [(4, 3, 1, 24), (8, 3, 2, 40), (16, 3, 1, 32), (20, 3, 1, 72), (48, 3, 1, 64),
                                       (80, 3, 2, 33), (20, 1, 1, 24), (100, 1, 1, 130), (4, 1, 1, 8)])
def test_conv_nhwc_any_channels_integer(hip, Cc, k, s, F):
    """C % 4 == 0 but not a multiple of 32, on integer data (exact sums):
    the input is a channel slice whose neighbouring channels hold 1e30, so a
    chunk read past the pixel's C channels (the K tail of a 1x1, a panel
    that spans taps) would show; the output is a slice too."""
    case(f"conv nhwc any-C C{Cc} k{k} s{s} F{F}")
    B, Hh = 2, 23
    p = k // 2
    OH = (Hh + 2 * p - k) // s + 1
    rng = np.random.default_rng(Cc * 10 + k)
    x = rng.integers(-3, 4, (B, Cc, Hh, Hh)).astype(np.float32)
    Wt = rng.integers(-2, 3, (F, Cc * k * k)).astype(np.float32)
    b = rng.integers(-5, 6, F).astype(np.float32)
    ref = R.conv_forward(x, Wt, b, k, s, p, acLEAKY)
    xin = np.full((B, Hh, Hh, Cc + 12), 1e30, np.float32)
    xin[..., 4:4 + Cc] = nhwc(x)
    outbuf = np.full((B, OH, OH, F + 8), 7.0, np.float32)
    dout = D(outbuf)
    hip.conv2dForwardNHWC(B, Cc, Hh, Hh, F, k, s, p, D(xin), 4, D(tap_major(Wt, F, Cc, k)), D(b), acLEAKY, dout, 4,
                          inPix=Cc + 12, outPix=F + 8)
    got = H(dout, hip)
    assert np.array_equal(got[..., 4:4 + F].transpose(0, 3, 1, 2), ref)
    assert np.all(got[..., :4] == 7.0) and np.all(got[..., 4 + F:] == 7.0)


@pytest.mark.parametrize("cfg", CONV_LEAN_CFGS)
@pytest.mark.parametrize("hi", [0, 4, CONV_TAIL_BASE + 3, CONV_TAIL_SLOT_BASE + 2])
def test_conv_nhwc_forced_configs(hip, cfg, hi):
    """Every lean tile, plain, split-K (every tile cut), and tail splits per
    CU and per workgroup slot, on integer data (exact sums)."""
    B, Cc, Hh, F, k = 4, 64, 104, 96, 3
    case(f"conv nhwc cfg{cfg} hi{hi}")
    rng = np.random.default_rng(cfg * 100 + hi)
    x = rng.integers(-3, 4, (B, Cc, Hh, Hh)).astype(np.float32)
    Wt = rng.integers(-2, 3, (F, Cc * k * k)).astype(np.float32)
    b = rng.integers(-5, 6, F).astype(np.float32)
    ref = R.conv_forward(x, Wt, b, k, 1, 1, acLEAKY)
    dout = torch.empty((B, Hh, Hh, F), dtype=torch.float32, device="cuda")
    hip.setConvAutotune(True, cfg + CONV_SPLIT_UNIT * hi)
    try:
        hip.conv2dForwardNHWC(B, Cc, Hh, Hh, F, k, 1, 1, D(nhwc(x)), 0, D(tap_major(Wt, F, Cc, k)), D(b), acLEAKY,
                              dout, 0)
    finally:
        hip.setConvAutotune(True, -1)
    assert np.array_equal(H(dout, hip).transpose(0, 3, 1, 2), ref)


@pytest.mark.parametrize("cfg", [11, 12, 13, 16, 18])
@pytest.mark.parametrize("tail", [CONV_TAIL_BASE + 3, CONV_TAIL_SLOT_BASE + 2])
def test_conv_nhwc_tail_split_residual(hip, cfg, tail):
    """Tail splits with a fused residual read from a channel slice (the
    reduction launch loads the residual with the pieces) on integer data:
    exact, and the rest of the output buffer untouched."""
    B, Cc, Hh, F, k = 4, 64, 52, 96, 3
    case(f"conv nhwc tail-split residual cfg{cfg} hi{tail}")
    rng = np.random.default_rng(cfg * 13 + tail)
    x = rng.integers(-3, 4, (B, Cc, Hh, Hh)).astype(np.float32)
    Wt = rng.integers(-2, 3, (F, Cc * k * k)).astype(np.float32)
    b = rng.integers(-5, 6, F).astype(np.float32)
    res = rng.integers(-5, 6, (B, F, Hh, Hh)).astype(np.float32)
    ref = R.addvv(R.conv_forward(x, Wt, b, k, 1, 1, acLEAKY), res).reshape(B, F, Hh, Hh)
    rin = np.zeros((B, Hh, Hh, F + 8), np.float32)
    rin[..., 8:] = nhwc(res)
    dout = D(np.full((B, Hh, Hh, F + 4), 7.0, np.float32))
    hip.setConvAutotune(True, cfg + CONV_SPLIT_UNIT * tail)
    try:
        hip.conv2dForwardNHWC(B, Cc, Hh, Hh, F, k, 1, 1, D(nhwc(x)), 0, D(tap_major(Wt, F, Cc, k)), D(b), acLEAKY,
                              dout, 4, outPix=F + 4, residual=D(rin), resOffset=8, resPix=F + 8)
    finally:
        hip.setConvAutotune(True, -1)
    got = H(dout, hip)
    assert np.array_equal(got[..., 4:].transpose(0, 3, 1, 2), ref)
    assert np.all(got[..., :4] == 7.0)


# (B, C, H, F, k, stride, pad, residual): ragged pixel and filter counts (not
# multiples of the 32/64 tile), stride 2, 1x1 with one group per wave (K = 32
# over up to 16 waves: some waves get no group), and YOLOv3's 13x13 batch-1
# shape
WSPLIT_SHAPES = [
    (1, 64, 13, 96, 3, 1, 1, True),
    (2, 32, 10, 40, 3, 2, 1, False),
    (1, 32, 9, 70, 1, 1, 0, True),
    (3, 96, 7, 33, 1, 1, 0, False),
    (1, 512, 13, 1024, 3, 1, 1, False),
]


@pytest.mark.parametrize("cfg", CONV_WSPLIT_CFGS)
@pytest.mark.parametrize("shape", WSPLIT_SHAPES)
def test_conv_nhwc_wsplit_integer(hip, cfg, shape):
    """Every wave-split tile (K of a tile split over the waves of its
    workgroup, partial tiles summed in LDS) on integer data: every partial
    sum is exact, so the result equals the oracle bit for bit; channel-slice
    strides for x, out and the residual, the rest of the output untouched."""
    B, Cc, Hh, F, k, s, p, with_res = shape
    case(f"conv nhwc wsplit cfg{cfg} {shape}")
    OH = (Hh + 2 * p - k) // s + 1
    rng = np.random.default_rng(cfg * 1000 + Cc + F)
    x = rng.integers(-3, 4, (B, Cc, Hh, Hh)).astype(np.float32)
    Wt = rng.integers(-2, 3, (F, Cc * k * k)).astype(np.float32)
    b = rng.integers(-5, 6, F).astype(np.float32)
    ref = R.conv_forward(x, Wt, b, k, s, p, acLEAKY)
    xin = np.zeros((B, Hh, Hh, Cc + 32), np.float32)
    xin[..., 32:] = nhwc(x)
    res = rin = None
    if with_res:
        res = rng.integers(-5, 6, (B, F, OH, OH)).astype(np.float32)
        ref = R.addvv(ref, res)
        rin = np.zeros((B, OH, OH, F + 4), np.float32)
        rin[..., 4:] = nhwc(res)
    dout = D(np.full((B, OH, OH, F + 8), 7.0, np.float32))
    hip.setConvAutotune(True, cfg)
    try:
        hip.conv2dForwardNHWC(B, Cc, Hh, Hh, F, k, s, p, D(xin), 32, D(tap_major(Wt, F, Cc, k)), D(b), acLEAKY,
                              dout, 8, inPix=Cc + 32, outPix=F + 8,
                              residual=None if rin is None else D(rin), resOffset=4, resPix=F + 4)
    finally:
        hip.setConvAutotune(True, -1)
    got = H(dout, hip)
    assert np.array_equal(got[..., 8:].transpose(0, 3, 1, 2), ref)
    assert np.all(got[..., :8] == 7.0)


@pytest.mark.parametrize("cfg", CONV_WSPLIT_CFGS)
@pytest.mark.parametrize("act", [acLEAKY, acLINEAR, acLOGISTIC])
def test_conv_nhwc_wsplit_vs_oracle(hip, cfg, act):
    """Wave-split tiles on YOLOv3's batch-1 26x26 3x3 layer shape (C 256 ->
    512) with random data: per tensor within 1e-5 of the oracle.  The fused
    logistic is TNNCuda's 1/(1 + exp(-x)) (cuda_sgemm.cu:305-309), so that
    case is held against the float64 sigmoid of the oracle's linear output
    (the oracle's logistic is the CPU path's polynomial)."""
    B, Cc, Hh, F, k = 1, 256, 26, 512, 3
    case(f"conv nhwc wsplit cfg{cfg} act{act} vs oracle")
    x = synth.uniform(90 + cfg, (B, Cc, Hh, Hh))
    Wt = synth.normal(91, (F, Cc * k * k), (2.0 / (Cc * k * k)) ** 0.5)
    b = synth.normal(92, (F,), 0.1)
    if act == acLOGISTIC:
        lin = R.conv_forward(x, Wt, b, k, 1, 1, acLINEAR).astype(np.float64)
        ref = 1.0 / (1.0 + np.exp(-lin))
    else:
        ref = R.conv_forward(x, Wt, b, k, 1, 1, act)
    dout = torch.empty((B, Hh, Hh, F), dtype=torch.float32, device="cuda")
    hip.setConvAutotune(True, cfg)
    try:
        hip.conv2dForwardNHWC(B, Cc, Hh, Hh, F, k, 1, 1, D(nhwc(x)), 0, D(tap_major(Wt, F, Cc, k)), D(b), act, dout, 0)
    finally:
        hip.setConvAutotune(True, -1)
    assert R.rel_err(H(dout, hip).transpose(0, 3, 1, 2), ref) <= TOL


# forced tilings that reach every channels-last epilogue: a lean tile, a lean
# tile with a tail split (the reduction kernel's epilogue), a wave-split tile
EPI_TILINGS = [11, 12 + CONV_SPLIT_UNIT * (CONV_TAIL_BASE + 3), 20, 22]


@pytest.mark.parametrize("forced", EPI_TILINGS)
@pytest.mark.parametrize("k", [1, 3])
def test_conv_nhwc_upsample_variant(hip, forced, k):
    """tnh_conv2d_fwd_nhwc_upsample equals conv2dForwardNHWC followed by
    upSampleNHWC bit for bit, into a channel slice of a wider (route)
    buffer whose other channels stay untouched; and the conv itself is
    within 1e-5 of the oracle."""
    B, Cc, Hh, F, s, scale = 2, 64, 13, 96, 2, 1.0
    case(f"conv nhwc upsample variant k{k} forced {forced}")
    p = k // 2
    x = synth.uniform(61, (B, Cc, Hh, Hh))
    Wt = synth.normal(62, (F, Cc * k * k), (2.0 / (Cc * k * k)) ** 0.5)
    b = synth.normal(63, (F,), 0.1)
    ref = R.upsample_fwd(R.conv_forward(x, Wt, b, k, 1, p, acLEAKY), s, scale)
    dx, dw, db = D(nhwc(x)), D(tap_major(Wt, F, Cc, k)), D(b)
    pix = F + 40
    fused = D(np.full((B, Hh * s, Hh * s, pix), 7.0, np.float32))
    plain = torch.empty((B, Hh, Hh, F), dtype=torch.float32, device="cuda")
    twostep = D(np.full((B, Hh * s, Hh * s, pix), 7.0, np.float32))
    hip.setConvAutotune(True, forced)
    try:
        hip.conv2dForwardNHWCUpsample(B, Cc, Hh, Hh, F, k, 1, p, dx, 0, dw, db, acLEAKY, s, scale, fused, 24,
                                      outPix=pix)
        hip.conv2dForwardNHWC(B, Cc, Hh, Hh, F, k, 1, p, dx, 0, dw, db, acLEAKY, plain, 0)
    finally:
        hip.setConvAutotune(True, -1)
    hip.upSampleNHWC(B, F, Hh, Hh, s, scale, plain, 0, F, twostep, 24, pix)
    got, want = H(fused, hip), H(twostep, hip)
    assert np.array_equal(got, want)
    assert np.all(got[..., :24] == 7.0) and np.all(got[..., 24 + F:] == 7.0)
    assert R.rel_err(got[..., 24:24 + F].transpose(0, 3, 1, 2), ref) <= TOL


# (H, k, head offset in floats): 13x13 (169 pixels, single head stores),
# 26x26 (16-byte head stores), 26x26 with a head offset that is not 16-byte
# aligned (single stores again), a 3x3 head
YOLO_VARIANTS = [(13, 1, 0), (26, 1, 0), (26, 1, 1), (26, 3, 0)]


@pytest.mark.parametrize("forced", EPI_TILINGS)
@pytest.mark.parametrize("Hh,k,yoff", YOLO_VARIANTS)
def test_conv_nhwc_yolo_variant(hip, forced, Hh, k, yoff):
    """tnh_conv2d_fwd_nhwc_yolo writes the same channels-last output as
    conv2dForwardNHWC and the same NCHW head as yoloForwardNHWC on it, bit
    for bit (3 anchors x (5 + 80 classes) = 255 filters), and nothing
    outside the head."""
    B, Cc, n, classes = 2, 128, 3, 80
    F = n * (5 + classes)
    p = k // 2
    case(f"conv nhwc yolo variant forced {forced} H{Hh} k{k} head offset {yoff}")
    x = synth.uniform(64, (B, Cc, Hh, Hh))
    Wt = synth.normal(65, (F, Cc * k * k), (2.0 / (Cc * k * k)) ** 0.5)
    b = synth.normal(66, (F,), 0.1)
    dx, dw, db = D(nhwc(x)), D(tap_major(Wt, F, Cc, k)), D(b)
    out_f = torch.empty((B, Hh, Hh, F), dtype=torch.float32, device="cuda")
    head_buf = D(np.full(yoff + B * F * Hh * Hh + 8, 7.0, np.float32))
    out_p = torch.empty_like(out_f)
    head_p = torch.empty((B, F, Hh, Hh), dtype=torch.float32, device="cuda")
    hip.setConvAutotune(True, forced)
    try:
        hip.conv2dForwardNHWCYolo(B, Cc, Hh, Hh, F, k, 1, p, dx, 0, dw, db, acLINEAR, out_f, 0, n, classes, head_buf,
                                  yoloOffset=yoff)
        hip.conv2dForwardNHWC(B, Cc, Hh, Hh, F, k, 1, p, dx, 0, dw, db, acLINEAR, out_p, 0)
    finally:
        hip.setConvAutotune(True, -1)
    hip.yoloForwardNHWC(B, n, classes, Hh, Hh, out_p, 0, F, head_p)
    assert np.array_equal(H(out_f, hip), H(out_p, hip))
    got = H(head_buf, hip)
    assert np.array_equal(got[yoff:yoff + B * F * Hh * Hh].reshape(B, F, Hh, Hh), H(head_p, hip))
    assert np.all(got[:yoff] == 7.0) and np.all(got[yoff + B * F * Hh * Hh:] == 7.0)
    ref = R.conv_forward(x, Wt, b, k, 1, p, acLINEAR)
    assert R.rel_err(H(out_f, hip).transpose(0, 3, 1, 2), ref) <= TOL


def test_conv_nhwc_variants_reject(hip):
    """The epilogue variants refuse a filter count that is not anchors x (5 +
    classes) and an upsample stride below 1."""
    x = torch.zeros(1, 4, 4, 32, device="cuda")
    w = torch.zeros(40, 32, device="cuda")
    out = torch.zeros(1, 4, 4, 40, device="cuda")
    head = torch.zeros(1, 40, 4, 4, device="cuda")
    with pytest.raises(TNHError):
        hip.conv2dForwardNHWCYolo(1, 32, 4, 4, 40, 1, 1, 0, x, 0, w, None, acLINEAR, out, 0, 3, 80, head)
    with pytest.raises(TNHError):
        hip.conv2dForwardNHWCUpsample(1, 32, 4, 4, 40, 1, 1, 0, x, 0, w, None, acLINEAR, 0, 1.0, out, 0)


def test_conv_nhwc_rejects_unsupported(hip):
    x = torch.zeros(1, 8, 8, 48, device="cuda")
    w = torch.zeros(32, 9 * 48, device="cuda")
    out = torch.zeros(1, 8, 8, 32, device="cuda")
    with pytest.raises(TNHError):  # C % 4 != 0
        hip.conv2dForwardNHWC(1, 6, 8, 8, 32, 3, 1, 1, x, 0, w, None, acLEAKY, out, 0, inPix=48)
    with pytest.raises(TNHError):  # 1x1 with stride 2
        hip.conv2dForwardNHWC(1, 32, 8, 8, 32, 1, 2, 0, x, 0, w, None, acLEAKY, out, 0, inPix=48)


@pytest.mark.parametrize("B,Cc,Hh,Ww,s,scale,inPad,outPad,outOff", [
    (2, 256, 13, 13, 2, 1.0, 0, 0, 0),      # YOLOv3 upsample (16-byte path)
    (3, 128, 7, 9, 2, 0.5, 4, 384, 128),    # into a channel slice of a route buffer
    (1, 6, 5, 4, 3, 2.0, 1, 3, 1),          # odd channels and strides: scalar path, stride 3
])
def test_upsample_nhwc_vs_oracle(hip, B, Cc, Hh, Ww, s, scale, inPad, outPad, outOff):
    """Channels-last nearest upsample (a channel slice in and out): bit-exact
    against the oracle's NCHW upsample; the rest of the output buffer is
    untouched."""
    case(f"upsample nhwc B{B} C{Cc} {Hh}x{Ww} s{s} scale{scale} pads {inPad},{outPad} off{outOff}")
    x = synth.normal(81, (B, Cc, Hh, Ww))
    ref = R.upsample_fwd(x, s, scale)
    inPix, outPix = Cc + inPad, Cc + outPad
    xin = np.zeros((B, Hh, Ww, inPix), np.float32)
    xin[..., :Cc] = nhwc(x)
    dout = D(np.full((B, Hh * s, Ww * s, outPix), 7.0, np.float32))
    hip.upSampleNHWC(B, Cc, Hh, Ww, s, scale, D(xin), 0, inPix, dout, outOff, outPix)
    got = H(dout, hip)
    assert np.array_equal(got[..., outOff:outOff + Cc].transpose(0, 3, 1, 2), ref)
    rest = np.concatenate([got[..., :outOff], got[..., outOff + Cc:]], axis=-1)
    assert np.all(rest == 7.0)


@pytest.mark.parametrize("B,Cc,Hh,Ww,size,s,pad,inPad,outPad", [
    (2, 16, 416, 416, 2, 2, 1, 0, 0),       # YOLOv3-tiny's first maxpool (16-byte path)
    (1, 512, 13, 13, 2, 1, 1, 0, 0),        # the stride-1 maxpool: the last row and column see one tap inside
    (2, 256, 26, 26, 2, 2, 1, 128, 0),      # input a channel slice of a route buffer
    (3, 6, 11, 9, 3, 2, 2, 1, 3),           # odd channels (scalar path), window offset -1, slices both sides
    (1, 8, 7, 7, 5, 3, 4, 0, 8),            # windows wider than the stride, output slice
])
def test_maxpool_nhwc_vs_oracle(hip, B, Cc, Hh, Ww, size, s, pad, inPad, outPad):
    """Channels-last max pool: the oracle's values (tnh_maxpool_fwd's CPU
    semantics) bit for bit, on data with ties and signed zeros (the first of
    equal values is kept: +0 / -0 order shows), channel slices in and out
    leaving the rest of the output buffer untouched."""
    case(f"maxpool nhwc B{B} C{Cc} {Hh}x{Ww} size{size} s{s} pad{pad}")
    rng = np.random.default_rng(Cc + size)
    x = rng.integers(-2, 3, (B, Cc, Hh, Ww)).astype(np.float32)
    x[x == 0] = np.where(rng.random(int((x == 0).sum())) < 0.5, -0.0, 0.0).astype(np.float32)
    ref, _ = R.maxpool_fwd(x, size, s, s, pad, with_idx=False)
    OH, OW = ref.shape[2:]
    xin = np.full((B, Hh, Ww, Cc + inPad), 9.0, np.float32)
    xin[..., inPad:] = nhwc(x)
    outbuf = np.full((B, OH, OW, Cc + outPad), 7.0, np.float32)
    dout = D(outbuf)
    hip.forwardMaxPoolNHWC(B, Cc, Hh, Ww, OH, OW, s, s, pad, size, D(xin), inPad, Cc + inPad, dout, outPad,
                           Cc + outPad)
    got = H(dout, hip)
    g = got[..., outPad:].transpose(0, 3, 1, 2)
    assert np.array_equal(g.view(np.uint32), np.ascontiguousarray(ref).view(np.uint32))
    assert np.all(got[..., :outPad] == 7.0)


def test_maxpool_nhwc_rejects(hip):
    x = torch.zeros(1, 4, 4, 8, device="cuda")
    out = torch.zeros(1, 2, 2, 8, device="cuda")
    with pytest.raises(TNHError):  # output dims that do not match
        hip.forwardMaxPoolNHWC(1, 8, 4, 4, 3, 3, 2, 2, 0, 2, x, 0, 8, out, 0, 8)
    with pytest.raises(TNHError):  # pixel stride below the channel count
        hip.forwardMaxPoolNHWC(1, 8, 4, 4, 2, 2, 2, 2, 0, 2, x, 0, 4, out, 0, 8)
