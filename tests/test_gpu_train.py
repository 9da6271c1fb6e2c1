"""GPU parity of the training-direction kernels and of the config-3 training
step (conv-BN-leaky x3, maxpool, avgpool, connected, softmax cross-entropy,
SGD) against the CPU oracle (oracle/trainref.py) on identical inputs.

Bit-exact: element-wise kernels given identical inputs (normalize_delta,
clamp, avgpool backward, cross-entropy delta, the fused SGD / parameter
updates, which are the reference's fused multiply-adds) and integer-valued
weight-gradient GEMMs.  Per-tensor max|g - r| / max|r| for reductions and
GEMMs (accumulation order differs from the reference's AVX sums)."""
import numpy as np
import pytest
import torch

from oracle import refcpu as R
from oracle import trainref as T
from tensorium_amd import synth, trainnet
from tensorium_amd.nnhip import WEIGHTS_TAP_MAJOR, TNHError, acLEAKY, acLINEAR, acLOGISTIC

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


@pytest.mark.parametrize("shape", [(128, 32, 32, 32), (4, 3, 5, 7), (2, 130, 1, 1)])
def test_means_vars(hip, shape):
    case(f"means_vars {shape}")
    x = synth.normal(301, shape, 2.0) + np.float32(1)
    B, Cc = shape[:2]
    m_ref, v_ref = T.means_vars(x, Cc, B)
    dm, dv = (torch.empty(Cc, dtype=torch.float32, device="cuda") for _ in range(2))
    dx = D(x)
    hip.meansAndVars(x.size, Cc, B, dx, 0, dm, dv)
    e = R.rel_err(H(dm, hip), m_ref)
    if e > TOL:  # say whether the input or the reduction went wrong
        same = np.array_equal(H(dx, hip), x)
        hip.meansAndVars(x.size, Cc, B, dx, 0, dm, dv)
        print(f"[diag] means rel_err {e}; device input intact: {same}; "
              f"second run rel_err {R.rel_err(H(dm, hip), m_ref)}", flush=True)
    assert e <= TOL
    assert R.rel_err(H(dv, hip), v_ref) <= TOL


@pytest.mark.parametrize("shape,off", [((128, 64, 16, 16), 0), ((1, 8, 300, 300), 0), ((3, 5, 33, 17), 1),
                                       ((64, 10, 1, 1), 0), ((3, 70000, 1, 1), 0)])
def test_channel_reductions_large_and_ragged(hip, shape, off):
    """The multi-workgroup channel reductions (statistics, their deltas,
    addDots) on many workgroups per channel, rows longer than one unit
    (90 000 floats), an unaligned offset (scalar loads), one element per
    channel and more channels than a grid's y dimension holds (70 000, as a
    wide connected layer's statistics): within the per-tensor bound of the oracle's float64 sums, and
    identical bits on a second call (fixed summation order)."""
    case(f"channel reductions {shape} offset {off}")
    B, Cc = shape[:2]
    x = synth.normal(310, shape, 1.5) + np.float32(0.5)
    d = synth.normal(311, shape)
    m_ref, v_ref = T.means_vars(x, Cc, B)
    md_ref, vd_ref = T.means_vars_delta(d, x, m_ref, v_ref, B)
    acc0 = synth.normal(312, (Cc,))
    dots_ref = T.add_dots(acc0, x, d, B)
    # backwardBias: dst[i] += the sum of channel i's deltas (= addDots with ones)
    bias_ref = T.add_dots(acc0, np.ones_like(d), d, B)
    dx = D(np.concatenate([np.zeros(off, np.float32), x.ravel()]))
    dd = D(np.concatenate([np.zeros(off, np.float32), d.ravel()]))
    res = []
    for _ in range(2):
        dm, dv, dmd, dvd = (torch.empty(Cc, dtype=torch.float32, device="cuda") for _ in range(4))
        dacc, dbias = D(acc0), D(acc0)
        hip.meansAndVars(x.size, Cc, B, dx, off, dm, dv)
        hip.meansAndVarsDelta(d.size, Cc, B, dd, dx, off, D(m_ref), D(v_ref), dmd, dvd)
        hip.addDots(x.size, Cc, B, dx, dd, off, dacc)
        hip.backwardBias(Cc, dbias, d.size, dd, off, 1, B)
        res.append([H(t, hip) for t in (dm, dv, dmd, dvd, dacc, dbias)])
    for a, b in zip(*res):
        assert np.array_equal(a, b)
    m, v, md, vd, dots, bias = res[0]
    for got, ref in ((m, m_ref), (v, v_ref), (md, md_ref), (vd, vd_ref), (dots, dots_ref), (bias, bias_ref)):
        assert R.rel_err(got, ref) <= TOL


def test_bn_statistics_equals_the_reference_sequence(hip):
    """tnh_bn_statistics == meansAndVars, then rolling.Multiply(1 - m) and
    rolling.axpy(m, stat) (nbaselayer.pas:351-355), bit for bit."""
    case("bn statistics + rolling update")
    B, Cc = 32, 48
    x = synth.normal(313, (B, Cc, 12, 12), 2.0)
    rm0, rv0 = synth.normal(314, (Cc,)), synth.uniform(315, (Cc,), 0.5, 2.0)
    mom = float(np.float32(0.1))
    keep = float(np.float32(1) - np.float32(0.1))
    dx = D(x)
    dm, dv, dm2, dv2 = (torch.empty(Cc, dtype=torch.float32, device="cuda") for _ in range(4))
    rm, rv, rm2, rv2 = D(rm0), D(rv0), D(rm0), D(rv0)
    hip.bnStatistics(x.size, Cc, B, dx, 0, dm, dv, rm, rv, mom)
    hip.meansAndVars(x.size, Cc, B, dx, 0, dm2, dv2)
    hip.scale(Cc, keep, rm2, 1)
    hip.axpy(Cc, mom, dm2, 0, 1, rm2, 0, 1)
    hip.scale(Cc, keep, rv2, 1)
    hip.axpy(Cc, mom, dv2, 0, 1, rv2, 0, 1)
    for a, b in ((dm, dm2), (dv, dv2), (rm, rm2), (rv, rv2)):
        assert np.array_equal(H(a, hip), H(b, hip))


def test_bn_backward_kernels(hip):
    case("means_vars_delta / normalize_delta / add_dots")
    B, Cc, Hh = 16, 24, 9
    x = synth.normal(302, (B, Cc, Hh, Hh), 1.5) + np.float32(0.3)
    d = synth.normal(303, (B, Cc, Hh, Hh))
    mean, var = T.means_vars(x, Cc, B)
    md_ref, vd_ref = T.means_vars_delta(d, x, mean, var, B)
    dx, dd = D(x), D(d)
    dmean, dvar = D(mean), D(var)
    dmd, dvd = (torch.empty(Cc, dtype=torch.float32, device="cuda") for _ in range(2))
    hip.meansAndVarsDelta(d.size, Cc, B, dd, dx, 0, dmean, dvar, dmd, dvd)
    assert R.rel_err(H(dmd, hip), md_ref) <= TOL
    assert R.rel_err(H(dvd, hip), vd_ref) <= TOL
    # normalize_delta is element-wise: bit-exact given the oracle's md / vd
    ref = T.normalize_delta(d, x, mean, var, md_ref, vd_ref, B)
    hip.normalizeDelta(d.size, Cc, B, dd, dx, 0, dmean, dvar, D(md_ref), D(vd_ref))
    assert np.array_equal(H(dd, hip), ref)
    acc0 = synth.normal(304, (Cc,))
    ref = T.add_dots(acc0, x, d, B)
    dacc = D(acc0)
    hip.addDots(x.size, Cc, B, dx, D(d), 0, dacc)
    assert R.rel_err(H(dacc, hip), ref) <= TOL


def test_softmax_cross_entropy_clamp(hip):
    case("softmax / cross-entropy / clamp")
    B = 300
    logits = synth.normal(305, (B, 10), 4.0)
    lab = (synth.splitmix64(306, B) % np.uint64(10)).astype(np.int64)
    truth = np.zeros((B, 10), np.float32)
    truth[np.arange(B), lab] = 1
    p_ref = T.softmax_batch(logits)
    dp = torch.empty((B, 10), dtype=torch.float32, device="cuda")
    hip.softmaxBatch(10, D(logits), 0, B, 10, 1, 10, 1, 1.0, dp, 0)
    p = H(dp, hip)
    assert np.max(np.abs(p - p_ref) / np.maximum(p_ref, 1e-30)) <= 1e-6
    delta_ref, err_ref = T.cross_entropy(p, truth)
    dd, de = torch.empty_like(dp), torch.empty_like(dp)
    hip.crossEntropySoftmax(B * 10, dp, D(truth), dd, de)
    assert np.array_equal(H(dd, hip), delta_ref)
    assert R.rel_err(H(de, hip), err_ref) <= 1e-6
    big = synth.normal(307, (1000,), 3.0)
    db = D(big)
    hip.clamp(1000, 1.0, db, db)
    assert np.array_equal(H(db, hip), T.clamp(big, -1, 1))


def test_avgpool(hip):
    case("avgpool fwd/bwd")
    x = synth.normal(308, (7, 20, 8, 8))
    ref = T.avgpool_fwd(x)
    dy = torch.empty((7, 20), dtype=torch.float32, device="cuda")
    hip.avgPoolForward(7, 20, 8, 8, D(x), dy)
    assert R.rel_err(H(dy, hip), ref) <= TOL
    g = synth.normal(309, (7, 20))
    base = synth.normal(310, x.shape)
    ref = T.avgpool_bwd(base.copy(), g)
    db = D(base)
    hip.avgPoolBackward(7, 20, 8, 8, D(g), db)
    assert np.array_equal(H(db, hip), ref)


def test_sgd_param_update_bit_exact(hip):
    case("sgd / param update")
    w = synth.normal(311, (4097,))
    wu = synth.normal(312, (4097,), 0.1)
    w_ref, wu_ref = T.sgd_update(w, wu, 1e-3, 128, 0.9, 1e-4)
    dw, dwu = D(w), D(wu)
    hip.sgdUpdate(4097, 1e-3, 128, 0.9, 1e-4, dw, dwu)
    assert np.array_equal(H(dw, hip), w_ref) and np.array_equal(H(dwu, hip), wu_ref)
    p_ref, pu_ref = T.param_update(w, wu, 1e-3, 128, 0.9)
    dw, dwu = D(w), D(wu)
    hip.paramUpdate(4097, 1e-3, 128, 0.9, dw, dwu)
    assert np.array_equal(H(dw, hip), p_ref) and np.array_equal(H(dwu, hip), pu_ref)


@pytest.mark.parametrize("B,F,K,L", [(128, 32, 27, 1024), (128, 64, 288, 256), (3, 40, 70, 48), (2, 5, 9, 30)])
def test_wgrad_gemm(hip, B, F, K, L):
    """sum_b delta_b * col_b^T accumulated into dW (beta 1), vs the
    reference's per-image NT SGEMM loop; L = 30 takes the per-image path."""
    case(f"wgrad B{B} F{F} K{K} L{L}")
    A = synth.normal(313, (B, F, L))
    Bm = synth.normal(314, (B, K, L))
    C0 = synth.normal(315, (F, K))
    ref = C0.copy()
    for b in range(B):
        R.sgemm(0, 1, F, K, L, 1.0, A[b], L, Bm[b], L, 1.0, ref, K)
    dC = D(C0)
    hip.gemmNTBatchReduce(F, K, L, 1.0, D(A), 0, L, F * L, D(Bm), 0, L, K * L, 1.0, dC, 0, K, B)
    assert R.rel_err(H(dC, hip), ref) <= TOL
    # integer-valued data: every partial sum is exact, so any order is bit-exact
    Ai = np.floor(synth.uniform(316, (B, F, L), -4, 4)).astype(np.float32)
    Bi = np.floor(synth.uniform(317, (B, K, L), -4, 4)).astype(np.float32)
    ref = np.zeros((F, K), np.float32)
    for b in range(B):
        R.sgemm(0, 1, F, K, L, 1.0, Ai[b], L, Bi[b], L, 1.0, ref, K)
    dC = torch.zeros((F, K), dtype=torch.float32, device="cuda")
    hip.gemmNTBatchReduce(F, K, L, 1.0, D(Ai), 0, L, F * L, D(Bi), 0, L, K * L, 1.0, dC, 0, K, B)
    assert np.array_equal(H(dC, hip), ref)


def _batch(seed, B):
    x = synth.uniform(seed, (B, 3, 32, 32))
    lab = (synth.splitmix64(seed + 1, B) % np.uint64(10)).astype(np.int64)
    truth = np.zeros((B, 10), np.float32)
    truth[np.arange(B), lab] = 1
    return x, truth


@pytest.mark.parametrize("B", [128, 8, 3, 1])
def test_cifar_train_step(hip, B):
    """One full trainEpoch iteration (forward, backward, update) on the device
    vs the oracle from identical parameters and inputs: loss, BN statistics,
    every gradient accumulator, the conv2/conv3 input deltas and the updated
    parameters, per tensor."""
    case(f"cifar train step B{B}")
    params = trainnet.init_params()
    x, truth = _batch(320, B)
    ref = T.CifarStep(params)
    loss_ref = ref.forward(x, truth)
    ref.backward()
    # the activation outputs are stored so they can be compared (the default
    # forms them again in the backward: the same bits, checked separately)
    gpu = trainnet.CifarTrainer(hip, params, B, store_bn_outputs=True, defer_wgrad_sum=False)
    dx, dt = D(x), D(truth)
    gpu.forward(dx, dt)
    gpu.backward()
    loss = gpu.cost()
    assert abs(float(loss) - float(loss_ref)) <= TOL * abs(float(loss_ref))
    for i in range(3):
        assert R.rel_err(gpu.host(f"mean{i}"), ref.t[f"mean{i}"]) <= TOL, f"mean{i}"
        assert R.rel_err(gpu.host(f"var{i}"), ref.t[f"var{i}"]) <= TOL, f"var{i}"
        assert R.rel_err(gpu.host(f"rm{i}"), ref.p[f"rm{i}"]) <= TOL, f"rolling mean {i}"
        assert R.rel_err(gpu.host(f"out{i}"), ref.t[f"out{i}"]) <= TOL, f"out{i}"
        assert R.rel_err(gpu.host(f"u_w{i}"), ref.p[f"u_w{i}"]) <= TOL, f"dW{i}"
        assert R.rel_err(gpu.host(f"u_s{i}"), ref.p[f"u_s{i}"]) <= TOL, f"dScale{i}"
        assert np.all(gpu.host(f"u_b{i}") == 0)
    for i in (1, 2):
        assert R.rel_err(gpu.host(f"dx{i}"), ref.t[f"dx{i}"]) <= TOL, f"input delta of conv{i + 1}"
    assert R.rel_err(gpu.host("u_fw"), ref.p["u_fw"]) <= TOL
    assert R.rel_err(gpu.host("u_fb"), ref.p["u_fb"]) <= TOL
    ref.update(B)
    gpu.update()
    for k in ("w0", "w1", "w2", "s0", "s1", "s2", "fw", "fb", "u_w1", "u_fw"):
        assert R.rel_err(gpu.host(k), ref.p[k]) <= TOL, k


def test_cifar_train_loss_falls(hip):
    """Several device steps on one batch: the loss decreases (descent)."""
    case("cifar train loss falls")
    B = 32
    x, truth = _batch(330, B)
    gpu = trainnet.CifarTrainer(hip, trainnet.init_params(), B, lr=0.1)
    dx, dt = D(x), D(truth)
    losses = []
    for _ in range(5):
        gpu.step(dx, dt)
        losses.append(float(gpu.cost()))
    assert np.all(np.isfinite(losses)) and losses[-1] < losses[0]


def test_reductions_on_two_forked_streams(hip):
    """Channel reductions forked onto two streams at once, each with many
    workgroups per channel: backwardBias on the main stream while
    meansAndVars and addDots run on a second stream.  Each stream keeps its
    own partial-sum buffer, so the results equal the same calls made one
    after another on one stream, bit for bit."""
    case("channel reductions on two forked streams")
    B, Cc, Hh = 64, 64, 32
    x = synth.normal(340, (B, Cc, Hh, Hh), 1.5) + np.float32(0.5)
    d = synth.normal(341, (B, Cc, Hh, Hh))
    acc0 = synth.normal(342, (Cc,))
    dx, dd = D(x), D(d)
    n = x.size

    def bufs():
        return [torch.empty(Cc, dtype=torch.float32, device="cuda") for _ in range(2)] + [D(acc0), D(acc0)]

    m1, v1, acc1, bb1 = bufs()
    hip.meansAndVars(n, Cc, B, dx, 0, m1, v1)
    hip.addDots(n, Cc, B, dx, dd, 0, acc1)
    hip.backwardBias(Cc, bb1, n, dd, 0, 1, B)
    one = [H(t, hip) for t in (m1, v1, acc1, bb1)]

    m2, v2, acc2, bb2 = bufs()
    torch.cuda.synchronize()
    side = torch.cuda.Stream()  # default priority
    main = hip.stream
    fork, join = hip.eventCreate(), hip.eventCreate()
    try:
        for rep in range(3):
            hip.eventRecord(fork)
            hip.setStream(side.cuda_stream)
            hip.streamWaitEvent(fork)
            hip.meansAndVars(n, Cc, B, dx, 0, m2, v2)
            hip.addDots(n, Cc, B, dx, dd, 0, acc2)
            hip.eventRecord(join)
            hip.setStream(main)
            hip.backwardBias(Cc, bb2, n, dd, 0, 1, B)
            hip.streamWaitEvent(join)
            got = [H(t, hip) for t in (m2, v2, acc2, bb2)]
            for name, a, b in zip(("means", "vars", "dots", "bias"), got, one):
                assert np.array_equal(a, b), (rep, name)
            acc2.copy_(torch.from_numpy(acc0))
            bb2.copy_(torch.from_numpy(acc0))
            torch.cuda.synchronize()
    finally:
        hip.setStream(main)
        hip.eventDestroy(fork)
        hip.eventDestroy(join)


def test_cifar_train_step_graph_replays_equal_eager(hip):
    """The config-3 step captured into a HIP graph (as bench.py times it) and
    replayed three times, with eager work and synchronizations between the
    replays, against a second trainer from the same parameters stepping
    eagerly: every parameter, momentum buffer and the loss equal after each
    step, bit for bit (the captured step launches the kernels the eager one
    does, with the same scratch splits)."""
    case("cifar train step: graph replays vs eager steps, B 32")
    B = 32
    x, truth = _batch(350, B)
    params = trainnet.init_params()
    a = trainnet.CifarTrainer(hip, params, B)
    b = trainnet.CifarTrainer(hip, params, B)
    dx, dt = D(x), D(truth)
    keys = ("w0", "w1", "w2", "s0", "s2", "fw", "fb", "u_w0", "u_w2", "u_s1", "u_fw", "rm1", "rv2")
    try:
        a.capture(dx, dt)  # runs one eager step first
        hip.useTorchStream()
        b.step(dx, dt)
        for rep in range(3):
            hip.resetStream()
            a.replay()
            hip.finish()
            hip.useTorchStream()
            b.step(dx, dt)
            hip.finish()
            for k in keys:
                assert np.array_equal(a.host(k), b.host(k)), (rep, k)
            assert float(a.cost()) == float(b.cost()), rep
            torch.cuda.synchronize()
    finally:
        a.release_graph()
        hip.useTorchStream()


@pytest.mark.parametrize("shape,off", [((128, 32, 32, 32), 0), ((3, 5, 33, 17), 1), ((64, 10, 1, 1), 0)])
def test_means_then_variances(hip, shape, off):
    """TNNCuda.means then TNNCuda.variances with those means, as
    TBaseLayer.batchNormGPU calls them in training (nbaselayer.pas:583-584):
    equal to meansAndVars bit for bit, and within the per-tensor bound of the
    oracle (CPU MeansAndVars: the unbiased S - 1 divisor)."""
    case(f"means + variances {shape} offset {off}")
    B, Cc = shape[:2]
    x = synth.normal(360, shape, 2.0) + np.float32(0.7)
    m_ref, v_ref = T.means_vars(x, Cc, B)
    dx = D(np.concatenate([np.zeros(off, np.float32), x.ravel()]))
    dm, dv, dm2, dv2 = (torch.empty(Cc, dtype=torch.float32, device="cuda") for _ in range(4))
    hip.means(x.size, Cc, B, dx, off, dm)
    hip.variances(x.size, Cc, B, dx, off, dm, dv)
    hip.meansAndVars(x.size, Cc, B, dx, off, dm2, dv2)
    m, v = H(dm, hip), H(dv, hip)
    assert np.array_equal(m, H(dm2, hip))
    assert np.array_equal(v, H(dv2, hip))
    assert R.rel_err(m, m_ref) <= TOL
    assert R.rel_err(v, v_ref) <= TOL
    # variances about means the caller supplies (not the batch's): the
    # residual sum of squares about those values, / (S - 1)
    shift = (m_ref + np.float32(0.25)).astype(np.float32)
    hip.variances(x.size, Cc, B, dx, off, D(shift), dv)
    xx = x.reshape(B, Cc, -1).astype(np.float64)
    want = ((xx - shift.astype(np.float64)[None, :, None]) ** 2).sum(axis=(0, 2)) / (x.size // Cc - 1)
    assert R.rel_err(H(dv, hip), want.astype(np.float32)) <= TOL


@pytest.mark.parametrize("shape,off,act", [((128, 32, 16, 16), 0, 9), ((3, 5, 33, 17), 1, 9), ((64, 10, 1, 1), 0, 0),
                                           ((8, 24, 9, 9), 0, 4)])
def test_bn_backward_scale_equals_three_calls(hip, shape, off, act):
    """tnh_bn_backward_scale (DeriveArray + addDots + forwardScale of
    batchNormBack in one pass) against the three separate calls: the deltas
    and the scale updates bit for bit (16-byte and scalar walks, leaky,
    logistic and linear)."""
    case(f"bn backward scale {shape} offset {off} act {act}")
    B, Cc = shape[:2]
    out = synth.normal(370, shape, 1.0)
    if act == 0:
        out = (np.float32(1) / (np.float32(1) + np.exp(-out))).astype(np.float32)
    xn = synth.normal(371, shape)
    d0 = synth.normal(372, shape)
    g = synth.uniform(373, (Cc,), 0.5, 1.5)
    acc0 = synth.normal(374, (Cc,))
    n = d0.size
    pad = np.zeros(off, np.float32)
    dout, dxn = D(np.concatenate([pad, out.ravel()])), D(np.concatenate([pad, xn.ravel()]))
    da, db = D(np.concatenate([pad, d0.ravel()])), D(np.concatenate([pad, d0.ravel()]))
    ua, ub, dg = D(acc0), D(acc0), D(g)
    ov, xv, av, bv = (t[off:] for t in (dout, dxn, da, db))
    hip.bnBackwardScale(n, Cc, B, ov, act, xv, dg, av, ua)
    hip.DeriveArray(n, ov, 0, act, bv)
    hip.addDots(n, Cc, B, xv, bv, 0, ub)
    hip.forwardScale(n, bv, 0, Cc, dg, 1, B)
    assert np.array_equal(H(da, hip), H(db, hip))
    assert np.array_equal(H(ua, hip), H(ub, hip))


def _im2col_np(x, k, pad, stride, dil):
    """im2col of a batch [B][C][H][W] -> [B][C*k*k][OH*OW] (sim2Col's order)."""
    B, C, Hh, W = x.shape
    OH = (Hh + 2 * pad - dil * (k - 1) - 1) // stride + 1
    OW = (W + 2 * pad - dil * (k - 1) - 1) // stride + 1
    xp = np.zeros((B, C, Hh + 2 * pad, W + 2 * pad), np.float32)
    xp[:, :, pad:pad + Hh, pad:pad + W] = x
    col = np.empty((B, C, k, k, OH, OW), np.float32)
    for ky in range(k):
        for kx in range(k):
            col[:, :, ky, kx] = xp[:, :, ky * dil:ky * dil + stride * (OH - 1) + 1:stride,
                                   kx * dil:kx * dil + stride * (OW - 1) + 1:stride]
    return col.reshape(B, C * k * k, OH * OW), OH, OW


@pytest.mark.parametrize("B,C,Hh,F,k,pad,stride,dil", [
    (8, 3, 32, 32, 3, 1, 1, 1),     # config-3 conv1: OW 32, one output row per panel
    (8, 32, 16, 64, 3, 1, 1, 1),    # conv2: two rows per panel
    (8, 64, 8, 128, 3, 1, 1, 1),    # conv3: four rows per panel
    (2, 16, 64, 24, 3, 1, 2, 1),    # stride 2 (OW 32)
    (1, 8, 64, 16, 3, 1, 1, 1),     # OW 64: two panels per row
    (4, 64, 16, 32, 1, 0, 1, 1),    # 1x1
    (3, 8, 20, 16, 3, 2, 1, 2),     # dilation 2, OH*OW = 400: the image-by-image path
    (2, 4, 12, 8, 5, 2, 1, 1),      # 5x5, OW 12: the image-by-image path
])
def test_conv_wgrad(hip, B, C, Hh, F, k, pad, stride, dil):
    """tnh_conv2d_wgrad (the im2col inside the GEMM's loader): within 1e-5 of
    float64 sum_b delta_b * im2col(x_b)^T with alpha 0.5 / beta 1; where it
    runs fused, bit for bit equal to tnh_im2col_batched followed by
    tnh_sgemm_nt_batch_reduce; on integer data exact."""
    case(f"conv wgrad B{B} C{C} H{Hh} F{F} k{k} pad{pad} s{stride} d{dil}")
    x = synth.normal(330, (B, C, Hh, Hh))
    col, OH, OW = _im2col_np(x, k, pad, stride, dil)
    L, K = OH * OW, C * k * k
    delta = synth.normal(331, (B, F, L))
    dW0 = synth.normal(332, (F, K))
    ref = dW0.astype(np.float64) + 0.5 * np.einsum("bfl,bkl->fk", delta.astype(np.float64), col.astype(np.float64))
    dW = D(dW0)
    hip.convWeightGradient(B, C, Hh, Hh, F, k, k, pad, pad, stride, stride, dil, dil, D(x), C * Hh * Hh, D(delta),
                           F * L, 0.5, 1.0, dW)
    got = H(dW, hip)
    assert R.rel_err(got, ref) <= TOL
    fused = L % 32 == 0 and OW % 4 == 0 and (OW % 32 == 0 or 32 % OW == 0)
    if fused:
        dcol = torch.empty((B, K, L), dtype=torch.float32, device="cuda")
        hip.im2colStridedBatched(C, Hh, Hh, k, k, pad, pad, stride, stride, dil, dil, D(x), C * Hh * Hh, 0, dcol, K * L,
                                 0, B)
        assert np.array_equal(H(dcol, hip), col)
        dW2 = D(dW0)
        hip.gemmNTBatchReduce(F, K, L, 0.5, D(delta), 0, L, F * L, dcol, 0, L, K * L, 1.0, dW2, 0, K, B)
        assert np.array_equal(H(dW2, hip), got)
    xi = np.floor(synth.uniform(333, x.shape, -4, 4)).astype(np.float32)
    di = np.floor(synth.uniform(334, delta.shape, -4, 4)).astype(np.float32)
    coli, _, _ = _im2col_np(xi, k, pad, stride, dil)
    refi = np.einsum("bfl,bkl->fk", di.astype(np.float64), coli.astype(np.float64)).astype(np.float32)
    dW = torch.zeros((F, K), dtype=torch.float32, device="cuda")
    hip.convWeightGradient(B, C, Hh, Hh, F, k, k, pad, pad, stride, stride, dil, dil, D(xi), C * Hh * Hh, D(di), F * L,
                           1.0, 0.0, dW)
    assert np.array_equal(H(dW, hip), refi)


def test_cifar_step_fused_wgrad_equals_im2col_path(hip):
    """The training step with the fused weight gradients gives the same bits
    as with the reference's im2col + NT product (every gradient and the
    updated parameters)."""
    case("cifar step fused wgrad vs im2col")
    params = trainnet.init_params()
    x, truth = _batch(321, 16)
    out = []
    for fused in (True, False):
        gpu = trainnet.CifarTrainer(hip, params, 16, fused_wgrad=fused)
        gpu.forward(D(x), D(truth))
        gpu.backward()
        gpu.update()
        out.append({k: gpu.host(k).copy() for k in ("u_w0", "u_w1", "u_w2", "w0", "w1", "w2", "s0", "u_fw")})
    for k in out[0]:
        assert np.array_equal(out[0][k], out[1][k]), k


@pytest.mark.parametrize("F,C,k", [(64, 32, 3), (128, 64, 3), (5, 7, 3), (6, 4, 1), (3, 2, 5)])
def test_pack_weights_dgrad(hip, F, C, k):
    """The training step's dual repack: the tap-major copy equals
    tnh_conv2d_pack_weights', the flipped one is w[f][c][k-1-ky][k-1-kx] at
    [c][ky][kx][f], bit for bit; a NULL tap-major copy is skipped."""
    case(f"pack_weights_dgrad F{F} C{C} k{k}")
    w = synth.normal(340, (F, C, k, k))
    tap = torch.empty(w.size, dtype=torch.float32, device="cuda")
    flip = torch.empty(w.size, dtype=torch.float32, device="cuda")
    hip.packConvWeightsDgrad(F, C, k, D(w), tap, flip)
    assert np.array_equal(H(tap, hip).reshape(F, k, k, C), w.transpose(0, 2, 3, 1))
    assert np.array_equal(H(flip, hip).reshape(C, k, k, F), w[:, :, ::-1, ::-1].transpose(1, 2, 3, 0))
    flip2 = torch.empty(w.size, dtype=torch.float32, device="cuda")
    hip.packConvWeightsDgrad(F, C, k, D(w), None, flip2)
    assert np.array_equal(H(flip2, hip), H(flip, hip))


@pytest.mark.parametrize("B,F,C,hh", [(128, 64, 32, 16), (128, 128, 64, 8), (3, 48, 16, 10)])
def test_conv_input_delta_as_convolution(hip, B, F, C, hh):
    """The conv input delta as tnh_conv2d_fwd of the output delta with the
    flipped weights (3x3, stride 1, pad 1) against torch's transposed
    convolution in float64 and against the reference sequence (TN product +
    col2im) on the GPU, within 1e-5 per tensor."""
    case(f"conv input delta B{B} F{F} C{C} {hh}x{hh}")
    w = synth.normal(341, (F, C, 3, 3), 0.1)
    d = synth.normal(342, (B, F, hh, hh))
    ref = torch.nn.functional.conv_transpose2d(torch.from_numpy(d).double(), torch.from_numpy(w).double(),
                                               padding=1).numpy()
    flip = torch.empty(w.size, dtype=torch.float32, device="cuda")
    hip.packConvWeightsDgrad(F, C, 3, D(w), None, flip)
    dx = torch.empty((B, C, hh, hh), dtype=torch.float32, device="cuda")
    hip.conv2dForward(B, F, hh, hh, C, 3, 1, 1, D(d), 0, flip, None, acLINEAR, dx, 0, weightLayout=WEIGHTS_TAP_MAJOR)
    got = H(dx, hip)
    assert R.rel_err(got, ref) <= TOL
    K, L = C * 9, hh * hh
    col = torch.empty((B, K, L), dtype=torch.float32, device="cuda")
    hip.gemmStridedBatched(True, False, K, L, F, 1.0, D(w.reshape(F, K)), 0, K, 0, D(d), 0, L, F * L, 0.0, col, 0, L,
                           K * L, B)
    dx2 = torch.zeros((B, C, hh, hh), dtype=torch.float32, device="cuda")
    hip.col2imStridedBatched(C, hh, hh, 3, 3, 1, 1, 1, 1, 1, 1, col, K * L, 0, dx2, C * hh * hh, 0, B)
    assert R.rel_err(got, H(dx2, hip)) <= TOL


@pytest.mark.parametrize("shape,act", [((128, 32, 32, 32), acLEAKY), ((8, 64, 8, 8), acLEAKY), ((3, 5, 7, 9), acLINEAR),
                                       ((4, 8, 2, 2), acLEAKY)])
def test_bn_backward_equals_the_sequence(hip, shape, act):
    """tnh_bn_backward (three launches; four for rows of 4 elements, whose
    workgroups would hold 256 channel rows) against bnBackwardScale,
    meansAndVarsDelta and normalizeDelta: delta, dgamma and the mean /
    variance deltas bit for bit."""
    case(f"bn_backward {shape} act{act}")
    B, F, h, w = shape
    n = B * F * h * w
    out = synth.normal(350, shape)
    xn = synth.normal(351, shape)
    x = synth.normal(352, shape)
    gamma = synth.normal(353, (F,))
    mean = synth.normal(354, (F,), 0.1)
    var = np.abs(synth.normal(355, (F,))) + np.float32(0.5)
    d0 = synth.normal(356, shape)
    su0 = synth.normal(357, (F,))
    res = []
    for fused in (True, False):
        d, su = D(d0), D(su0)
        md = torch.empty(F, dtype=torch.float32, device="cuda")
        vd = torch.empty(F, dtype=torch.float32, device="cuda")
        if fused:
            hip.bnBackward(n, F, B, D(out), act, D(xn), D(x), D(gamma), D(mean), D(var), d, su, md, vd)
        else:
            hip.bnBackwardScale(n, F, B, D(out), act, D(xn), D(gamma), d, su)
            hip.meansAndVarsDelta(n, F, B, d, D(x), 0, D(mean), D(var), md, vd)
            hip.normalizeDelta(n, F, B, d, D(x), 0, D(mean), D(var), md, vd)
        res.append([H(t_, hip).copy() for t_ in (d, su, md, vd)])
    for a, b in zip(*res):
        assert np.array_equal(a, b)


def _bn_back_inputs(shape, seed):
    B, F, h, w = shape
    out = synth.normal(seed, shape)
    xn = synth.normal(seed + 1, shape)
    x = synth.normal(seed + 2, shape)
    gamma = synth.normal(seed + 3, (F,))
    mean = synth.normal(seed + 4, (F,), 0.1)
    var = np.abs(synth.normal(seed + 5, (F,))) + np.float32(0.5)
    return [D(a) for a in (out, xn, x, gamma, mean, var)], synth.normal(seed + 6, (F,))


@pytest.mark.parametrize("shape,act", [((128, 32, 32, 32), acLEAKY), ((4, 3, 6, 6), acLINEAR),
                                       ((2, 5, 4, 8), acLEAKY), ((3, 2, 2, 2), acLEAKY)])
def test_bn_backward_maxpool_equals_the_calls(hip, shape, act):
    """tnh_bn_backward_maxpool against tnh_maxpool_bwd into a zeroed delta
    then tnh_bn_backward: delta, dgamma and the mean / variance deltas bit
    for bit, with ties in the windows and +0 / -0 pool deltas; the fused
    call does not read its delta (NaN before); indexes it did not see a
    2x2 stride-2 pool write are refused."""
    case(f"bn_backward_maxpool {shape} act{act}")
    B, F, h, w = shape
    n = B * F * h * w
    src = synth.normal(390, shape)
    src[0, 0, 0, :2] = src[0, 0, 1, :2] = 0.25  # a tie inside the first window
    pidx = torch.empty((B, F, h // 2, w // 2), dtype=torch.int64, device="cuda")
    pooled = torch.empty((B, F, h // 2, w // 2), dtype=torch.float32, device="cuda")
    hip.forwardMaxPool(B, F, h // 2, w // 2, D(src), F, h, w, 2, 2, 0, 2, pidx, pooled)
    pdel = synth.normal(391, (B, F, h // 2, w // 2))
    pdel.reshape(-1)[::7] = np.float32(-0.0)
    pdel.reshape(-1)[3::11] = np.float32(0.0)
    (out, xn, x, gamma, mean, var), su0 = _bn_back_inputs(shape, 392)
    res = []
    for fused in (True, False):
        su = D(su0)
        md = torch.empty(F, dtype=torch.float32, device="cuda")
        vd = torch.empty(F, dtype=torch.float32, device="cuda")
        if fused:
            d = torch.full(shape, float("nan"), dtype=torch.float32, device="cuda")
            hip.bnBackwardMaxPool(n, F, B, h, w, pidx, D(pdel), out, act, xn, x, gamma, mean, var, d, su, md, vd)
        else:
            d = torch.zeros(shape, dtype=torch.float32, device="cuda")
            hip.backwardMaxPool(B, F, h // 2, w // 2, d, pidx, D(pdel))
            hip.bnBackward(n, F, B, out, act, xn, x, gamma, mean, var, d, su, md, vd)
        res.append([H(t_, hip).copy() for t_ in (d, su, md, vd)])
    for a, b in zip(*res):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    # an address no pool wrote (8 bytes past an allocation's start)
    other = torch.zeros(pidx.numel() + 1, dtype=torch.int64, device="cuda")[1:]
    with pytest.raises(TNHError, match="2x2"):
        hip.bnBackwardMaxPool(n, F, B, h, w, other, D(pdel), out, act, xn, x, gamma, mean, var, d, su, md, vd)


@pytest.mark.parametrize("shape,act", [((128, 128, 8, 8), acLEAKY), ((3, 5, 3, 3), acLINEAR),
                                       ((2, 4, 1, 1), acLEAKY)])
def test_bn_backward_avgpool_equals_the_calls(hip, shape, act):
    """tnh_bn_backward_avgpool against tnh_avgpool_bwd into a zeroed delta
    then tnh_bn_backward, bit for bit (-0 pool deltas included); the fused
    call does not read its delta."""
    case(f"bn_backward_avgpool {shape} act{act}")
    B, F, h, w = shape
    n = B * F * h * w
    adel = synth.normal(395, (B, F))
    adel.reshape(-1)[::5] = np.float32(-0.0)
    (out, xn, x, gamma, mean, var), su0 = _bn_back_inputs(shape, 396)
    res = []
    for fused in (True, False):
        su = D(su0)
        md = torch.empty(F, dtype=torch.float32, device="cuda")
        vd = torch.empty(F, dtype=torch.float32, device="cuda")
        if fused:
            d = torch.full(shape, float("nan"), dtype=torch.float32, device="cuda")
            hip.bnBackwardAvgPool(n, F, B, D(adel), out, act, xn, x, gamma, mean, var, d, su, md, vd)
        else:
            d = torch.zeros(shape, dtype=torch.float32, device="cuda")
            hip.avgPoolBackward(B, F, h, w, D(adel), d)
            hip.bnBackward(n, F, B, out, act, xn, x, gamma, mean, var, d, su, md, vd)
        res.append([H(t_, hip).copy() for t_ in (d, su, md, vd)])
    for a, b in zip(*res):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("shape,rolling", [((128, 32, 32, 32), True), ((128, 64, 16, 16), True), ((4, 3, 6, 8), False),
                                           ((8, 4, 2, 4), True)])
def test_bn_train_forward_maxpool_equals_the_calls(hip, shape, rolling):
    """tnh_bn_train_forward_maxpool against tnh_bn_statistics then
    tnh_bn_forward_maxpool: mean, variance, the rolling statistics, x_norm,
    out, the pooled values and indices bit for bit (planes of 2x4 take the
    path with the final step in its own launch)."""
    case(f"bn_train_forward_maxpool {shape} rolling{rolling}")
    B, F, h, w = shape
    n = B * F * h * w
    x = synth.normal(400, shape) * np.float32(1.7) + np.float32(0.3)
    gamma, beta = synth.normal(401, (F,)), synth.normal(402, (F,))
    rm0, rv0 = synth.normal(403, (F,)), np.abs(synth.normal(404, (F,)))
    m = float(np.float32(0.1))
    res = []
    for fused in (True, False):
        mean = torch.empty(F, dtype=torch.float32, device="cuda")
        var = torch.empty(F, dtype=torch.float32, device="cuda")
        rm, rv = (D(rm0), D(rv0)) if rolling else (None, None)
        xn = torch.empty(shape, dtype=torch.float32, device="cuda")
        out = torch.empty(shape, dtype=torch.float32, device="cuda")
        pool = torch.empty((B, F, h // 2, w // 2), dtype=torch.float32, device="cuda")
        pidx = torch.empty((B, F, h // 2, w // 2), dtype=torch.int64, device="cuda")
        if fused:
            hip.bnTrainForwardMaxPool(B, F, h, w, D(x), xn, out, mean, var, rm, rv, m, D(gamma), D(beta), acLEAKY,
                                      pool, pidx)
        else:
            hip.bnStatistics(n, F, B, D(x), 0, mean, var, rm, rv, m)
            hip.bnForwardMaxPool(B, F, h, w, D(x), xn, out, mean, var, D(gamma), D(beta), acLEAKY, pool, pidx)
        res.append([H(t_, hip).copy() for t_ in (mean, var, xn, out, pool, pidx) + ((rm, rv) if rolling else ())])
    for a, b in zip(*res):
        assert np.array_equal(a, b)


@pytest.mark.parametrize("shape", [(128, 128, 8, 8), (3, 5, 3, 3), (6, 7, 1, 1)])
def test_bn_train_forward_avgpool_equals_the_calls(hip, shape):
    """tnh_bn_train_forward_avgpool against tnh_bn_statistics then
    tnh_bn_forward_avgpool, bit for bit."""
    case(f"bn_train_forward_avgpool {shape}")
    B, F, h, w = shape
    n = B * F * h * w
    x = synth.normal(405, shape)
    gamma, beta = synth.normal(406, (F,)), synth.normal(407, (F,))
    rm0, rv0 = synth.normal(408, (F,)), np.abs(synth.normal(409, (F,)))
    m = float(np.float32(0.1))
    res = []
    for fused in (True, False):
        mean = torch.empty(F, dtype=torch.float32, device="cuda")
        var = torch.empty(F, dtype=torch.float32, device="cuda")
        rm, rv = D(rm0), D(rv0)
        xn = torch.empty(shape, dtype=torch.float32, device="cuda")
        out = torch.empty(shape, dtype=torch.float32, device="cuda")
        avg = torch.empty((B, F), dtype=torch.float32, device="cuda")
        if fused:
            hip.bnTrainForwardAvgPool(B, F, h * w, D(x), xn, out, mean, var, rm, rv, m, D(gamma), D(beta), acLEAKY,
                                      avg)
        else:
            hip.bnStatistics(n, F, B, D(x), 0, mean, var, rm, rv, m)
            hip.bnForwardAvgPool(B, F, h * w, D(x), xn, out, mean, var, D(gamma), D(beta), acLEAKY, avg)
        res.append([H(t_, hip).copy() for t_ in (mean, var, rm, rv, xn, out, avg)])
    for a, b in zip(*res):
        assert np.array_equal(a, b)


def test_cifar_step_fused_stats_equals_the_calls(hip):
    """The training step with the statistics' final steps taken by the
    normalize passes gives the same bits as with bnStatistics."""
    case("cifar step fused statistics vs calls")
    params = trainnet.init_params()
    x, truth = _batch(324, 16)
    keys = ("u_w0", "u_w1", "u_w2", "u_s0", "u_s1", "u_s2", "w0", "w1", "w2", "u_fw", "rm0", "rv1", "rm2")
    out = []
    for fused in (True, False):
        gpu = trainnet.CifarTrainer(hip, params, 16, fused_stats=fused)
        gpu.forward(D(x), D(truth))
        gpu.backward()
        gpu.update()
        out.append({k: gpu.host(k).copy() for k in keys})
    for k in keys:
        assert np.array_equal(out[0][k], out[1][k]), k


XNORM_CASES = [(shape, form, acLEAKY) for shape in [(16, 32, 32, 32), (8, 64, 8, 8), (3, 5, 6, 6), (6, 7, 1, 1)]
               for form in ("plain", "maxpool", "avgpool") if not (form == "maxpool" and shape[2] == 1)]
XNORM_CASES += [((4, 6, 8, 8), "plain", acLOGISTIC), ((4, 6, 8, 8), "plain", acLINEAR)]


@pytest.mark.parametrize("shape,form,act", XNORM_CASES)
def test_bn_backward_forms_xnorm(hip, shape, form, act):
    """tnh_bn_backward (and its _maxpool / _avgpool forms) with xNorm NULL
    (x_norm formed in the first pass from x, mean and variance) and with
    output NULL too (the activation's output formed from x_norm, the scales
    and the biases), against the same call given what tnh_bn_forward stored:
    every output bit for bit (planes of one element take the other variance
    clamp)."""
    B, F, h, w = shape
    case(f"bn_backward xNorm / output NULL {form} {shape} act{act}")
    n = B * F * h * w
    x = synth.normal(410, shape, 1.5)
    mean = synth.normal(411, (F,), 0.1)
    var = np.abs(synth.normal(412, (F,))) + np.float32(0.3)
    var[0] = np.float32(1e-13)  # below both clamps
    gamma, beta = synth.normal(413, (F,)), synth.normal(414, (F,))
    dx, dm, dv, dg, db = D(x), D(mean), D(var), D(gamma), D(beta)
    xn = torch.empty(shape, dtype=torch.float32, device="cuda")
    out = torch.empty(shape, dtype=torch.float32, device="cuda")
    hip.bnForward(n, F, B, dx, xn, out, dm, dv, dg, db, act)
    d0 = synth.normal(415, shape)
    su0 = synth.normal(416, (F,))
    extra = ()
    if form == "maxpool":
        pidx = torch.empty((B, F, h // 2, w // 2), dtype=torch.int64, device="cuda")
        pooled = torch.empty((B, F, h // 2, w // 2), dtype=torch.float32, device="cuda")
        hip.forwardMaxPool(B, F, h // 2, w // 2, out, F, h, w, 2, 2, 0, 2, pidx, pooled)
        extra = (pidx, D(synth.normal(417, (B, F, h // 2, w // 2))))
    elif form == "avgpool":
        extra = (D(synth.normal(418, (B, F))),)
    res = []
    for given in ("both", "out", "none"):
        d, su = D(d0), D(su0)
        md = torch.empty(F, dtype=torch.float32, device="cuda")
        vd = torch.empty(F, dtype=torch.float32, device="cuda")
        rest = (None if given == "none" else out, act, xn if given == "both" else None, dx, dg, dm, dv, d, su, md,
                vd, db)
        if form == "plain":
            hip.bnBackward(n, F, B, *rest)
        elif form == "maxpool":
            hip.bnBackwardMaxPool(n, F, B, h, w, *extra, *rest)
        else:
            hip.bnBackwardAvgPool(n, F, B, *extra, *rest)
        res.append([H(t_, hip).copy() for t_ in (d, su, md, vd)])
    for other in res[1:]:
        for a, b in zip(res[0], other):
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_cifar_step_formed_xnorm_equals_stored(hip):
    """The training step with x_norm and the activation outputs formed
    again in the backward gives the same bits as with both stored by the
    forward."""
    case("cifar step x_norm formed vs stored")
    params = trainnet.init_params()
    x, truth = _batch(326, 16)
    keys = ("u_w0", "u_w1", "u_w2", "u_s0", "u_s1", "u_s2", "w0", "w1", "w2", "u_fw", "s2")
    out = []
    for keep in (True, False):
        gpu = trainnet.CifarTrainer(hip, params, 16, store_bn_outputs=keep)
        gpu.forward(D(x), D(truth))
        gpu.backward()
        gpu.update()
        out.append({k: gpu.host(k).copy() for k in keys})
    for k in keys:
        assert np.array_equal(out[0][k], out[1][k]), k


def test_cifar_step_fused_pool_bwd_equals_the_calls(hip):
    """The training step with the pool backwards formed inside the
    batch-norm backwards (no zeroed deltas) gives the same bits as with
    backwardMaxPool / avgPoolBackward into zeroed deltas, with the fused
    tail and with the call-by-call tail."""
    case("cifar step fused pool backward vs calls")
    params = trainnet.init_params()
    x, truth = _batch(323, 16)
    keys = ("u_w0", "u_w1", "u_w2", "u_s0", "u_s1", "u_s2", "w0", "w1", "w2", "u_fw", "u_fb")
    for head in (True, False):
        out = []
        for fused in (True, False):
            gpu = trainnet.CifarTrainer(hip, params, 16, fused_head=head, fused_pool_bwd=fused)
            gpu.forward(D(x), D(truth))
            gpu.backward()
            gpu.update()
            out.append({k: gpu.host(k).copy() for k in keys})
        for k in keys:
            assert np.array_equal(out[0][k], out[1][k]), (head, k)


def test_sgd_update_pack_equals_update_then_pack(hip):
    """tnh_sgd_update_pack: the weights and momenta of tnh_sgd_update bit for
    bit, and each listed layer's tap-major / flipped copies equal to
    tnh_conv2d_pack_weights_dgrad of the updated weights; elements outside
    the layers (a connected layer in the same arena) only updated; the
    parameter arena updated as tnh_param_update does, in the same launch and
    with no layer table too."""
    case("sgd_update_pack")
    layers = [(32, 3, 9), (64, 32, 9), (10, 6, 1)]
    sizes = [f * c * t for f, c, t in layers]
    n = sum(sizes) + 1290
    w0 = synth.normal(360, (n,))
    u0 = synth.normal(361, (n,))
    wa, ua = D(w0), D(u0)
    hip.sgdUpdate(n, 1e-3, 128, 0.9, 1e-4, wa, ua)
    wb, ub = D(w0), D(u0)
    offs = np.concatenate([[0], np.cumsum(sizes)])[:-1] + 1290  # the connected layer first
    taps = [torch.empty(sz, dtype=torch.float32, device="cuda") for sz in sizes]
    flips = [torch.empty(sz, dtype=torch.float32, device="cuda") for sz in sizes]
    npar = 1234
    p0, pu0 = synth.normal(362, (npar,)), synth.normal(363, (npar,))
    pa, pua = D(p0), D(pu0)
    hip.paramUpdate(npar, 1e-3, 128, 0.9, pa, pua)
    pb, pub = D(p0), D(pu0)
    hip.sgdUpdatePack(n, 1e-3, 128, 0.9, 1e-4, wb, ub,
                      [(int(o), f, c, t, tp, fl if i > 0 else None)
                       for i, ((f, c, t), o, tp, fl) in enumerate(zip(layers, offs, taps, flips))], npar, pb, pub)
    wref = H(wa, hip)
    assert np.array_equal(H(wb, hip), wref) and np.array_equal(H(ub, hip), H(ua, hip))
    assert np.array_equal(H(pb, hip), H(pa, hip)) and np.array_equal(H(pub, hip), H(pua, hip))
    # no layer table: the plain update of both arenas
    wc, uc, pc, puc = D(w0), D(u0), D(p0), D(pu0)
    hip.sgdUpdatePack(n, 1e-3, 128, 0.9, 1e-4, wc, uc, [], npar, pc, puc)
    assert np.array_equal(H(wc, hip), wref) and np.array_equal(H(uc, hip), H(ua, hip))
    assert np.array_equal(H(pc, hip), H(pa, hip)) and np.array_equal(H(puc, hip), H(pua, hip))
    for i, ((f, c, t), o) in enumerate(zip(layers, offs)):
        k = int(round(t ** 0.5))
        tp = torch.empty(f * c * t, dtype=torch.float32, device="cuda")
        fl = torch.empty(f * c * t, dtype=torch.float32, device="cuda")
        hip.packConvWeightsDgrad(f, c, k, wa[int(o):int(o) + f * c * t], tp, fl)
        assert np.array_equal(H(taps[i], hip), H(tp, hip)), i
        if i > 0:
            assert np.array_equal(H(flips[i], hip), H(fl, hip)), i


@pytest.mark.parametrize("shape,act,idx", [((128, 32, 32, 32), acLEAKY, True), ((4, 3, 6, 8), acLINEAR, True),
                                           ((2, 5, 4, 12), acLEAKY, False)])
def test_bn_forward_maxpool_equals_the_two_calls(hip, shape, act, idx):
    """tnh_bn_forward_maxpool against tnh_bn_forward then tnh_maxpool_fwd
    (2x2, stride 2): x_norm, out, the pooled values and int64 indices bit
    for bit (ties included); the 7-argument maxpool backward then finds the
    geometry (the plain scatter, equal to the oracle's)."""
    case(f"bn_forward_maxpool {shape} act{act} idx{idx}")
    B, F, h, w = shape
    n = B * F * h * w
    x = synth.normal(370, shape)
    x[0, 0, 0, :4] = x[0, 0, 1, :4] = 0.25  # ties inside the first windows
    mean, var = synth.normal(371, (F,), 0.1), np.abs(synth.normal(372, (F,))) + np.float32(0.5)
    gamma, beta = synth.normal(373, (F,)), synth.normal(374, (F,))
    res = []
    for fused in (True, False):
        xn = torch.empty(shape, dtype=torch.float32, device="cuda")
        out = torch.empty(shape, dtype=torch.float32, device="cuda")
        pool = torch.empty((B, F, h // 2, w // 2), dtype=torch.float32, device="cuda")
        pidx = torch.empty((B, F, h // 2, w // 2), dtype=torch.int64, device="cuda") if idx else None
        if fused:
            hip.bnForwardMaxPool(B, F, h, w, D(x), xn, out, D(mean), D(var), D(gamma), D(beta), act, pool, pidx)
        else:
            hip.bnForward(n, F, B, D(x), xn, out, D(mean), D(var), D(gamma), D(beta), act)
            hip.forwardMaxPool(B, F, h // 2, w // 2, out, F, h, w, 2, 2, 0, 2, pidx, pool)
        res.append([H(t_, hip).copy() for t_ in (xn, out, pool) + ((pidx,) if idx else ())])
    for a, b in zip(*res):
        assert np.array_equal(a, b)
    if idx:
        delta = synth.normal(375, (B, F, h // 2, w // 2))
        base = synth.normal(376, shape)
        ref = R.maxpool_bwd(res[0][3], delta, base.copy())
        xn = torch.empty(shape, dtype=torch.float32, device="cuda")
        out = torch.empty(shape, dtype=torch.float32, device="cuda")
        pool = torch.empty((B, F, h // 2, w // 2), dtype=torch.float32, device="cuda")
        pidx = torch.empty((B, F, h // 2, w // 2), dtype=torch.int64, device="cuda")
        hip.bnForwardMaxPool(B, F, h, w, D(x), xn, out, D(mean), D(var), D(gamma), D(beta), act, pool, pidx)
        db = D(base)
        hip.backwardMaxPool(B, F, h // 2, w // 2, db, pidx, D(delta))
        assert np.array_equal(H(db, hip), ref)


@pytest.mark.parametrize("shape", [(128, 128, 8, 8), (3, 5, 4, 4), (2, 7, 1, 1), (4, 3, 3, 5)])
@pytest.mark.parametrize("act", [acLEAKY, acLINEAR])
def test_bn_forward_avgpool_equals_the_two_calls(hip, shape, act):
    """tnh_bn_forward_avgpool against tnh_bn_forward then tnh_avgpool_fwd:
    x_norm, out and the plane averages bit for bit (planes of one element
    take the other variance clamp, as tnh_bn_forward does)."""
    case(f"bn_forward_avgpool {shape} act{act}")
    B, F, h, w = shape
    n = B * F * h * w
    x = synth.normal(380, shape)
    mean, var = synth.normal(381, (F,), 0.1), np.abs(synth.normal(382, (F,))) + np.float32(0.5)
    var[0] = np.float32(1e-13)  # below the clamps: the two forms differ here
    gamma, beta = synth.normal(383, (F,)), synth.normal(384, (F,))
    res = []
    for fused in (True, False):
        xn = torch.empty(shape, dtype=torch.float32, device="cuda")
        out = torch.empty(shape, dtype=torch.float32, device="cuda")
        avg = torch.empty((B, F), dtype=torch.float32, device="cuda")
        if fused:
            hip.bnForwardAvgPool(B, F, h * w, D(x), xn, out, D(mean), D(var), D(gamma), D(beta), act, avg)
        else:
            hip.bnForward(n, F, B, D(x), xn, out, D(mean), D(var), D(gamma), D(beta), act)
            hip.avgPoolForward(B, F, h, w, out, avg)
        res.append([H(t_, hip).copy() for t_ in (xn, out, avg)])
    for a, b in zip(*res):
        assert np.array_equal(a, b)
    # the averages against a float64 mean, within rounding
    ref = res[1][1].reshape(B * F, h * w).astype(np.float64).mean(axis=1).reshape(B, F)
    assert np.abs(res[0][2] - ref).max() <= 1e-5 * max(1.0, np.abs(ref).max())


@pytest.mark.parametrize("B,F,hw,classes", [(128, 128, 64, 10), (5, 37, 9, 3)])
def test_softmax_head(hip, B, F, hw, classes):
    """The fused tail against the oracle's sequence on the same inputs: the
    averages within 1e-6 of float64; given the GPU's averages, the logits
    (sdot_avx2 order + bias), the softmax, the cross-entropy delta, the
    weight gradient (TN saxpy chains), the input delta (NN chains) and the
    average-pool backward bit for bit; the error within 1e-6, the bias
    gradient within 1e-6 (the oracle sums in float64)."""
    case(f"softmax head B{B} F{F} hw{hw} classes{classes}")
    x = synth.normal(380, (B, F, hw))
    W = synth.normal(381, (classes, F), 0.2)
    bias = synth.normal(382, (classes,), 0.1)
    lab = (synth.splitmix64(383, B) % np.uint64(classes)).astype(np.int64)
    truth = np.zeros((B, classes), np.float32)
    truth[np.arange(B), lab] = 1
    dev = lambda *sh: torch.empty(sh, dtype=torch.float32, device="cuda")  # noqa: E731
    avg, logits, prob, delta, err = dev(B, F), dev(B, classes), dev(B, classes), dev(B, classes), dev(B, classes)
    dW = D(W)
    hip.softmaxHeadForward(B, F, hw, classes, D(x), avg, dW, D(bias), D(truth), logits, prob, delta, err)
    a = H(avg, hip)
    assert np.max(np.abs(a - x.astype(np.float64).mean(axis=2))) <= 1e-6 * max(1.0, np.abs(a).max())
    ref = np.zeros((B, classes), np.float32)
    R.sgemm(0, 1, B, classes, F, 1.0, a, F, W, F, 0.0, ref, classes)
    ref = R.forward_bias(ref, bias, B)
    assert np.array_equal(H(logits, hip), ref)
    p_ref = R.softmax_rows(ref)
    assert np.array_equal(H(prob, hip), p_ref)
    d_ref, e_ref = T.cross_entropy(p_ref, truth)
    assert np.array_equal(H(delta, hip), d_ref)
    assert np.max(np.abs(H(err, hip) - e_ref)) <= 1e-6 * max(1.0, np.abs(e_ref).max())
    # backward from a delta that the clamp cuts
    dl = synth.normal(384, (B, classes), 1.5)
    uw0, ub0 = synth.normal(385, (classes, F)), synth.normal(386, (classes,))
    base = synth.normal(387, (B, F, hw))
    duw, dub, dda, din, ddl = D(uw0), D(ub0), dev(B, F), D(base), D(dl)
    hip.softmaxHeadBackward(B, F, hw, classes, 1.0, ddl, avg, dW, duw, dub, dda, din)
    dc = T.clamp(dl, -1, 1)
    assert np.array_equal(H(ddl, hip), dc)
    uw = uw0.copy()
    R.sgemm(1, 0, classes, F, B, 1.0, dc, classes, a, F, 1.0, uw, F)
    assert np.array_equal(H(duw, hip), uw)
    assert R.rel_err(H(dub, hip), T.add_sums(ub0, dc, B)) <= 1e-6  # a sequential fp32 sum against float64
    dA = np.zeros((B, F), np.float32)
    R.sgemm(0, 0, B, F, classes, 1.0, dc, classes, W, F, 1.0, dA, F)
    assert np.array_equal(H(dda, hip), dA)
    assert np.array_equal(H(din, hip), T.avgpool_bwd(base.reshape(B, F, hw, 1).copy(), dA).reshape(B, F, hw))


def test_cifar_step_fused_head_matches_the_calls(hip):
    """The training step with the fused tail against the call-by-call tail:
    loss and every gradient within 1e-5 per tensor (the tails' sums run in
    different orders)."""
    case("cifar step fused head vs calls")
    params = trainnet.init_params()
    x, truth = _batch(322, 32)
    out = []
    for fused in (True, False):
        gpu = trainnet.CifarTrainer(hip, params, 32, fused_head=fused, defer_wgrad_sum=False)
        gpu.forward(D(x), D(truth))
        gpu.backward()
        out.append((float(gpu.cost()), {k: gpu.host(k).copy() for k in ("u_fw", "u_fb", "u_w2", "u_s2", "u_w0")}))
    assert abs(out[0][0] - out[1][0]) <= TOL * abs(out[1][0])
    for k in out[0][1]:
        assert R.rel_err(out[0][1][k], out[1][1][k]) <= TOL, k


def test_cifar_step_deferred_wgrad_sum_equals_the_calls(hip):
    """Weight gradients kept as split sums (tnh_conv2d_wgrad_pieces) and added
    by the update's pass (tnh_sgd_update_pack_pieces) against
    tnh_conv2d_wgrad's own reduction: every weight, momentum buffer and the
    packed copies equal bit for bit after two steps."""
    case("cifar step deferred wgrad sums vs tnh_conv2d_wgrad")
    params = trainnet.init_params()
    x, truth = _batch(360, 64)
    keys = ("w0", "w1", "w2", "u_w0", "u_w1", "u_w2", "s1", "u_s2", "fw", "u_fw")
    out = []
    for defer in (True, False):
        gpu = trainnet.CifarTrainer(hip, params, 64, defer_wgrad_sum=defer)
        if defer:
            assert gpu.pieces[0] is None and gpu.pieces[1] is not None and gpu.pieces[2] is not None
        dx, dt = D(x), D(truth)
        for _ in range(2):
            gpu.step(dx, dt)
        hip.finish()
        got = {k: gpu.host(k).copy() for k in keys}
        got["packed2"] = gpu.packed[2].numpy()
        got["flipped1"] = gpu.flipped[1].numpy()
        out.append(got)
    for k in out[0]:
        assert np.array_equal(out[0][k], out[1][k]), k


@pytest.mark.parametrize("B,C,H,F", [(4, 32, 16, 64), (1, 64, 8, 128), (2, 16, 32, 24)])
def test_wgrad_pieces_through_the_update_equal_wgrad(hip, B, C, H, F):
    """tnh_conv2d_wgrad_pieces + tnh_sgd_update_pack_pieces against
    tnh_conv2d_wgrad (alpha = beta = 1) + tnh_sgd_update_pack on the same
    data: updated weights, momentum buffer and tap-major copy equal bit for
    bit (a single piece included: batch 1, 8x8); gradients of fewer than 8192
    weights in several pieces are refused."""
    case(f"wgrad pieces B{B} C{C} H{H} F{F}")
    from tensorium_amd.nnhip import DeviceArray

    K = C * 9
    x = synth.uniform(370, (B, C, H, H), -1, 1)
    d = synth.normal(371, (B, F, H, H), 1.0)
    w0 = synth.normal(372, (F * K,), 0.05)
    u0 = synth.normal(373, (F * K,), 0.01)
    dx, dd = DeviceArray.from_numpy(x), DeviceArray.from_numpy(d)
    if F * K < 8192:  # 16 pieces here: refused, the query included
        with pytest.raises(TNHError, match="wave"):
            hip.convWeightGradientPieces(B, C, H, H, F, 3, 3, 1, 1, 1, 1, 1, 1, dx, C * H * H, dd, F * H * H)
        return
    res = []
    for deferred in (True, False):
        w, u = DeviceArray.from_numpy(w0), DeviceArray.from_numpy(u0)
        tap = DeviceArray(F * K)
        layer = [(0, F, C, 9, tap, None)]
        if deferred:
            n = hip.convWeightGradientPieces(B, C, H, H, F, 3, 3, 1, 1, 1, 1, 1, 1, dx, C * H * H, dd, F * H * H)
            pieces = DeviceArray(n * F * K)
            with pytest.raises(TNHError, match="fewer than"):
                hip.convWeightGradientPieces(B, C, H, H, F, 3, 3, 1, 1, 1, 1, 1, 1, dx, C * H * H, dd, F * H * H,
                                             pieces, n * F * K - 1)
            assert hip.convWeightGradientPieces(B, C, H, H, F, 3, 3, 1, 1, 1, 1, 1, 1, dx, C * H * H, dd,
                                                F * H * H, pieces, n * F * K) == n
            hip.sgdUpdatePack(F * K, 1e-3, B, 0.9, 1e-4, w, u, layer, pieces=[(pieces, n)])
        else:
            hip.convWeightGradient(B, C, H, H, F, 3, 3, 1, 1, 1, 1, 1, 1, dx, C * H * H, dd, F * H * H, 1.0, 1.0, u)
            hip.sgdUpdatePack(F * K, 1e-3, B, 0.9, 1e-4, w, u, layer)
        res.append((w.numpy(), u.numpy(), tap.numpy()))
    for a, b in zip(*res):
        assert np.array_equal(a, b)
