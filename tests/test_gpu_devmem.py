"""The library on its own device memory: buffers from tnh_malloc
(TNNHip.createDeviceBuffer, TNNCuda.createDeviceBuffer nncuda.pas:488),
uploads and downloads through tnh_h2d / tnh_d2h (writeBuffer / readBuffer,
nncuda.pas:512, 499), no torch tensor anywhere: what a Pascal caller of
pascal/nnhip.pas does.  Checked against the CPU oracle."""
import numpy as np
import pytest

from oracle import refcpu as R
from tensorium_amd import synth
from tensorium_amd.nnhip import WEIGHTS_TAP_MAJOR, DeviceBuffer, acLEAKY

pytestmark = pytest.mark.gpu


def case(msg):
    print(f"[case] {msg}", flush=True)


def up(hip, a):
    a = np.ascontiguousarray(a, dtype=np.float32)
    buf = hip.createDeviceBuffer(a.size)
    hip.writeBuffer(buf, a.nbytes, a)
    return buf


def down(hip, buf, shape):
    out = np.empty(shape, np.float32)
    hip.finish()
    hip.readBuffer(buf, out.nbytes, out)
    return out


@pytest.mark.parametrize("B,C,H,F,k", [(2, 64, 26, 128, 3), (1, 32, 13, 64, 1)])
def test_conv_on_library_buffers(hip, B, C, H, F, k):
    """conv (reference-layout and packed weights) + bias + leaky on
    tnh_malloc buffers only: within 1e-5 of the oracle."""
    case(f"devmem conv B{B} C{C} H{H} F{F} k{k}")
    p = k // 2
    x = synth.uniform(501, (B, C, H, H))
    Wt = synth.normal(502, (F, C * k * k), (2.0 / (C * k * k)) ** 0.5)
    b = synth.normal(503, (F,), 0.1)
    ref = R.conv_forward(x, Wt, b, k, 1, p, acLEAKY)
    bufs = [up(hip, x), up(hip, Wt), up(hip, b)]
    out = hip.createDeviceBuffer(ref.size)
    packed = hip.createDeviceBuffer(Wt.size)
    try:
        assert all(isinstance(t, DeviceBuffer) for t in bufs + [out, packed])
        hip.conv2dForward(B, C, H, H, F, k, 1, p, bufs[0], 0, bufs[1], bufs[2], acLEAKY, out, 0)
        assert R.rel_err(down(hip, out, ref.shape), ref) <= 1e-5
        hip.packConvWeights(F, C, k, bufs[1], packed)
        hip.conv2dForward(B, C, H, H, F, k, 1, p, bufs[0], 0, packed, bufs[2], acLEAKY, out, 0,
                          weightLayout=WEIGHTS_TAP_MAJOR)
        assert R.rel_err(down(hip, out, ref.shape), ref) <= 1e-5
    finally:
        for t in bufs + [out, packed]:
            hip.freeDeviceBuffer(t)


def test_sgemm_on_library_buffers(hip):
    """TNNHip.gemm on tnh_malloc buffers: integer-valued operands make the
    product exact, so it must equal numpy's bit for bit."""
    case("devmem sgemm 256x192x320")
    M, N, K = 256, 192, 320
    rng = np.random.default_rng(504)
    A = rng.integers(-8, 9, (M, K)).astype(np.float32)
    Bm = rng.integers(-8, 9, (K, N)).astype(np.float32)
    a, bb = up(hip, A), up(hip, Bm)
    c = hip.createDeviceBuffer(M * N)
    try:
        hip.gemm(False, False, M, N, K, 1.0, a, 0, K, bb, 0, N, 0.0, c, 0, N)
        assert np.array_equal(down(hip, c, (M, N)), A @ Bm)
    finally:
        for t in (a, bb, c):
            hip.freeDeviceBuffer(t)


def test_config3_trainer_on_library_memory(hip):
    """The config-3 trainer allocates everything through tnh_malloc
    (DeviceArray): one step on DeviceArray inputs, loss and updated weights
    against the oracle's step within the per-tensor bound."""
    from oracle import trainref as T
    from tensorium_amd import trainnet
    from tensorium_amd.nnhip import DeviceArray

    case("devmem config-3 step B16")
    B = 16
    x = synth.uniform(505, (B, 3, 32, 32))
    lab = (synth.splitmix64(506, B) % np.uint64(10)).astype(np.int64)
    truth = np.zeros((B, 10), np.float32)
    truth[np.arange(B), lab] = 1
    params = trainnet.init_params()
    ref = T.CifarStep(params)
    loss_ref = ref.forward(x, truth)
    ref.backward()
    ref.update(B)
    gpu = trainnet.CifarTrainer(hip, params, B)
    assert all(isinstance(v, DeviceArray) for v in list(gpu.p.values()) + list(gpu.t.values()))
    gpu.forward(DeviceArray.from_numpy(x), DeviceArray.from_numpy(truth))
    gpu.backward()
    loss = gpu.cost()
    gpu.update()
    assert abs(float(loss) - float(loss_ref)) <= 1e-5 * abs(float(loss_ref))
    for k in ("w0", "w1", "w2", "fw", "s1"):
        assert R.rel_err(gpu.host(k), ref.p[k]) <= 1e-5, k


def test_second_stream_from_the_library(hip):
    """tnh_stream_create / tnh_stream_destroy: an SGEMM on a second stream,
    joined through an event, equals the same SGEMM on the context stream;
    destroying the selected stream or the context's own is refused."""
    from tensorium_amd.nnhip import DeviceArray, TNHError

    case("devmem second stream")
    A = synth.uniform(520, (64, 96), -1, 1)
    Bm = synth.uniform(521, (96, 80), -1, 1)
    dA, dB = DeviceArray.from_numpy(A), DeviceArray.from_numpy(Bm)
    c0, c1 = DeviceArray((64, 80)), DeviceArray((64, 80))
    hip.resetStream()
    main = hip.stream
    hip.gemm(False, False, 64, 80, 96, 1.0, dA, 0, 96, dB, 0, 80, 0.0, c0, 0, 80)
    side = hip.streamCreate()
    ev = hip.eventCreate()
    try:
        hip.setStream(side)
        with pytest.raises(TNHError, match="selected"):
            hip.streamDestroy(side)
        hip.gemm(False, False, 64, 80, 96, 1.0, dA, 0, 96, dB, 0, 80, 0.0, c1, 0, 80)
        hip.eventRecord(ev)
        hip.setStream(main)
        hip.streamWaitEvent(ev)
        with pytest.raises(TNHError, match="own stream"):
            hip.streamDestroy(main)
        assert np.array_equal(c0.numpy(), c1.numpy())
    finally:
        hip.resetStream()
        hip.streamDestroy(side)
        hip.eventDestroy(ev)
        hip.useTorchStream()
