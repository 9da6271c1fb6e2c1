"""GPU parity of TNNHip's element-wise methods that serve the layers around
the convolution path (subvv, mulvv, fmavv, power, fmavss, the logistic and
L2 costs, inverseSqrt, SWISH, dropout) against numpy on the same inputs.

Bit-exact where the operation is IEEE fp32 arithmetic with one rounding per
step (sub, mul, a multiply then an add, 1/sqrt, the costs' deltas and the
dropout mask); within 1e-6 relative where a transcendental (log, exp) is
evaluated by a different library; power within one fp32 ulp (the double
result is rounded to fp32 once on both sides, so only a double pow that
differs in its last bit near a rounding boundary can differ)."""
import numpy as np
import pytest
import torch

from tensorium_amd import synth

pytestmark = pytest.mark.gpu


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


def ulps(a, b):
    ia = a.astype(np.float32).view(np.int32).astype(np.int64)
    ib = b.astype(np.float32).view(np.int32).astype(np.int64)
    return np.abs(ia - ib)


@pytest.mark.parametrize("n,inc", [(1, 1), (1000, 1), (777, 3), (70001, 2)])
def test_subvv_mulvv_fmavv_strided(hip, n, inc):
    """subv / mulv / fmav (cuda_sgemm.cu:789, 1664, 1670) with offsets and
    increments: dst[i*incc + dstOffset] = src1[i*inca + o1] op src2[...]."""
    case(f"subvv/mulvv/fmavv n={n} inc={inc}")
    off = 5
    size = off + n * inc + 3
    a = synth.normal(400 + n, (size,))
    b = synth.normal(401 + n, (size,))
    c = synth.normal(402 + n, (size,))
    base = synth.normal(403 + n, (size,))
    sl = slice(off, off + n * inc, inc)
    for name, ref in (("subvv", a[sl] - b[sl]), ("mulvv", a[sl] * b[sl])):
        dd = D(base)
        getattr(hip, name)(n, D(a), off, inc, D(b), off, inc, dd, off, inc)
        got = H(dd, hip)
        exp = base.copy()
        exp[sl] = ref
        assert np.array_equal(got, exp), name
    dd = D(base)
    hip.fmavv(n, D(a), off, inc, D(b), off, inc, D(c), off, inc, dd, off, inc)
    exp = base.copy()
    exp[sl] = (a[sl] * b[sl]).astype(np.float32) + c[sl]
    assert np.array_equal(H(dd, hip), exp)


def test_power(hip):
    """TTensor.power (ntensors.pas:8507-8530) / power (cuda_sgemm.cu:1679):
    y = x^a with the base at xOffset + i*incx."""
    case("power")
    n = 5000
    x = np.abs(synth.normal(410, (2 * n + 1,), 3.0)) + np.float32(1e-3)
    for a in (2.0, 0.5, -1.5, 3.0, 0.0):
        dy = D(np.zeros(n + 2, np.float32))
        hip.power(n, D(x), 1, 2, a, dy, 2, 1)
        got = H(dy, hip)
        ref = np.power(x[1:1 + 2 * n:2].astype(np.float64), np.float64(np.float32(a))).astype(np.float32)
        assert got[0] == 0 and got[1] == 0
        assert int(ulps(got[2:], ref).max()) <= 1, a
    # negative bases with integral exponents
    xn = synth.normal(411, (n,), 2.0)
    dy = D(np.zeros(n, np.float32))
    hip.power(n, D(xn), 0, 1, 3.0, dy, 0, 1)
    ref = np.power(xn.astype(np.float64), 3.0).astype(np.float32)
    assert int(ulps(H(dy, hip), ref).max()) <= 1


@pytest.mark.parametrize("n,off", [(1, 0), (4096, 0), (1000, 37)])
def test_fmavss(hip, n, off):
    """sfmavss (ntensors.pas:3355) through TNNCuda.fmavss (nncuda.pas:1290):
    dst[offset + i] = src[offset + i] * scalar + bias; the elements before
    the offset are left alone (the YOLO head's scale_x_y step,
    nyololayer.pas:1099)."""
    case(f"fmavss n={n} off={off}")
    src = synth.normal(420 + n, (off + n + 4,))
    base = synth.normal(421 + n, src.shape)
    s, bias = np.float32(1.05), np.float32(-0.025)
    dd = D(base)
    hip.fmavss(n, D(src), off, float(s), float(bias), dd)
    exp = base.copy()
    exp[off:off + n] = (src[off:off + n] * s).astype(np.float32) + bias
    assert np.array_equal(H(dd, hip), exp)
    # in place, as TYoloLayer calls it
    dd = D(src)
    hip.fmavss(n, dd, off, float(s), float(bias), dd)
    exp = src.copy()
    exp[off:off + n] = (src[off:off + n] * s).astype(np.float32) + bias
    assert np.array_equal(H(dd, hip), exp)


def test_logistic_and_l2_costs(hip):
    """crossEntropyLogistics (cuda_sgemm.cu:814-828) and cost_l2
    (cuda_sgemm.cu:1655-1662): delta exact, logistic error within 1e-6."""
    case("logistic / L2 costs")
    n = 30001
    p = synth.uniform(430, (n,))
    p[:4] = [0.0, 1.0, 1e-9, 1 - 1e-7]      # the epsilon clamps
    t = (synth.uniform(431, (n,)) > 0.5).astype(np.float32)
    t[4:8] = [0.25, 0.75, 0.0, 1.0]
    dd, de = D(np.zeros(n, np.float32)), D(np.zeros(n, np.float32))
    hip.crossEntropyLogistic(n, D(p), D(t), dd, de)
    assert np.array_equal(H(dd, hip), t - p)
    p64, t64 = p.astype(np.float64), t.astype(np.float64)
    eps = np.float64(np.float32(1e-6))
    err = -t64 * np.log(np.maximum(p64, eps)) - (1 - t64) * np.log(np.maximum((1 - p).astype(np.float64), eps))
    got = H(de, hip).astype(np.float64)
    assert np.max(np.abs(got - err) / np.maximum(np.abs(err), 1e-6)) <= 1e-6
    pr, tr = synth.normal(432, (n,)), synth.normal(433, (n,))
    hip.costL2(n, D(pr), D(tr), dd, de)
    r = tr - pr
    assert np.array_equal(H(dd, hip), r)
    assert np.array_equal(H(de, hip), r * r)


def test_inverse_sqrt(hip):
    """inverse_sqrt (cuda_sgemm.cu:1811-1817): dst = 1/sqrt(max(src, 1e-6))
    at offset + i*stride; fp32 sqrt and divide are correctly rounded."""
    case("inverseSqrt")
    n = 4000
    x = synth.normal(440, (3 * n + 2,), 4.0)
    x[2] = 0.0
    x[5] = 1e-9
    base = synth.normal(441, x.shape)
    dd = D(base)
    hip.inverseSqrt(n, 0.0, D(x), dd, 3, 2)
    sl = slice(2, 2 + 3 * n, 3)
    exp = base.copy()
    exp[sl] = np.float32(1) / np.sqrt(np.maximum(x[sl], np.float32(1e-6)))
    assert np.array_equal(H(dd, hip), exp)


def test_swish(hip):
    """array_activate_swish (cuda_sgemm.cu:512-522): s = 1/(1+exp(-x)),
    output_sigmoid = s, output = x*s, from x + offset."""
    case("SWISH")
    n, off = 20000, 11
    x = synth.normal(450, (off + n,), 6.0)
    ds, do = D(np.zeros(off + n, np.float32)), D(np.zeros(off + n, np.float32))
    hip.activateArraySWISH(n, D(x), off, ds, do)
    xs = x[off:].astype(np.float64)
    s = 1 / (1 + np.exp(-xs))
    gs, go = H(ds, hip)[off:], H(do, hip)[off:]
    assert np.max(np.abs(gs - s) / s) <= 1e-6
    assert np.max(np.abs(go - xs * s) / np.maximum(np.abs(xs * s), 1e-30)) <= 1e-6
    assert np.array_equal(go, x[off:] * gs)


def test_dropout(hip):
    """forward_dropout / backward_dropout (cuda_sgemm.cu:1634-1653): rnd
    holds a uniform [0, 1) draw per element, dst = rnd < p ? 0 : src*scale;
    backward applies the forward's mask.  The draw is splitmix64 of
    (seed, i), the generator of the library's synthetic data."""
    case("dropout")
    n, p = 100003, 0.3
    scale = 1 / (1 - p)
    src = synth.normal(460, (n,))
    drnd, ddst = D(np.zeros(n, np.float32)), D(np.zeros(n, np.float32))
    seed = hip.forwardDropout(n, D(src), p, scale, drnd, ddst, seed=12345)
    assert seed == 12345
    rnd, dst = H(drnd, hip), H(ddst, hip)
    assert np.array_equal(rnd, synth.uniform(12345, (n,)))
    assert rnd.min() >= 0 and rnd.max() < 1
    keep = ~(rnd < np.float32(p))
    assert np.array_equal(dst, np.where(keep, src * np.float32(scale), np.float32(0)))
    assert abs((~keep).mean() - p) < 0.01
    g = synth.normal(461, (n,))
    dg = D(np.zeros(n, np.float32))
    hip.backwardDropout(n, D(g), p, scale, drnd, dg)
    assert np.array_equal(H(dg, hip), np.where(keep, g * np.float32(scale), np.float32(0)))
    # a fresh seed per call when none is given: the masks differ
    s1 = hip.forwardDropout(n, D(src), p, scale, drnd, ddst)
    r1 = H(drnd, hip).copy()
    s2 = hip.forwardDropout(n, D(src), p, scale, drnd, ddst)
    assert s1 != s2 and not np.array_equal(r1, H(drnd, hip))
