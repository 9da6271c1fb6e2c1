"""Pins the oracle's YOLO-head logistic (refcpu.c logistic_ref, exact mode)
bit for bit, independently of the C code.

The reference's AVX2 logistic_array (nactivation.pas:36-127) is an
instruction sequence on float32:
    t = 0 - x                       (vsubps, :59)
    t = t >= MAX_EXP ? MAX_EXP : t  (vcmpgeps/vblendvps, :60-62)
    t = t <= MIN_EXP ? MIN_EXP : t  (vcmpleps/vblendvps, :61-63)
    t = l2e * t                     (vmulps, :64)
    i = floor(t); f = t - i         (vroundps mode 1, vsubps, vcvtps2dq, :65-67)
    p = fma(f, c2, c1)              (vfmadd213ps, :68-69)
    p = fma(p, f, c0)               (vfmadd213ps, :71)
    e = bits(p) + (i << 23)         (vpslld, vpaddd, :70, :72)
    y = 1 / (1 + e)                 (vaddps, then vrcpps :73-74; the parity
                                     gate uses an IEEE division instead of
                                     the host-specific vrcpps)
Here every step is evaluated on exact rationals and rounded once to
float32 (round to nearest, ties to even, with subnormals), which is what
each of those IEEE single-precision instructions does.  The expected bit
patterns below were computed that way and are committed as data; the test
checks the exact derivation still produces them, that the oracle produces
them, that the cases derivable by hand (x = 0; t with fraction 1/2; the
clamps) agree, and that a true-exp sigmoid does not: a restatement that
used expf, dropped a clamp, truncated instead of flooring, or evaluated in
double would fail here."""
import math
from fractions import Fraction as Fr

import numpy as np

from oracle import refcpu as R

# (bits of x, bits of logistic(x)) -- exact-mode reference values
TABLE = [
    (0x00000000, 0x3effc788),  # 0
    (0x80000000, 0x3effc788),  # -0
    (0x3f800000, 0x3f3b1a11),  # 1
    (0xbf800000, 0x3e89b685),  # -1
    (0x3f000000, 0x3f1f71ab),  # 0.5
    (0xc0300000, 0x3d7654de),  # -2.75
    (0x40400000, 0x3f73d6fb),  # 3
    (0xc0e80000, 0x3a3a07df),  # -7.25
    (0x41400000, 0x3f7fff98),  # 12
    (0xc1780000, 0x3447699c),  # -15.5
    (0x41a00000, 0x3f800000),  # 20
    (0xc1a00000, 0x310d80eb),  # -20
    (0x358637bd, 0x3f001c4c),  # 1e-6
    (0xb58637bd, 0x3effc780),  # -1e-6
    (0x42700000, 0x3f800000),  # 60
    (0xc2700000, 0x142d43e7),  # -60
    (0x42aeac4f, 0x3f800000),  # 87.33654 (t at MIN_EXP)
    (0xc2b17217, 0x00200e3d),  # -88.72283 (t at MAX_EXP)
    (0x42c80000, 0x3f800000),  # 100 (t clamped to MIN_EXP)
    (0xc2c80000, 0x00200e3d),  # -100 (t clamped to MAX_EXP)
    (0x7f800000, 0x3f800000),  # +inf
    (0xff800000, 0x00200e3d),  # -inf
    (0x3eb17218, 0x3f15ef0e),  # t = -0.5 exactly
    (0xbfddce9e, 0x3e19c4bd),  # t = 2.5 exactly
    (0x40e8e5bf, 0x3f7fd2c2),  # t = -10.5 exactly
    (0xc073fce1, 0x3cb10771),  # t = 5.5 exactly
]
HALF_POINTS = {0x3eb17218: -0.5, 0xbfddce9e: 2.5, 0x40e8e5bf: -10.5, 0xc073fce1: 5.5}

L2E, C0, C1, C2 = (np.float32(v) for v in ("1.442695041", "1.00172476", "0.657636276", "0.3371894346"))
MAX_EXP, MIN_EXP = np.float32("8.872283E+001"), np.float32("-8.733654E+001")


def f32(q):
    """The float32 nearest to the rational q (ties to even; subnormals;
    overflow to infinity)."""
    if q == 0:
        return np.float32(0.0)
    s = -1 if q < 0 else 1
    a = abs(q)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    while Fr(2) ** e > a:
        e -= 1
    while Fr(2) ** (e + 1) <= a:
        e += 1
    qu = Fr(2) ** (max(e, -126) - 23)
    m = a / qu
    n = m.numerator // m.denominator
    rem = m - n
    if rem > Fr(1, 2) or (rem == Fr(1, 2) and n % 2 == 1):
        n += 1
    r = n * qu
    if r >= Fr(2) ** 128:
        return np.float32(s * math.inf)
    return np.float32(s * float(r))


def Q(v):
    return Fr(float(v))


def bits(v):
    return int(np.float32(v).view(np.uint32))


def from_bits(b):
    return np.uint32(b & 0xFFFFFFFF).view(np.float32)


def derive(x):
    """logistic_array's instruction sequence, each step exact then rounded once."""
    x = np.float32(x)
    if math.isnan(x):
        return np.float32("nan")
    t = np.float32(-x) if math.isinf(x) else f32(0 - Q(x))
    if t >= MAX_EXP:
        t = MAX_EXP
    if t <= MIN_EXP:
        t = MIN_EXP
    t = f32(Q(L2E) * Q(t))
    i = math.floor(Q(t))
    f = f32(Q(t) - i)
    p = f32(Q(f) * Q(C2) + Q(C1))
    p = f32(Q(p) * Q(f) + Q(C0))
    e = from_bits(bits(p) + (i << 23))
    d = f32(Q(e) + 1)
    return f32(1 / Q(d))


def test_f32_rounding_helper():
    """The rounding helper against float32 conversions and hand cases."""
    for q in (Fr(1, 3), Fr(-2, 7), Fr(10 ** 20, 3), Fr(1, 10 ** 40), Fr(7, 2 ** 150)):
        assert bits(f32(q)) == bits(np.float32(float(q)))
    assert f32(1 + Fr(1, 2 ** 24)) == np.float32(1.0)  # tie -> even
    assert bits(f32(1 + Fr(3, 2 ** 24))) == bits(np.float32(1)) + 2  # tie at 1.5 ulp -> even (2 ulp)
    assert f32(Fr(2) ** 128) == np.float32(np.inf)
    assert bits(f32(Fr(1, 2 ** 149))) == 1  # smallest subnormal


def test_derivation_reproduces_the_table():
    for xb, yb in TABLE:
        assert bits(derive(from_bits(xb))) == yb, hex(xb)


def test_oracle_matches_the_table_bit_for_bit():
    x = np.array([from_bits(xb) for xb, _ in TABLE], np.float32)
    y = R.activate(x.copy(), 0, exact=True)
    assert [bits(v) for v in y] == [yb for _, yb in TABLE]
    nan = R.activate(np.array([np.nan], np.float32), 0, exact=True)
    assert np.isnan(nan[0])


def test_hand_derived_cases():
    """x = 0: t = 0, f = 0, so p = c0 and y = 1/(1 + c0) (a true sigmoid gives
    0.5).  t with fraction 1/2: p = fl(fl(c1 + c2/2)/2 + c0) (halving is
    exact), e = p * 2^floor(t).  The clamps: x <= -88.72283 gives t = MAX_EXP,
    x >= 87.33654 gives t = MIN_EXP."""
    table = dict(TABLE)
    y0 = f32(1 / Q(f32(1 + Q(C0))))
    assert table[0x00000000] == table[0x80000000] == bits(y0) != bits(np.float32(0.5))
    p_half = f32(Q(f32(Q(C1) + Q(C2) / 2)) / 2 + Q(C0))
    for xb, t in HALF_POINTS.items():
        x = from_bits(xb)
        assert f32(Q(L2E) * Q(f32(0 - Q(x)))) == np.float32(t)  # the table's x really gives this t
        e = Q(p_half) * Fr(2) ** math.floor(t)
        assert table[xb] == bits(f32(1 / Q(f32(e + 1))))
    assert table[0xc2c80000] == table[0xc2b17217] == table[0xff800000]   # clamped at MAX_EXP
    assert table[0x42c80000] == table[0x42aeac4f] == table[0x7f800000] == bits(np.float32(1))


def test_true_sigmoid_fails_the_table():
    """A plain 1/(1 + exp(-x)) (correctly rounded) disagrees with the reference
    polynomial on every point where it is not saturated at 1."""
    differs = 0
    for xb, yb in TABLE:
        x = float(from_bits(xb))
        sig = np.float32(1.0 / (1.0 + math.exp(-x))) if x > -700 else np.float32(0.0)
        if bits(sig) != yb:
            differs += 1
        else:
            assert yb == bits(np.float32(1.0)), hex(xb)
    assert differs >= 20
