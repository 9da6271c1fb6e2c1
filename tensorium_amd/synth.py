"""Seeded synthetic inputs shared by the GPU runs and the CPU oracle.

One 64-bit seed per (config, tensor).  Generator: splitmix64, counter form
(the i-th output of a stream seeded with s is mix(s + (i+1)*0x9E3779B97F4A7C15)).
  U[0,1)   = (x >> 40) * 2^-24                      (exactly representable fp32)
  U[a,b)   = a + (b - a)*u, computed in fp32
  N(0, s)  = Box-Muller in float64 on pairs (u1, u2) of 53-bit uniforms,
             z0 = sqrt(-2 ln(1-u1)) cos(2 pi u2), z1 = ... sin(...),
             scaled by s and rounded to fp32.
The same bytes are handed to the GPU and to the CPU oracle, so inputs are
identical by construction.
"""
import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def splitmix64(seed, n):
    """First n outputs of splitmix64 seeded with `seed` (uint64 array)."""
    with np.errstate(over="ignore"):
        z = np.uint64(seed) + (np.arange(1, n + 1, dtype=np.uint64) * _GOLDEN)
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def uniform(seed, shape, a=0.0, b=1.0):
    n = int(np.prod(shape))
    u = (splitmix64(seed, n) >> np.uint64(40)).astype(np.float32) * np.float32(2.0 ** -24)
    if a == 0.0 and b == 1.0:
        return u.reshape(shape)
    return (np.float32(a) + np.float32(b - a) * u).astype(np.float32).reshape(shape)


def normal(seed, shape, sigma=1.0):
    n = int(np.prod(shape))
    m = (n + 1) // 2
    x = splitmix64(seed, 2 * m)
    u = (x >> np.uint64(11)).astype(np.float64) * 2.0 ** -53
    u1, u2 = u[0::2], u[1::2]
    r = np.sqrt(-2.0 * np.log(1.0 - u1))
    z = np.empty(2 * m, dtype=np.float64)
    z[0::2] = r * np.cos(2.0 * np.pi * u2)
    z[1::2] = r * np.sin(2.0 * np.pi * u2)
    return (z[:n] * sigma).astype(np.float32).reshape(shape)
