"""tnh_conv2d_fwd_nhwc_noalloc (the channels-last convolution for callers that
cannot allocate device memory) against tnh_conv2d_fwd_nhwc through the C ABI:
bit-identical outputs on two calls in a row, the second with a smaller
input (the static scratch still holds the first call's pieces), with the
tiling the allocating entry point tuned and with forced tail-split and
split-K tilings (the ones that use the scratch); a forced tiling that needs
more scratch than the array holds is refused without a launch, while a tuned
one gives way to the cost model's tiling; the calls leave the device's free
memory unchanged.  Both are also checked against the CPU
oracle (per-tensor 1e-5)."""
import numpy as np
import pytest
import torch

from oracle import refcpu as R
from tensorium_amd import synth
from tensorium_amd.nnhip import CONV_SPLIT_UNIT, CONV_TAIL_BASE, TNHError, acLEAKY

pytestmark = pytest.mark.gpu
TOL = 1e-5
LEAN_128x64 = 13  # tnh_conv2d_set_autotune tile id of the 128x64x32 lean tile
LEAN_128x128 = 14


def case(msg):
    print(f"[case] {msg}", flush=True)


def nhwc(a):
    return np.ascontiguousarray(a.transpose(0, 2, 3, 1))


class Layer:
    """One 3x3 conv + bias + leaky + residual layer on seeded data."""

    def __init__(self, B, C, Hh, F, seed):
        self.B, self.C, self.H, self.F = B, C, Hh, F
        x = synth.uniform(seed, (B, C, Hh, Hh))
        w = synth.normal(seed + 1, (F, C * 9), (2.0 / (C * 9)) ** 0.5)
        b = synth.normal(seed + 2, (F,), 0.1)
        r = synth.uniform(seed + 3, (B, F, Hh, Hh), -1, 1)
        ref = R.conv_forward(x, w, b, 3, 1, 1, acLEAKY)
        self.ref = nhwc(ref + r)
        tap = np.ascontiguousarray(w.reshape(F, C, 3, 3).transpose(0, 2, 3, 1).reshape(F, 9 * C))
        self.dx, self.dw, self.db, self.dr = (torch.from_numpy(a).cuda() for a in (nhwc(x), tap, b, nhwc(r)))
        torch.cuda.synchronize()

    def run(self, hip, noAlloc, out=None):
        if out is None:
            out = torch.full((self.B, self.H, self.H, self.F), 7.0, dtype=torch.float32, device="cuda")
            torch.cuda.synchronize()
        hip.conv2dForwardNHWC(self.B, self.C, self.H, self.H, self.F, 3, 1, 1, self.dx, 0, self.dw, self.db, acLEAKY,
                              out, 0, residual=self.dr, noAlloc=noAlloc)
        hip.finish()
        return out


@pytest.fixture
def restore_autotune(hip):
    yield
    hip.setConvAutotune(True, -1)


# forced tilings that put K pieces in the scratch: tail split of the 128x64
# tile into 4 pieces (rounds of one tile per CU), and split-K into 3 pieces
# (every tile cut) of the 128x128 tile; -1: the tiling the allocating entry
# point tunes for the shape
@pytest.mark.parametrize("forced", [-1, LEAN_128x64 + CONV_SPLIT_UNIT * (CONV_TAIL_BASE + 4),
                                    LEAN_128x128 + CONV_SPLIT_UNIT * 3])
def test_noalloc_equals_allocating_entry_point(hip, restore_autotune, forced):
    big = Layer(4, 64, 52, 128, 501)
    small = Layer(1, 64, 26, 128, 601)
    hip.setConvAutotune(True, forced)
    case(f"conv nhwc noalloc forced={forced}: allocating entry point, big then small")
    want_big = big.run(hip, False).cpu().numpy()
    want_small = small.run(hip, False).cpu().numpy()
    case(f"conv nhwc noalloc forced={forced}: no-alloc entry point, big then small")
    got_big = big.run(hip, True).cpu().numpy()
    got_small = small.run(hip, True).cpu().numpy()
    assert np.array_equal(got_big, want_big)
    assert np.array_equal(got_small, want_small)
    assert R.rel_err(got_big, big.ref) <= TOL
    assert R.rel_err(got_small, small.ref) <= TOL


def test_noalloc_untuned_shape_and_free_memory(hip, restore_autotune):
    """A shape the allocating entry point never saw (cost-model tiling), after
    a warm-up call: the free device memory is the same before and after."""
    warm = Layer(1, 32, 20, 64, 701)
    fresh = Layer(3, 96, 38, 192, 801)
    hip.setConvAutotune(True, -1)
    case("conv nhwc noalloc: warm-up call")
    warm.run(hip, True)
    out = torch.full((3, 38, 38, 192), 7.0, dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    free0, _ = torch.cuda.mem_get_info()
    case("conv nhwc noalloc: untuned shape")
    fresh.run(hip, True, out)
    free1, _ = torch.cuda.mem_get_info()
    assert free1 == free0
    assert R.rel_err(out.cpu().numpy(), fresh.ref) <= TOL


def test_noalloc_refuses_a_tiling_beyond_the_scratch(hip, restore_autotune):
    """Split-K into 8 pieces of every 128x128 tile of an 8 x 52 x 52 x 256
    layer needs 338 tiles x 8 pieces x 64 KiB = 177 MB of pieces: refused
    before any launch (the output keeps its fill)."""
    from tensorium_amd.nnhip import TNHError as E

    assert hip.noAllocScratchBytes() == 64 << 20
    L = Layer(8, 256, 52, 256, 901)
    hip.setConvAutotune(True, LEAN_128x128 + CONV_SPLIT_UNIT * 8)
    out = torch.full((8, 52, 52, 256), 7.0, dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    case("conv nhwc noalloc: tiling beyond the static scratch")
    with pytest.raises(E, match="scratch"):
        L.run(hip, True, out)
    assert bool((out == 7.0).all())
    # the allocating entry point runs the same tiling
    L.run(hip, False, out)
    assert R.rel_err(out.cpu().numpy(), L.ref) <= TOL
    assert E is TNHError


def test_noalloc_after_tuning_never_refuses(hip, restore_autotune):
    """A layer whose timed tuning may choose split pieces larger than the
    static scratch (8 x 52 x 52 x 256, 3x3 over 256 channels: split-K into 4
    pieces of every 128x128 tile would need 88 MB): after the allocating
    entry point tuned it, the no-alloc call runs without an error, on two
    calls in a row, the second with a smaller batch.  Its output equals the
    allocating entry point's bit for bit when the tuned pieces fit the
    scratch; otherwise it runs the cost model's tiling (whole K if need be)
    and stays within the oracle's bound."""
    L = Layer(8, 256, 52, 256, 911)
    S = Layer(2, 256, 52, 256, 921)
    hip.setConvAutotune(True, -1)
    case("conv nhwc noalloc after tuning: allocating entry point (tunes)")
    want = L.run(hip, False).cpu().numpy()
    want_s = S.run(hip, False).cpu().numpy()
    case("conv nhwc noalloc after tuning: no-alloc entry point, big then small")
    got = L.run(hip, True).cpu().numpy()
    got_s = S.run(hip, True).cpu().numpy()
    print(f"noalloc after tuning: equal to the allocating call: {np.array_equal(got, want)} (8 images), "
          f"{np.array_equal(got_s, want_s)} (2 images)", flush=True)
    assert R.rel_err(got, L.ref) <= TOL
    assert R.rel_err(got_s, S.ref) <= TOL
    assert R.rel_err(want, L.ref) <= TOL
