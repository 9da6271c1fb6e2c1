"""nnhip.DeviceArray's views on the CPU: the byte offset and shape of each
block a[key] selects, against numpy's view of the same key on an index
array (no device memory is touched: the arrays wrap a made-up address)."""
import itertools

import numpy as np
import pytest

from tensorium_amd.nnhip import DeviceArray

BASE = 1 << 20


def fake(shape, dtype=np.float32):
    return DeviceArray(shape, dtype, None, BASE)


def numpy_block(shape, key):
    """(first element, shape) of numpy's view, or None when numpy's view is
    not one contiguous block."""
    v = np.arange(int(np.prod(shape))).reshape(shape)[key]
    if v.size == 0:
        return None
    flat = v.reshape(-1)
    if not np.array_equal(flat, np.arange(flat[0], flat[0] + flat.size)):
        return None
    return int(flat[0]), v.shape


def keys(shape):
    opts = []
    for n in shape:
        opts.append([slice(None), 0, n - 1, slice(1, n), slice(0, 1), slice(0, max(n - 1, 1))])
    for k in range(1, len(shape) + 1):
        yield from itertools.product(*opts[:k])


@pytest.mark.parametrize("shape", [(7,), (4, 3), (1, 8, 3, 3), (2, 3, 4, 5), (5, 1, 4)])
def test_views_match_numpy(shape):
    a = fake(shape)
    for key in keys(shape):
        want = numpy_block(shape, key)
        if want is None:
            v = np.arange(int(np.prod(shape))).reshape(shape)[key]
            if v.size == 0:
                continue
            with pytest.raises(TypeError, match="contiguous"):
                a[key]
            continue
        first, sh = want
        got = a[key]
        assert got.shape == sh, (key, got.shape, sh)
        assert got.ptr == BASE + 4 * first, key
        assert got.numel() == int(np.prod(sh))


def test_view_reshape_and_int64():
    a = fake((4, 6), np.int64)
    b = a[1:3].view(3, 4)
    assert b.shape == (3, 4) and b.ptr == BASE + 8 * 6
    with pytest.raises(ValueError):
        a.view(5, 5)
    with pytest.raises(IndexError):
        a[4]
    with pytest.raises(TypeError):
        a[::2]
