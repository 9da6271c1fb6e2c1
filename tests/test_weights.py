"""Darknet .weights reader/writer and the batch-norm fold (CPU).

Pins: a hand-packed byte fixture fixes the field order (header, 32- vs 64-bit
`seen`, biases / scales / rolling mean / rolling variance / weights per conv,
nothing for parameter-free layers); write -> read is the identity; a truncated
file raises; the product's float32 fold equals the oracle's restatement of
fuseBatchNorm (nConvolutionLayer.pas:104-128) bit for bit, and a folded conv
equals the unfolded conv + BN normalize of the oracle within the conv bound."""
import struct

import numpy as np
import pytest

from oracle import refcpu as R
from tensorium_amd import darknet, synth, weights as WT

CFG = """[net]
height=8
width=8
channels=2
[convolutional]
batch_normalize=1
filters=3
size=3
stride=1
pad=1
activation=leaky
[convolutional]
filters=3
size=1
stride=1
pad=1
activation=linear
[shortcut]
from=-2
activation=linear
"""


def tiny():
    _, layers = darknet.parse_cfg(CFG)
    return layers


def test_byte_layout_fixture(tmp_path):
    layers = tiny()
    # conv 0: F=3, C=2, k=3 (K=18), BN; conv 1: F=3, C=3, k=1 (K=3), no BN
    vals = np.arange(3 + 3 * 3 + 3 * 18 + 3 + 3 * 3, dtype=np.float32) * 0.5 - 7
    p = tmp_path / "t.weights"
    p.write_bytes(struct.pack("<iiiQ", 0, 2, 5, 123456789012) + vals.astype("<f4").tobytes())
    hdr, params = WT.read_weights(p, layers)
    assert (hdr["major"], hdr["minor"], hdr["revision"], hdr["seen"]) == (0, 2, 5, 123456789012)
    assert not hdr["trailing_bytes"]
    o = 0
    for name, n in (("biases", 3), ("scales", 3), ("rolling_mean", 3), ("rolling_variance", 3), ("weights", 54)):
        assert np.array_equal(params[0][name].ravel(), vals[o:o + n]), name
        o += n
    assert params[0]["weights"].shape == (3, 18)
    assert set(params[1]) == {"biases", "weights"}
    assert np.array_equal(params[1]["biases"], vals[o:o + 3])
    assert np.array_equal(params[1]["weights"].ravel(), vals[o + 3:o + 12])
    assert 2 not in params  # the shortcut stores nothing


def test_seen_width_follows_version(tmp_path):
    layers = tiny()
    n = 3 * 4 + 54 + 3 + 9
    body = np.zeros(n, "<f4").tobytes()
    p = tmp_path / "old.weights"
    p.write_bytes(struct.pack("<iiiI", 0, 1, 0, 77) + body)  # major*10+minor = 1 < 2: 32-bit seen
    hdr, _ = WT.read_weights(p, layers)
    assert hdr["seen"] == 77 and not hdr["trailing_bytes"]


def test_round_trip_and_truncation(tmp_path):
    layers = tiny()
    rng = np.random.default_rng(3)
    params = {}
    for L in layers:
        if L["type"] == "convolutional":
            params[L["index"]] = {name: rng.standard_normal(n).astype(np.float32) for name, n in WT.conv_blobs(L)}
    p = tmp_path / "rt.weights"
    WT.write_weights(p, layers, params, major=0, minor=2, revision=7, seen=42)
    hdr, back = WT.read_weights(p, layers)
    assert hdr["seen"] == 42 and hdr["revision"] == 7
    for i, blob in params.items():
        for name, a in blob.items():
            assert np.array_equal(back[i][name].ravel(), a), (i, name)
    data = p.read_bytes()
    (tmp_path / "cut.weights").write_bytes(data[:-8])
    with pytest.raises(ValueError, match="layer 1"):
        WT.read_weights(tmp_path / "cut.weights", layers)


def test_fold_equals_oracle_bit_exact():
    rng = np.random.default_rng(11)
    F, K = 37, 75
    W = rng.standard_normal((F, K)).astype(np.float32)
    b = rng.standard_normal(F).astype(np.float32)
    s = rng.uniform(0.5, 2, F).astype(np.float32)
    m = rng.standard_normal(F).astype(np.float32)
    v = rng.uniform(0, 3, F).astype(np.float32)
    v[:3] = [0.0, 1e-9, np.nan]  # below the 1e-6 floor, and NaN (max() picks the floor)
    Wf, bf = WT.fold_bn(W, b, s, m, v)
    Wr, br = R.fuse_bn(W, b, s, m, v)
    assert np.array_equal(Wf.view(np.uint32), Wr.view(np.uint32))
    assert np.array_equal(bf.view(np.uint32), br.view(np.uint32))
    # closed form of the floor: var 0 and 1e-9 divide by sqrt(1e-6) = 1e-3
    assert np.array_equal(Wf[0], (W[0] * (s[0] / np.float32(1e-3))).astype(np.float32))


def test_folded_conv_matches_conv_plus_bn():
    """fold(W, BN) applied as one conv equals conv then the BN affine map
    (exact-mode normalize) within the conv bound: the fold is the right
    algebra, not only the right float ops."""
    x = synth.uniform(61, (2, 4, 9, 9))
    W = synth.normal(62, (6, 36), 0.2)
    b = synth.normal(63, (6,), 0.1)
    s = synth.uniform(64, (6,), 0.5, 1.5)
    m = synth.normal(65, (6,), 0.1)
    v = synth.uniform(66, (6,), 0.2, 2.0)
    Wf, bf = WT.fold_bn(W, b, s, m, v)
    got = R.conv_forward(x, Wf, bf, 3, 1, 1, 4)  # linear activation
    y = R.conv_forward(x, W, np.zeros(6, np.float32), 3, 1, 1, 4).astype(np.float64)
    ref = (y - m[None, :, None, None]) / np.sqrt(np.maximum(v, 1e-6))[None, :, None, None] * s[None, :, None, None] \
        + b[None, :, None, None]
    assert R.rel_err(got, ref) <= 1e-5


def test_yolov3_blob_count_matches_published_file_size():
    """The darknet yolov3.weights file is 248 007 048 bytes: a 20-byte header
    (0, 2, 0, 64-bit seen) and 62 001 757 floats.  Our cfg and the blob
    layout must add up to exactly that."""
    _, layers = darknet.load_cfg("yolov3.cfg")
    n = sum(c for L in layers if L["type"] == "convolutional" for _, c in WT.conv_blobs(L))
    assert n == 62001757
    assert 12 + 8 + 4 * n == 248007048
