"""Darknet ``.weights`` files: read, write, and fold batch norm into the convs.

Format (TDarknetParser.loadWeights, nparser.pas:1275-1320; the field order of
each convolution from loadConvolutionalWeights, nparser.pas:1140-1170):

  header   int32 major, int32 minor, int32 revision, then ``seen``:
           uint64 when major*10 + minor >= 2, else uint32
  per convolutional layer, in layer order, little-endian float32:
           biases[F]
           if batch_normalize: scales[F], rolling_mean[F], rolling_variance[F]
           weights[F * C * k * k]   (filter-major [F][C][ky][kx])

Layers without parameters (shortcut, route, upsample, yolo, maxpool) store
nothing.  A file that ends before the last convolution's blob raises
ValueError naming the layer (the reference prints a warning and keeps
whatever it read).  Weighted shortcut layers are not part of the supported
layer set and are rejected by the cfg parser's shapes.

``fold_bn`` is TBaseConvolutionalLayer.fuseBatchNorm (nConvolutionLayer.pas:
104-128) in the same float32 operation order:
  pre = scale / sqrt(max(var, 1e-6));  bias = bias - mean * pre;  W = W * pre
"""
from __future__ import annotations

import struct

import numpy as np

EPSILON = np.float32(1e-6)  # sEPSILON, ntensors.pas:95


def _seen_is_64(major, minor):
    return major * 10 + minor >= 2


def conv_blobs(L):
    """(name, count) of the float32 blobs of conv layer L, in file order."""
    F = L["filters"]
    K = L["in"][0] * L["size"] * L["size"]
    blobs = [("biases", F)]
    if L.get("bn"):
        blobs += [("scales", F), ("rolling_mean", F), ("rolling_variance", F)]
    blobs.append(("weights", F * K))
    return blobs


def read_weights(path, layers):
    """Returns (header, params): header = dict(major, minor, revision, seen);
    params[i] = dict of float32 arrays (biases, [scales, rolling_mean,
    rolling_variance,] weights [F, C*k*k]) for every convolutional layer i."""
    with open(path, "rb") as f:
        raw = f.read(12)
        if len(raw) < 12:
            raise ValueError(f"{path}: truncated header")
        major, minor, revision = struct.unpack("<iii", raw)
        wide = _seen_is_64(major, minor)
        raw = f.read(8 if wide else 4)
        if len(raw) < (8 if wide else 4):
            raise ValueError(f"{path}: truncated header")
        seen = struct.unpack("<Q" if wide else "<I", raw)[0]
        params = {}
        for L in layers:
            if L["type"] != "convolutional":
                continue
            p = {}
            for name, n in conv_blobs(L):
                a = np.fromfile(f, dtype="<f4", count=n)
                if a.size < n:
                    raise ValueError(f"{path}: file ends inside layer {L['index']} ({name}: {a.size} of {n} floats)")
                p[name] = a.astype(np.float32, copy=False)
            p["weights"] = p["weights"].reshape(L["filters"], -1)
            params[L["index"]] = p
        rest = f.read(1)
    header = dict(major=major, minor=minor, revision=revision, seen=seen, trailing_bytes=len(rest) > 0)
    return header, params


def write_weights(path, layers, params, major=0, minor=2, revision=0, seen=0):
    """Writes params (as returned by read_weights) in the darknet format."""
    with open(path, "wb") as f:
        f.write(struct.pack("<iii", major, minor, revision))
        f.write(struct.pack("<Q" if _seen_is_64(major, minor) else "<I", seen))
        for L in layers:
            if L["type"] != "convolutional":
                continue
            p = params[L["index"]]
            for name, n in conv_blobs(L):
                a = np.ascontiguousarray(p[name], dtype="<f4").reshape(-1)
                if a.size != n:
                    raise ValueError(f"layer {L['index']} {name}: {a.size} floats, expected {n}")
                a.tofile(f)


def fold_bn(weights, biases, scales, mean, var):
    """fuseBatchNorm in float32: returns (W', b') with W' = W * pre and
    b' = b - mean * pre, pre = scale / sqrt(max(var, 1e-6)) per filter."""
    W = np.asarray(weights, np.float32)
    F = W.shape[0]
    v = np.asarray(var, np.float32)
    v = np.where(v > EPSILON, v, EPSILON)  # max(v, eps); a NaN variance takes eps, as Pascal's max does
    pre = (np.asarray(scales, np.float32) / np.sqrt(v)).astype(np.float32)
    b = (np.asarray(biases, np.float32) - np.asarray(mean, np.float32) * pre).astype(np.float32)
    Wf = (W.reshape(F, -1) * pre[:, None]).astype(np.float32).reshape(W.shape)
    return Wf, b


def load_weights(path, layers):
    """Reads a .weights file and returns {conv index: (W [F, C*k*k], bias [F])}
    with batch norm folded, the input of darknet.Network."""
    _, params = read_weights(path, layers)
    out = {}
    for i, p in params.items():
        if "scales" in p:
            out[i] = fold_bn(p["weights"], p["biases"], p["scales"], p["rolling_mean"], p["rolling_variance"])
        else:
            out[i] = (p["weights"], p["biases"])
    return out
