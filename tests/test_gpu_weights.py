"""A network loaded from a darknet .weights file (batch norm folded on the
host by tensorium_amd.weights) runs on the GPU and matches the oracle fed the
same file's parameters folded by the oracle's fuseBatchNorm restatement."""
import numpy as np
import pytest
import torch

from oracle import netref
from oracle import refcpu as R
from tensorium_amd import darknet, synth, weights as WT

pytestmark = pytest.mark.gpu

CFG = """[net]
height=26
width=26
channels=16
[convolutional]
batch_normalize=1
filters=32
size=3
stride=1
pad=1
activation=leaky
[convolutional]
batch_normalize=1
filters=32
size=1
stride=1
pad=1
activation=leaky
[shortcut]
from=-2
activation=linear
[convolutional]
batch_normalize=1
filters=64
size=3
stride=2
pad=1
activation=leaky
[convolutional]
filters=255
size=1
stride=1
pad=1
activation=linear
[yolo]
mask=0,1,2
anchors=10,13, 16,30, 33,23
classes=80
num=3
"""


def test_network_from_weights_file(hip, tmp_path):
    print("[case] network from a .weights file (BN folded on the host) vs oracle", flush=True)
    _, layers = darknet.parse_cfg(CFG)
    rng = np.random.default_rng(5)
    params = {}
    for L in layers:
        if L["type"] != "convolutional":
            continue
        fan = L["in"][0] * L["size"] ** 2
        p = {"biases": rng.normal(0, 0.1, L["filters"]).astype(np.float32),
             "weights": rng.normal(0, (2.0 / fan) ** 0.5, (L["filters"], fan)).astype(np.float32)}
        if L["bn"]:
            p["scales"] = rng.uniform(0.5, 1.5, L["filters"]).astype(np.float32)
            p["rolling_mean"] = rng.normal(0, 0.2, L["filters"]).astype(np.float32)
            p["rolling_variance"] = rng.uniform(0.3, 2.0, L["filters"]).astype(np.float32)
        params[L["index"]] = p
    path = tmp_path / "net.weights"
    WT.write_weights(path, layers, params, seen=640)
    loaded = WT.load_weights(path, layers)
    ref_w = {}
    for i, p in params.items():
        ref_w[i] = R.fuse_bn(p["weights"], p["biases"], p["scales"], p["rolling_mean"], p["rolling_variance"]) \
            if "scales" in p else (p["weights"], p["biases"])
    x = synth.uniform(71, (2, 16, 26, 26))
    ref = netref.forward(layers, ref_w, x)
    net = darknet.Network(hip, layers, 2, loaded)
    dx = torch.from_numpy(x).cuda()
    torch.cuda.synchronize()
    net.forward(dx)
    hip.finish()
    head = len(layers) - 2  # the linear 255-filter conv feeding the yolo layer
    assert R.rel_err(net.out[head].numpy(), ref[head]) <= 1e-5
