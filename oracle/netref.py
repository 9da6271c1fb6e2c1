"""CPU forward of a parsed darknet network through the oracle (TEST
INFRASTRUCTURE ONLY: parity tests and the cpu_baseline leg of bench.py).

Runs the reference layer semantics one layer at a time: conv (Conv2D + bias +
activation), shortcut (addvv + linear), route (per-image concat, or the
reference's whole-tensor concat), upsample, maxpool, yolo (copy + logistic,
exact reciprocal, then scale_x_y's x*s + (1-s)/2 on x and y).  Returns every layer's output."""
import numpy as np

from oracle import refcpu as R


def forward(layers, weights, x, route_mode="image"):
    outs = []
    prev = x
    B = x.shape[0]
    for L in layers:
        t = L["type"]
        if t == "convolutional":
            w, b = weights[L["index"]]
            y = R.conv_forward(prev, w, b, L["size"], L["stride"], L["pad"], L["act"])
        elif t == "shortcut":
            y = R.addvv(prev, outs[L["src"]]).reshape(prev.shape)
            R.activate(y, L["act"])
        elif t == "route":
            srcs = [outs[s] for s in L["srcs"]]
            if len(srcs) == 1:
                y = srcs[0]
            elif route_mode == "image":
                y = np.concatenate(srcs, axis=1)
            else:
                y = np.concatenate([s.ravel() for s in srcs]).reshape((B,) + L["out"])
        elif t == "upsample":
            y = R.upsample_fwd(prev, L["stride"], L["scale"])
        elif t == "maxpool" and L.get("depth"):
            y, _ = R.maxpool_depth_fwd(prev, L["out"][0], with_idx=False)
        elif t == "maxpool":
            y, _ = R.maxpool_fwd(prev, L["size"], L["stride"], L["stride"], L["pad"], with_idx=False)
        elif t == "yolo":
            y = R.yolo_fwd(prev, L["n"], L["classes"], exact=True)
            s = np.float32(L.get("scale_xy", 1.0))
            if s != 1:  # output.FusedMultiplyAdd on x, y (nyololayer.pas:822-823)
                v = y.reshape(B, L["n"], L["classes"] + 5, -1)
                v[:, :, :2] = (v[:, :, :2] * s).astype(np.float32) + np.float32(0.5) * (np.float32(1) - s)
        else:
            raise ValueError(t)
        outs.append(y)
        prev = y
    return outs
