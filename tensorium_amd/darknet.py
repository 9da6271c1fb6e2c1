"""Darknet cfg parsing and a device-resident network runner.

``parse_cfg`` reads a darknet .cfg (the format TDarknetParser consumes,
nparser.pas:782-940; INI sections as in nconfig.pas:15-45) into layer specs
with their shapes resolved.  ``Network`` plays the role of TNNet.forward
(nnet.pas:275-317) for inference on one GPU: every layer's output lives in
HBM and each layer is one or two launches through the C ABI.

Fusions (results bit-identical to the unfused layer sequence):
  * a convolution whose only consumer is the next layer, a ``[shortcut]``
    with linear activation, writes ``act(conv + bias) + other`` straight into
    the shortcut's buffer (the separate add of naddlayer.pas:698);
  * a single-input ``[route]`` is an alias of its input (no copy);
  * at batch 1 (NCHW) a multi-input route's inputs are written by their
    producers straight into their channel slices of the route buffer.

Route concat of several inputs is per image (darknet semantics).  The
reference's TConcatLayer copies whole batched tensors back to back
(nconcatlayer.pas:115 -> ntensors.pas:12045), which mixes images at batch > 1;
``route_mode="reference"`` reproduces that layout for parity studies.

``layout="nhwc"`` keeps every activation channels-last between layers (the
input image stays NCHW and the yolo heads are written NCHW, so the
network's interface does not change): both GEMM operands of a convolution
then load 16 bytes along K, and a route's inputs are written straight into
their channel slice of the route buffer (no concat copy).
"""
from __future__ import annotations

import math
import os

import numpy as np

from . import synth
from .nnhip import WEIGHTS_REFERENCE, WEIGHTS_TAP_MAJOR, DeviceArray, acLEAKY, acLINEAR, acLOGISTIC, release_stream

CFG_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cfg")
_ACT = {"leaky": acLEAKY, "linear": acLINEAR, "logistic": acLOGISTIC}


def read_sections(text):
    """[name] key=value sections, '#'/';' comments (nconfig.pas:15-45)."""
    secs = []
    for raw in text.splitlines():
        line = raw.split("#", 1)[0].split(";", 1)[0].strip()
        if not line:
            continue
        if line.startswith("["):
            secs.append((line.strip("[]").strip().lower(), {}))
        elif "=" in line and secs:
            k, v = line.split("=", 1)
            secs[-1][1][k.strip()] = v.strip()
    return secs


def parse_cfg(text, height=None, width=None):
    """Returns (net_options, layers); layers carry resolved in/out shapes (C, H, W)."""
    secs = read_sections(text)
    if not secs or secs[0][0] not in ("net", "network"):
        raise ValueError("cfg must start with [net]")
    net = secs[0][1]
    H = int(height or net.get("height", 416))
    W = int(width or net.get("width", 416))
    Cin = int(net.get("channels", 3))
    layers = []
    shape = (Cin, H, W)
    for idx, (name, o) in enumerate(secs[1:]):
        L = {"type": name, "index": idx, "in": shape}
        if name == "convolutional":
            k = int(o.get("size", 1))
            s = int(o.get("stride", 1))
            pad = int(o.get("padding", 0))
            if int(o.get("pad", 0)):  # parseConvolutional: pad=1 -> size div 2 (nparser.pas:154)
                pad = k // 2
            F = int(o["filters"])
            C, h, w = shape
            oh = (h + 2 * pad - k) // s + 1
            ow = (w + 2 * pad - k) // s + 1
            L.update(filters=F, size=k, stride=s, pad=pad, act=_ACT[o.get("activation", "logistic")],
                     bn=int(o.get("batch_normalize", 0)), out=(F, oh, ow))
        elif name == "shortcut":
            frm = int(o["from"])
            src = idx + frm if frm < 0 else frm
            L.update(src=src, act=_ACT[o.get("activation", "linear")], out=shape)
            if layers[src]["out"] != shape:
                raise ValueError(f"shortcut {idx}: shape mismatch with layer {src}")
        elif name == "route":
            srcs = [int(v) for v in o["layers"].split(",")]
            srcs = [idx + v if v < 0 else v for v in srcs]
            shapes = [layers[v]["out"] for v in srcs]
            if any(sh[1:] != shapes[0][1:] for sh in shapes):
                raise ValueError(f"route {idx}: spatial size mismatch")
            L.update(srcs=srcs, out=(sum(sh[0] for sh in shapes),) + shapes[0][1:])
        elif name == "upsample":
            s = int(o.get("stride", 2))
            C, h, w = shape
            L.update(stride=s, scale=float(o.get("scale", 1)), out=(C, h * s, w * s))
        elif name == "maxpool":
            k = int(o.get("size", 1))
            s = int(o.get("stride", 1))
            pad = int(o.get("padding", k - 1))  # parseMaxPool default (nparser.pas:257)
            C, h, w = shape
            depth = int(o.get("maxpool_depth", 0))  # nparser.pas:258-259
            if depth:  # max over channel groups, the image size kept (nMaxPoolLayer.pas:98-102)
                L.update(size=k, stride=s, pad=pad, depth=True, out=(int(o.get("out_channels", 1)), h, w))
            else:
                L.update(size=k, stride=s, pad=pad, out=(C, (h + pad - k) // s + 1, (w + pad - k) // s + 1))
        elif name == "yolo":
            mask = [int(v) for v in o.get("mask", "0").split(",")]
            classes = int(o.get("classes", 80))
            if shape[0] != len(mask) * (classes + 5):
                raise ValueError(f"yolo {idx}: {shape[0]} channels != {len(mask)}*(classes+5)")
            # anchors (w, h pairs in network pixels; parseYolo, nparser.pas): default 0.5 as TYoloLayer's biases
            a = [float(v) for v in o["anchors"].split(",")] if "anchors" in o else [0.5] * (2 * (max(mask) + 1))
            if len(a) % 2 or max(mask) >= len(a) // 2:
                raise ValueError(f"yolo {idx}: mask {mask} needs {max(mask) + 1} anchors, cfg has {len(a) // 2}")
            if int(o.get("new_coords", 0)) != 0:
                raise ValueError(f"yolo {idx}: new_coords is not supported")
            # scale_x_y (parseYolo, nparser.pas:554): x, y = x*s + (1-s)/2 after the logistic
            L.update(n=len(mask), classes=classes, mask=mask, scale_xy=float(o.get("scale_x_y", 1)),
                     anchors=[(a[2 * m], a[2 * m + 1]) for m in mask], out=shape)
        else:
            raise ValueError(f"unsupported layer type [{name}]")
        layers.append(L)
        shape = L["out"]
    return net, layers


def load_cfg(name="yolov3.cfg", height=None, width=None):
    path = name if os.path.isabs(name) else os.path.join(CFG_DIR, name)
    with open(path) as f:
        return parse_cfg(f.read(), height, width)


def conv_flops(layers, batch=1):
    """2*M*N*K summed over convolutions (the metric's algorithmic FLOP)."""
    tot = 0
    for L in layers:
        if L["type"] == "convolutional":
            F, oh, ow = L["out"]
            tot += 2 * F * (L["in"][0] * L["size"] ** 2) * oh * ow * batch
    return tot


def synthetic_weights(layers, seed=0x5EED):
    """He-normal weights N(0, sqrt(2/fan_in)), one splitmix64 seed per layer;
    BN folded with its default init (scale 1, mean 0, var 1 -> /sqrt(1)) and
    biases 0, as the benchmark configuration specifies."""
    out = {}
    for L in layers:
        if L["type"] != "convolutional":
            continue
        F = L["filters"]
        fan_in = L["in"][0] * L["size"] ** 2
        w = synth.normal(seed + 1000 * L["index"] + 1, (F, fan_in), math.sqrt(2.0 / fan_in))
        out[L["index"]] = (w, np.zeros(F, np.float32))
    return out


def consumers(layers):
    use = {i: [] for i in range(len(layers))}
    for L in layers:
        i = L["index"]
        if L["type"] == "shortcut":
            use[i - 1].append(i)
            use[L["src"]].append(i)
        elif L["type"] == "route":
            for s in L["srcs"]:
                use[s].append(i)
        elif i > 0:
            use[i - 1].append(i)
    return use


# The largest tensor one kernel call addresses: the kernels reach their
# operands through buffer resources of at most this many bytes.
MAX_CALL_BYTES = 0x7FFFFFF0


def pass_batch(layers, batch, max_pass_batch=None):
    """Images per forward pass: the largest count whose every activation
    tensor (the input image, each layer's output, each route buffer) stays
    within MAX_CALL_BYTES, capped by `max_pass_batch`.  A batch above it runs
    as several passes over the same buffers."""
    per_image = 4 * max([int(np.prod(layers[0]["in"]))] + [int(np.prod(L["out"])) for L in layers])
    limit = max(1, MAX_CALL_BYTES // per_image)
    if max_pass_batch is not None:
        limit = min(limit, max(1, int(max_pass_batch)))
    return min(batch, limit)


class Network:
    """Inference runner over the C ABI.  Weights and activations live in
    DeviceArrays (the library's own allocator, tnh_malloc); the input may be
    any device buffer the entry points take (a DeviceArray or a torch tensor
    on the device, ready before forward() is called).

    A batch whose activations would exceed the 2 GiB a kernel call addresses
    runs as consecutive passes of pass_batch() images over buffers sized for
    one pass; the yolo outputs cover the whole batch.  `max_pass_batch`
    lowers the pass size."""

    def __init__(self, hip, layers, batch, weights, device="cuda", fuse=True, route_mode="image", pack=True,
                 layout="nchw", fuse_heads=True, max_pass_batch=None):
        # `device` names the context's GPU, the one tnh_init selected
        if layout not in ("nchw", "nhwc"):
            raise ValueError(f"layout {layout!r}")
        if route_mode not in ("image", "reference"):
            raise ValueError(f"route_mode {route_mode!r}")
        if layout == "nhwc" and route_mode != "image":
            # the whole-tensor concat is a layout of NCHW batches; the
            # channels-last planner writes route inputs into per-image
            # channel slices and has no equivalent
            raise NotImplementedError("route_mode='reference' needs layout='nchw'")
        self.full_batch = batch
        self.pass_batch = pass_batch(layers, batch, max_pass_batch)
        if self.pass_batch < batch and route_mode != "image":
            # the whole-tensor concat mixes images across the batch, so it
            # cannot be split into passes
            raise NotImplementedError(f"route_mode='reference' with a batch above {self.pass_batch} "
                                      "(2 GiB per kernel call)")
        batch = self.pass_batch  # buffers hold one pass
        self.hip, self.layers, self.batch = hip, layers, batch
        self.route_mode = route_mode
        self.layout = layout
        if layout == "nhwc":
            pack = True  # the channels-last kernels read tap-major weights
        use = consumers(layers)
        self.fused = set()  # conv indices whose shortcut is fused
        if fuse:
            for L in layers:
                i = L["index"]
                if (L["type"] == "convolutional" and i + 1 < len(layers) and layers[i + 1]["type"] == "shortcut"
                        and layers[i + 1]["act"] == acLINEAR and use[i] == [i + 1] and layers[i + 1]["src"] != i):
                    self.fused.add(i)
        # Weights go to HBM once; 3x3 filters are repacked tap-major
        # ([F][ky][kx][C]) on the device, the layout of the fast conv path.
        self.w = {}
        for i, (w, b) in weights.items():
            L = layers[i]
            dw = DeviceArray.from_numpy(np.ascontiguousarray(w, dtype=np.float32))
            wl = WEIGHTS_REFERENCE
            if pack and L["size"] > 1:
                packed = DeviceArray(dw.shape)
                hip.packConvWeights(L["filters"], L["in"][0], L["size"], dw, packed)
                hip.finish()
                dw, wl = packed, WEIGHTS_TAP_MAJOR
            self.w[i] = (dw, DeviceArray.from_numpy(np.ascontiguousarray(b, dtype=np.float32)), wl)
        self.out = [None] * len(layers)
        self.input_shape = (self.full_batch,) + layers[0]["in"]
        self.up_fused, self.yolo_fused = set(), set()
        if layout == "nhwc":
            if fuse and fuse_heads:
                # a convolution read only by an upsample stores its result
                # straight as the upsampled image; one read only by a yolo
                # layer also writes the yolo head (one launch each instead of
                # two)
                for L in layers:
                    i = L["index"]
                    if (L["type"] != "convolutional" or i in self.fused or i == 0 or i + 1 >= len(layers)
                            or use[i] != [i + 1]):
                        continue
                    nxt = layers[i + 1]["type"]
                    if nxt == "upsample":
                        self.up_fused.add(i)
                    elif nxt == "yolo":
                        self.yolo_fused.add(i)
            self._plan_nhwc(device)
            self._plan_branches(use)
            self._full_heads(device)
            return
        # At batch 1 a channel slice of an NCHW route buffer is contiguous, so
        # a route input's producer (convolution, shortcut or upsample) writes
        # straight into its slice and the route copies only the other inputs.
        placed = {}
        self.route_copies = {}
        if batch == 1 and route_mode == "image":
            for L in layers:
                if L["type"] == "route" and len(L["srcs"]) > 1:
                    C, h, w = L["out"]
                    buf = DeviceArray((1, C, h, w))
                    self.out[L["index"]] = buf
                    off, copies = 0, []
                    for s_ in L["srcs"]:
                        o = self._owner(s_)
                        cs = layers[s_]["out"][0]
                        if o not in placed and layers[o]["type"] in ("convolutional", "shortcut", "upsample"):
                            placed[o] = buf[:, off:off + cs]
                        else:
                            copies.append((s_, off))
                        off += cs
                    self.route_copies[L["index"]] = copies
        for L in layers:
            i = L["index"]
            if L["type"] == "route" and len(L["srcs"]) == 1:
                continue  # alias, resolved at run time
            if i in self.fused or self.out[i] is not None:
                continue  # writes into the shortcut's buffer / a route buffer
            C, h, w = L["out"]
            self.out[i] = placed[i] if i in placed else DeviceArray((batch, C, h, w))
        self._full_heads(device)

    def _full_heads(self, device):
        """Yolo outputs for the whole batch when it runs in several passes
        (each pass writes its images' slice); the batch size seen by the
        caller is the whole batch again."""
        if self.pass_batch < self.full_batch:
            for L in self.layers:
                if L["type"] == "yolo":
                    self.out[L["index"]] = DeviceArray((self.full_batch,) + L["out"])
        self.batch = self.full_batch

    # -- channels-last storage plan --------------------------------------------
    def _owner(self, i):
        """The layer whose storage holds layer i's output."""
        L = self.layers[i]
        if L["type"] == "route" and len(L["srcs"]) == 1:
            return self._owner(L["srcs"][0])
        if i in self.fused:
            return i + 1
        return i

    def _plan_nhwc(self, device):
        """store[i] = (tensor, channel offset, pixel stride) for every storage
        owner.  A multi-input route gets a [B, h, w, sum C] buffer and each
        input owner that is a convolution, shortcut or upsample not placed
        elsewhere writes straight into its channel slice; other inputs are
        copied (tnh_copy_channels).  Yolo outputs are NCHW head tensors."""
        layers, B = self.layers, self.batch
        L0 = layers[0]
        if L0["type"] != "convolutional" or L0["size"] != 3 or L0["in"][0] > 4:
            raise NotImplementedError("channels-last networks start with a 3x3 convolution on <= 4 channels")
        if any(L.get("depth") for L in layers):
            raise NotImplementedError("maxpool_depth needs layout='nchw'")
        self.store = {}
        self.copy_srcs = {}
        for L in layers:
            if L["type"] == "route" and len(L["srcs"]) > 1:
                C, h, w = L["out"]
                buf = DeviceArray((B, h, w, C))
                self.store[L["index"]] = (buf, 0, C)
                off, copies = 0, []
                for s_ in L["srcs"]:
                    o = self._owner(s_)
                    cs = layers[s_]["out"][0]
                    if o not in self.store and layers[o]["type"] in ("convolutional", "shortcut", "upsample",
                                                                      "maxpool"):
                        self.store[o] = (buf, off, C)
                    else:
                        copies.append((s_, off))
                    off += cs
                self.copy_srcs[L["index"]] = copies
        for L in layers:
            i, t = L["index"], L["type"]
            if t == "yolo":
                C, h, w = L["out"]
                self.out[i] = DeviceArray((B, C, h, w))
                continue
            if (t == "route" and len(L["srcs"]) == 1) or i in self.fused or i in self.store or i in self.up_fused:
                continue  # (an upsample-fused convolution stores only the upsample's output)
            C, h, w = L["out"]
            self.store[i] = (DeviceArray((B, h, w, C)), 0, C)
        for L in layers:  # nothing may read a yolo head as an activation
            srcs = L.get("srcs", []) + ([L["src"]] if "src" in L else [])
            if L["index"] > 0 and L["type"] != "route":
                srcs = srcs + [L["index"] - 1]
            for s_ in srcs:
                if layers[self._owner(s_)]["type"] == "yolo" and L["type"] != "route":
                    raise NotImplementedError(f"layer {L['index']} reads yolo layer {s_}")

    def _plan_branches(self, use):
        """Yolo head tails that can run beside the rest of the network: the
        convolutions ending in a yolo layer whose outputs feed only the next
        layer of the tail (YOLOv3: 80-82 and 92-94, while 83-91 and 95-106
        continue from layer 79 / 91).  A tail forks after the layer before it
        and joins at the end of the forward pass; the last yolo layer has
        nothing beside it and stays on the main stream."""
        layers = self.layers
        self.branches = {}  # first layer of a tail -> its yolo layer
        for L in layers:
            y = L["index"]
            if L["type"] != "yolo" or y + 1 >= len(layers):
                continue
            s_ = y
            while (s_ - 1 > 0 and layers[s_ - 1]["type"] == "convolutional" and use[s_ - 1] == [s_]
                   and s_ - 1 not in self.fused):
                s_ -= 1
            if s_ < y and all(c <= y for i in range(s_, y + 1) for c in use[i]):
                self.branches[s_] = y
        self._side = None
        self.use_branches = False

    def nhwc_store(self, i):
        """(tensor, channel offset, pixel stride) of layer i's output."""
        return self.store[self._owner(i)]

    def output(self, i):
        """Layer i's output copied to the host as a [B, C, h, w] numpy array
        (in NHWC mode: its channel slice of the channels-last storage,
        transposed).  Waits for the context stream."""
        if self.layers[i]["type"] == "yolo":
            return self.buffer(i).numpy()
        if self.pass_batch < self.full_batch:
            raise ValueError(f"the batch runs in passes of {self.pass_batch} images: only the yolo outputs "
                             "cover the whole batch")
        if self.layout == "nchw":
            return self.buffer(i).numpy()
        if i in self.up_fused:
            raise ValueError(f"layer {i} stores only its upsampled output (layer {i + 1})")
        t, off, pix = self.nhwc_store(i)
        C = self.layers[i]["out"][0]
        a = t.numpy().reshape(self.batch, t.shape[1], t.shape[2], pix)
        return np.ascontiguousarray(a[..., off:off + C].transpose(0, 3, 1, 2))

    def buffer(self, i):
        L = self.layers[i]
        if L["type"] == "route" and len(L["srcs"]) == 1:
            return self.buffer(L["srcs"][0])
        if i in self.fused:
            return self.out[i + 1]
        return self.out[i]

    def forward(self, x, on_layer=None, branches=None):
        """Runs every layer on the context stream; returns the yolo outputs.

        on_layer(i, begin): optional hook called before (begin=True) and after
        (begin=False) the launches of layer i (used to bracket them with
        events).  branches: run the yolo head tails on a second stream, forked
        and joined through events (channels-last networks; default:
        self.use_branches, which is off: in graph replays on ROCm 7.2 the
        cross-stream edges cost more than the overlap gains, 1.232 against
        1.188 ms at batch 1 and 8.86 against 8.80 ms at batch 16).  The
        first forward pass always runs on one stream (it tunes every shape
        alone on the GPU)."""
        if self.pass_batch < self.full_batch:
            return self._forward_passes(x, on_layer)
        hip = self.hip
        tails = getattr(self, "branches", {})
        if branches is None:
            branches = getattr(self, "use_branches", False) and on_layer is None
        if not getattr(self, "_tuned", False):
            branches = False
        self._tuned = True
        if branches and tails:
            return self._forward_branched(x, tails)
        prev = x
        heads = []
        for L in self.layers:
            i = L["index"]
            if on_layer:
                on_layer(i, True)
            prev = self._layer(L, prev, heads)
            if on_layer:
                on_layer(i, False)
        return heads

    def _forward_passes(self, x, on_layer):
        """forward() over a batch above pass_batch: consecutive passes over
        images [c0, c0 + c) through the one-pass buffers (a last, smaller
        pass uses their first c images), each yolo layer writing its slice of
        the whole-batch output."""
        ys = [L["index"] for L in self.layers if L["type"] == "yolo"]
        full = {y: self.out[y] for y in ys}
        try:
            for c0 in range(0, self.full_batch, self.pass_batch):
                c = min(self.pass_batch, self.full_batch - c0)
                self.batch = c
                for y in ys:
                    self.out[y] = full[y][c0:c0 + c]
                prev = x[c0:c0 + c]
                for L in self.layers:
                    if on_layer:
                        on_layer(L["index"], True)
                    prev = self._layer(L, prev, [])
                    if on_layer:
                        on_layer(L["index"], False)
        finally:
            self.batch = self.full_batch
            for y in ys:
                self.out[y] = full[y]
        self._tuned = True
        return [full[y] for y in ys]

    def _forward_branched(self, x, tails):
        """forward() with each yolo head tail on the side stream: the main
        stream records an event after the layer before the tail, the side
        stream waits for it and runs the tail, and the main stream waits for
        every tail's end event after the last layer (also under graph
        capture, where the events become the graph's edges)."""
        hip = self.hip
        if self._side is None:
            import weakref

            self._side = hip.streamCreate()  # default priority
            self._events = {s_: (hip.eventCreate(), hip.eventCreate()) for s_ in tails}
            weakref.finalize(self, release_stream, self._side, [e for pair in self._events.values() for e in pair])
        main = hip.stream
        side = self._side
        heads, joins = [], []
        prev = x
        skip = -1
        for L in self.layers:
            i = L["index"]
            if i <= skip:
                continue
            if i in tails:
                fork, join = self._events[i]
                hip.eventRecord(fork)
                hip.setStream(side)
                try:
                    hip.streamWaitEvent(fork)
                    for j in range(i, tails[i] + 1):
                        self._layer(self.layers[j], None, heads)
                    hip.eventRecord(join)
                finally:
                    hip.setStream(main)
                joins.append(join)
                skip = tails[i]
                continue
            prev = self._layer(L, prev, heads)
        for ev in joins:
            hip.streamWaitEvent(ev)
        return heads

    def _layer_nhwc(self, L, x, heads):
        hip, B = self.hip, self.batch
        i, t = L["index"], L["type"]
        if t == "convolutional":
            w, b, _ = self.w[i]
            C, h, ww = L["in"]
            if i == 0:
                src, soff, spix, nchw = x, 0, 0, True
            else:
                (src, soff, spix), nchw = self.nhwc_store(i - 1), False
            res, roff, rpix = None, 0, None
            if i in self.fused:
                res, roff, rpix = self.nhwc_store(self.layers[i + 1]["src"])
            if i in self.up_fused:
                up = self.layers[i + 1]
                dst, doff, dpix = self.nhwc_store(i + 1)
                hip.conv2dForwardNHWCUpsample(B, C, h, ww, L["filters"], L["size"], L["stride"], L["pad"], src, soff,
                                              w, b, L["act"], up["stride"], up["scale"], dst, doff, inPix=spix,
                                              outPix=dpix)
                return x
            dst, doff, dpix = self.nhwc_store(i)
            if i in self.yolo_fused:
                Y = self.layers[i + 1]
                hip.conv2dForwardNHWCYolo(B, C, h, ww, L["filters"], L["size"], L["stride"], L["pad"], src, soff, w,
                                          b, L["act"], dst, doff, Y["n"], Y["classes"], self.out[i + 1], inPix=spix,
                                          outPix=dpix)
                return x
            hip.conv2dForwardNHWC(B, C, h, ww, L["filters"], L["size"], L["stride"], L["pad"], src, soff, w, b,
                                  L["act"], dst, doff, inPix=spix, outPix=dpix, residual=res, resOffset=roff,
                                  resPix=rpix, nchwInput=nchw)
        elif t == "shortcut":
            if i - 1 not in self.fused:
                a_, b_, o_ = self.nhwc_store(i - 1), self.nhwc_store(L["src"]), self.nhwc_store(i)
                C = L["out"][0]
                if any(st[1] != 0 or st[2] != C for st in (a_, b_, o_)):
                    raise NotImplementedError("unfused shortcut on a channel slice")
                n = B * int(np.prod(L["out"]))
                hip.addvv(n, a_[0], 0, 1, b_[0], 0, 1, o_[0], 0, 1)
                hip.ActivateArray(n, o_[0], 0, L["act"])
        elif t == "route":
            if len(L["srcs"]) > 1:
                dst, doff, dpix = self.nhwc_store(i)
                _, h, ww = L["out"]
                for s_, off in self.copy_srcs[i]:
                    src, soff, spix = self.nhwc_store(s_)
                    hip.copyChannels(B * h * ww, self.layers[s_]["out"][0], src, soff, spix, dst, doff + off, dpix)
        elif t == "upsample":
            if i - 1 not in self.up_fused:
                C, h, ww = L["in"]
                src, soff, spix = self.nhwc_store(i - 1)
                dst, doff, dpix = self.nhwc_store(i)
                hip.upSampleNHWC(B, C, h, ww, L["stride"], L["scale"], src, soff, spix, dst, doff, dpix)
        elif t == "maxpool":
            C, h, ww = L["in"]
            _, oh, ow = L["out"]
            src, soff, spix = self.nhwc_store(i - 1)
            dst, doff, dpix = self.nhwc_store(i)
            hip.forwardMaxPoolNHWC(B, C, h, ww, oh, ow, L["stride"], L["stride"], L["pad"], L["size"], src, soff, spix,
                                   dst, doff, dpix)
        elif t == "yolo":
            if i - 1 not in self.yolo_fused:
                C, h, ww = L["in"]
                src, soff, spix = self.nhwc_store(i - 1)
                hip.yoloForwardNHWC(B, L["n"], L["classes"], h, ww, src, soff, spix, self.out[i])
            self._scale_xy(L, self.out[i])
            heads.append(self.out[i])
        return x

    def _scale_xy(self, L, out):
        """TYoloLayer.forwardGPU's scale_x_y step (nyololayer.pas:1098-1099):
        per image and anchor, the 2*h*w x / y entries become v*s + (1-s)/2
        (fmavss, a multiply then an add); nothing to do for s = 1."""
        s = np.float32(L.get("scale_xy", 1.0))
        if s == 1:
            return
        _, h, w = L["out"]
        bias = float(np.float32(0.5) * (np.float32(1) - s))
        per = (L["classes"] + 5) * h * w
        for b in range(self.batch):
            for a in range(L["n"]):
                self.hip.fmavss(2 * h * w, out, (b * L["n"] + a) * per, float(s), bias, out)

    def _layer(self, L, prev, heads):
        if self.layout == "nhwc":
            return self._layer_nhwc(L, prev, heads)
        hip, B = self.hip, self.batch
        i, t = L["index"], L["type"]
        if t == "convolutional":
            w, b, layout = self.w[i]
            C, h, ww = L["in"]
            res = None
            if i in self.fused:
                sc = self.layers[i + 1]
                res = self.buffer(sc["src"])
                dst = self.out[i + 1]
            else:
                dst = self.out[i]
            hip.conv2dForward(B, C, h, ww, L["filters"], L["size"], L["stride"], L["pad"], prev, 0, w, b,
                              L["act"], dst, 0, residual=res, weightLayout=layout)
            prev = dst
        elif t == "shortcut":
            if i - 1 not in self.fused:
                n = B * int(np.prod(L["out"]))
                hip.addvv(n, prev, 0, 1, self.buffer(L["src"]), 0, 1, self.out[i], 0, 1)
                hip.ActivateArray(n, self.out[i], 0, L["act"])
            prev = self.buffer(i)
        elif t == "route":
            if len(L["srcs"]) == 1:
                prev = self.buffer(L["srcs"][0])
            elif i in self.route_copies:  # batch 1: producers wrote their slices in place
                _, h, ww = L["out"]
                for s_, off in self.route_copies[i]:
                    n = int(np.prod(self.layers[s_]["out"]))
                    hip.copy(n, self.buffer(s_), 0, 1, self.out[i], off * h * ww, 1)
                prev = self.out[i]
            else:
                srcs = [self.buffer(s) for s in L["srcs"]]
                sizes = [int(np.prod(self.layers[s]["out"])) for s in L["srcs"]]
                if self.route_mode == "image":
                    hip.concat(B, srcs, sizes, self.out[i])
                else:  # whole batched tensors back to back (ntensors.pas:12045)
                    off = 0
                    for s, n in zip(srcs, sizes):
                        hip.copy(B * n, s, 0, 1, self.out[i], off, 1)
                        off += B * n
                prev = self.out[i]
        elif t == "upsample":
            C, h, ww = L["in"]
            hip.upSample(B, C, h, ww, prev, L["stride"], 1, L["scale"], self.out[i])
            prev = self.out[i]
        elif t == "maxpool":
            C, h, ww = L["in"]
            oc, oh, ow = L["out"]
            hip.forwardMaxPool(B, oc, oh, ow, prev, C, h, ww, L["stride"], L["stride"], L["pad"], L["size"],
                               None, self.out[i])
            prev = self.out[i]
        elif t == "yolo":
            C, h, ww = L["in"]
            hip.yoloForward(B, L["n"], L["classes"], h, ww, prev, self.out[i])
            self._scale_xy(L, self.out[i])
            heads.append(self.out[i])
            prev = self.out[i]
        return prev

    def capture(self, x):
        """Records one forward pass over the fixed input buffer `x` into a HIP
        graph on the library's own stream (after an eager pass has tuned the
        kernels); replay() then launches the whole network at once."""
        hip = self.hip
        hip.resetStream()
        if getattr(self, "_tuned", False):
            # one eager pass on the streams the capture uses: their split-K
            # scratch cannot be allocated while they are being captured
            self.forward(x)
        hip.finish()
        hip.graphBegin()
        try:
            heads = self.forward(x)
        finally:
            graph = hip.graphEnd()
        self.graph, self.graph_heads = graph, heads
        return heads

    def replay(self):
        self.hip.graphLaunch(self.graph)
        return self.graph_heads

    def release_graph(self):
        if getattr(self, "graph", None):
            self.hip.graphDestroy(self.graph)
            self.graph = None

    def detect(self, thresh=0.5, nms=0.45, img_w=None, img_h=None, relative=False, letter=False, capacity=8192):
        """TNNet.Detections and doNMSSort on the device after forward():
        decodes the yolo heads into boxes / objectness / class probabilities
        (tnh_yolo_detections), suppresses overlaps per class
        (tnh_yolo_nms_sort, skipped when nms is None) and returns per image
        (boxes [D, 4] in image pixels (or relative), objectness [D],
        prob [D, classes]) as numpy arrays: only the detection list leaves
        the GPU."""
        yl = [L for L in self.layers if L["type"] == "yolo"]
        if not yl:
            raise ValueError("network has no yolo layer")
        classes, n = yl[0]["classes"], yl[0]["n"]
        if any(L["classes"] != classes or L["n"] != n for L in yl):
            raise ValueError("yolo heads differ in classes or anchors per cell")
        _, H, W = self.layers[0]["in"]
        img_w, img_h = img_w or W, img_h or H
        B = self.batch
        key = (capacity, classes)
        if getattr(self, "_det_bufs", (None,))[0] != key:
            self._det_bufs = (key, DeviceArray((B, capacity, 4)), DeviceArray((B, capacity)),
                              DeviceArray((B, capacity, classes)), DeviceArray(B, np.int32))
        _, boxes, obj, prob, counts = self._det_bufs
        self.hip.yoloDetections(B, [self.out[L["index"]] for L in yl], [L["out"][1:] for L in yl], n, classes,
                                [L["anchors"] for L in yl], W, H, img_w, img_h, thresh, relative, letter, capacity,
                                boxes, obj, prob, counts)
        if nms is not None:
            self.hip.yoloNmsSort(B, classes, capacity, boxes, prob, counts, nms)
        self.hip.finish()
        cnt = counts.numpy()
        if (cnt > capacity).any():
            raise ValueError(f"{int(cnt.max())} detections exceed the capacity {capacity}")
        return [(boxes[b, :c].numpy(), obj[b, :c].numpy(), prob[b, :c].numpy()) for b, c in enumerate(cnt)]

    def head_convs(self):
        """Indices of the convolutions feeding the yolo layers (pre-logistic)."""
        return [L["index"] - 1 for L in self.layers if L["type"] == "yolo"]
