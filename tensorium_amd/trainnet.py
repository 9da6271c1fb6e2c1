"""Device-resident training step of the config-3 network through the C ABI.

Plays TNNet.trainEpoch for one batch (nnet.pas:474-530: Propagate = forward
+ backward, then update) on the network

    conv3x3(32)-BN-leaky, maxpool 2/2, conv3x3(64)-BN-leaky, maxpool 2/2,
    conv3x3(128)-BN-leaky, avgpool, connected 128->10, softmax cross-entropy

with the layer semantics of the reference CPU path:
  * TConvolutionalLayer.forward with batch norm in training mode
    (nConvolutionLayer.pas:457-566, TBaseLayer.batchNorm nbaselayer.pas:336-370):
    conv, MeansAndVars, rolling statistics, then normalize, scale, bias and
    leaky in one pass (tnh_bn_forward, bit-identical to the separate passes);
  * TConvolutionalLayer.backward (nConvolutionLayer.pas:571-671): leaky
    derivative, batchNormBack (nbaselayer.pas:372-392), im2col, weight
    gradient, W^T * delta, col2im; the first layer computes no input delta;
  * TMaxPoolLayer forward with int64 indexes / backward
    (nMaxPoolLayer.pas:363-512), TAvgPoolLayer (navgpoollayer.pas:60-100),
    TConnectedLayer (nconnectedlayer.pas:157-322, delta clamped to [-1, 1]),
    TSoftmaxLayer with cross-entropy (nsoftmaxlayer.pas:123-182);
  * updates (nConvolutionLayer.pas:673-710, nconnectedlayer.pas:324-355):
    SGD with momentum and decay; BN biases receive no gradient (the
    reference's batchNormBack leaves bias_updates alone).

Every operation is one C-ABI call on the library stream; buffers come from
the library's own allocator (nnhip.DeviceArray over tnh_malloc), so the
trainer needs no other GPU framework; its inputs may be any device buffer
(a DeviceArray or a torch tensor).  Conv weights are kept in the reference layout
[F][C*9] for the backward GEMMs and repacked tap-major for the forward.
"""
from __future__ import annotations

import math

import numpy as np

from .nnhip import WEIGHTS_TAP_MAJOR, DeviceArray, acLEAKY, acLINEAR

BLOCKS = ((3, 32), (32, 64), (64, 128))  # (C_in, F) of the conv-BN-leaky blocks
CLASSES = 10


def init_params(seed=0xC1FA):
    """Reference-style initial parameters (host numpy): conv weights
    U(-sqrt(2/(9C)), sqrt(2/(9C))) (nConvolutionLayer.pas:216-220), connected
    U(-sqrt(2/128), sqrt(2/128)) (nconnectedlayer.pas:79-80), BN scales 1,
    biases and rolling statistics 0; splitmix64 streams (synth)."""
    from . import synth

    p = {}
    for i, (c, f) in enumerate(BLOCKS):
        r = math.sqrt(2.0 / (9 * c))
        p[f"w{i}"] = synth.uniform(seed + 10 * i + 1, (f, c * 9), -r, r)
        p[f"s{i}"] = np.ones(f, np.float32)
        p[f"b{i}"] = np.zeros(f, np.float32)
        p[f"rm{i}"] = np.zeros(f, np.float32)
        p[f"rv{i}"] = np.zeros(f, np.float32)
    r = math.sqrt(2.0 / BLOCKS[-1][1])
    p["fw"] = synth.uniform(seed + 100, (CLASSES, BLOCKS[-1][1]), -r, r)
    p["fb"] = np.zeros(CLASSES, np.float32)
    for k in list(p):
        if k[0] in "wsbf":  # w*, s*, b*, fw, fb carry momentum buffers
            p["u_" + k] = np.zeros_like(p[k])
    return p


class CifarTrainer:
    """One trainer per (batch, image size); `step(x, truth)` runs forward,
    backward and update on the device; `cost()` reads the loss back."""

    def __init__(self, hip, params, batch, size=32, lr=1e-3, momentum=0.9, decay=1e-4, bn_momentum=0.1,
                 fused_wgrad=True, conv_dgrad=True, fused_head=True, fused_pool_bwd=True, fused_stats=True,
                 store_bn_outputs=False, defer_wgrad_sum=True):
        """fused_wgrad: the conv weight gradients gather their column matrix
        inside the GEMM (tnh_conv2d_wgrad); False runs the reference's
        im2col + NT product (the same bits).  conv_dgrad: the conv input
        deltas are one convolution of the output delta with the flipped
        weights; False runs the reference's TN product + col2im (the same
        sums in another order).  fused_head: the average pool, the connected
        layer, softmax and cross-entropy forward in one launch and their
        backward in another; False runs them call by call.  fused_pool_bwd:
        the pool layers' backwards are formed inside the batch-norm backward
        below them (no zeroed delta, no scatter launch; the same bits);
        False runs backwardMaxPool / avgPoolBackward into zeroed deltas.
        fused_stats: the batch statistics' final step is taken by the
        normalize pass (the same bits); False calls bnStatistics first.
        store_bn_outputs: the forward stores x_norm and the activation's
        output for the backward, as the reference's layer does; False: the
        backward's first pass forms both again from x, the statistics, the
        scales and the biases (the same bits, four fewer passes over a
        layer's activations; out{i} is then stored only where a later layer
        reads it).  defer_wgrad_sum (with fused_wgrad): the weight gradients
        of 8192 and more weights keep their split sums in the trainer's
        memory (tnh_conv2d_wgrad_pieces) and the update's pass adds them to
        the weight updates (tnh_sgd_update_pack_pieces; the same bits, one
        reduction launch fewer per such layer); u_w{i} of those layers then
        holds the new gradient only after update()."""
        self.hip, self.B = hip, batch
        self.fused_wgrad, self.conv_dgrad, self.fused_head = fused_wgrad, conv_dgrad, fused_head
        self.fused_pool_bwd, self.fused_stats = fused_pool_bwd, fused_stats
        self.store_bn_outputs = store_bn_outputs
        self.defer_wgrad_sum = defer_wgrad_sum and fused_wgrad
        self._out_stored = [True] * len(BLOCKS)
        self.lr, self.momentum, self.decay, self.bnm = lr, momentum, decay, bn_momentum
        # Parameters live in two arenas (weights with decay; biases and
        # scales without), their momentum buffers in two more with the same
        # offsets, so each SGD step is two launches over all layers: the
        # update is element-wise with the same scalars for every tensor of an
        # arena, so this is bit-identical to per-tensor updates.
        self.p = {}
        self.arena = {}
        for group, keys in (("w", [k for k in params if k[0] == "w"] + ["fw"]),
                            ("p", [k for k in params if k[0] in "sb"] + ["fb"])):
            n = sum(params[k].size for k in keys)
            flat = DeviceArray(n)
            uflat = DeviceArray(n)
            off = 0
            for k in keys:
                v = np.ascontiguousarray(params[k])
                flat[off:off + v.size].copy_from(v.ravel())
                uflat[off:off + v.size].copy_from(np.ascontiguousarray(params["u_" + k]).ravel())
                self.p[k] = flat[off:off + v.size].view(v.shape)
                self.p["u_" + k] = uflat[off:off + v.size].view(v.shape)
                off += v.size
            self.arena[group] = (flat, uflat)
        for k, v in params.items():
            if k not in self.p:  # rolling statistics
                self.p[k] = DeviceArray.from_numpy(np.ascontiguousarray(v, dtype=np.float32))
        self.packed = [DeviceArray(self.p[f"w{i}"].shape) for i in range(len(BLOCKS))]
        self.flipped = [DeviceArray(self.p[f"w{i}"].shape) for i in range(len(BLOCKS))]
        B = batch
        t = {}
        h = size
        self.dims = []
        # deltas that the backward pass accumulates into (TNNet.forward zeroes
        # them, nnet.pas:287-294) share one arena: one fill per step
        zsizes = []
        hh = size
        for i, (c, f) in enumerate(BLOCKS):
            zsizes.append(("delta", i, (B, f, hh, hh)))
            if i > 0:
                zsizes.append(("dx", i, (B, c, hh, hh)))
            if i < len(BLOCKS) - 1:
                hh //= 2
        self.zero_arena = DeviceArray(sum(int(np.prod(sh)) for _, _, sh in zsizes))
        off = 0
        for name, i, sh in zsizes:
            n = int(np.prod(sh))
            t[f"{name}{i}"] = self.zero_arena[off:off + n].view(sh)
            off += n
        for i, (c, f) in enumerate(BLOCKS):
            self.dims.append((c, h, f))
            for name in ("x", "xn", "out") if store_bn_outputs else ("x", "out"):
                t[f"{name}{i}"] = DeviceArray((B, f, h, h))
            t[f"mean{i}"] = DeviceArray(f)
            t[f"var{i}"] = DeviceArray(f)
            t[f"md{i}"] = DeviceArray(f)
            t[f"vd{i}"] = DeviceArray(f)
            if i < len(BLOCKS) - 1:
                t[f"pool{i}"] = DeviceArray((B, f, h // 2, h // 2))
                t[f"pidx{i}"] = DeviceArray((B, f, h // 2, h // 2), np.int64)
                h //= 2
        self.final_hw = h
        F = BLOCKS[-1][1]
        t["avg"] = DeviceArray((B, F))
        t["avg_delta"] = DeviceArray((B, F))
        t["logits"] = DeviceArray((B, CLASSES))
        t["prob"] = DeviceArray((B, CLASSES))
        t["fc_delta"] = DeviceArray((B, CLASSES))
        t["err"] = DeviceArray((B, CLASSES))
        colmax = max(c * 9 * (hh * hh) for (c, hh, f) in self.dims)
        t["col"] = DeviceArray(B * colmax)
        self.t = t
        # split sums of the deferred weight gradients: [pieces][F][C*9] each
        self.pieces = [None] * len(self.dims)
        if self.defer_wgrad_sum:
            for i, (c, hh, f) in enumerate(self.dims):
                if i == 0 or f * c * 9 < 8192:
                    continue  # conv1: 864 weights, summed a wave per weight by tnh_conv2d_wgrad
                n = hip.convWeightGradientPieces(B, c, hh, hh, f, 3, 3, 1, 1, 1, 1, 1, 1, t[f"pool{i - 1}"],
                                                 c * hh * hh, t[f"delta{i}"], f * hh * hh)
                self.pieces[i] = (DeviceArray(n * f * c * 9), n)
        self._pack()

    def _pack_layers(self):
        w = self.arena["w"][0]
        out = []
        for i, (c, _, f) in enumerate(self.dims):
            off = (self.p[f"w{i}"].data_ptr() - w.data_ptr()) // 4
            flip = self.flipped[i] if (self.conv_dgrad and i > 0) else None
            out.append((off, f, c, 9, self.packed[i], flip))
        return out

    def _pack(self):
        for i, (c, _, f) in enumerate(self.dims):
            if self.conv_dgrad and i > 0:  # the first layer computes no input delta
                self.hip.packConvWeightsDgrad(f, c, 3, self.p[f"w{i}"], self.packed[i], self.flipped[i])
            else:
                self.hip.packConvWeights(f, c, 3, self.p[f"w{i}"], self.packed[i])

    # ------------------------------------------------------------- forward
    def forward(self, x, truth):
        hip, p, t, B = self.hip, self.p, self.t, self.B
        self.input = x
        h = x
        for i, (c, hh, f) in enumerate(self.dims):
            n = B * f * hh * hh
            y = t[f"x{i}"]
            hip.conv2dForward(B, c, hh, hh, f, 3, 1, 1, h, 0, self.packed[i], None, acLINEAR, y, 0,
                              weightLayout=WEIGHTS_TAP_MAJOR)
            last = i == len(self.dims) - 1
            # the activation's output is stored where the backward cannot form
            # it again or a later layer reads it (the unpooled last block)
            pooled = not last or (self.fused_head and hh * hh <= 64)
            self._out_stored[i] = self.store_bn_outputs or not pooled
            xn = t[f"xn{i}"] if self.store_bn_outputs else None
            out = t[f"out{i}"] if self._out_stored[i] else None
            bnm = float(np.float32(self.bnm))
            stats = (t[f"mean{i}"], t[f"var{i}"], p[f"rm{i}"], p[f"rv{i}"], bnm)
            if self.fused_stats and self.fused_head and i == len(self.dims) - 1 and hh * hh <= 64:
                # MeansAndVars (rolling = (1 - m) * rolling + m * stat), the
                # normalize pass and the head's average pool: three launches
                hip.bnTrainForwardAvgPool(B, f, hh * hh, y, xn, out, *stats, p[f"s{i}"], p[f"b{i}"], acLEAKY,
                                          t["avg"])
                h = None
                continue
            if self.fused_stats and i < len(self.dims) - 1:
                # ... and the 2x2 maxpool
                hip.bnTrainForwardMaxPool(B, f, hh, hh, y, xn, out, *stats, p[f"s{i}"], p[f"b{i}"], acLEAKY,
                                          t[f"pool{i}"], t[f"pidx{i}"])
                h = t[f"pool{i}"]
                continue
            # MeansAndVars, then rolling = (1 - m) * rolling, rolling = axpy(m, stat)
            hip.bnStatistics(n, f, B, y, 0, *stats)
            # x (y) is kept as the layer's pre-normalization copy; one pass
            # writes x_norm and act(scale * x_norm + bias)
            if i < len(self.dims) - 1:
                # ... and the 2x2 maxpool of out in the same pass
                hip.bnForwardMaxPool(B, f, hh, hh, y, xn, out, t[f"mean{i}"], t[f"var{i}"], p[f"s{i}"], p[f"b{i}"],
                                     acLEAKY, t[f"pool{i}"], t[f"pidx{i}"])
                h = t[f"pool{i}"]
            elif self.fused_head and hh * hh <= 64:
                # ... and the average of each plane (the head's average pool)
                hip.bnForwardAvgPool(B, f, hh * hh, y, xn, out, t[f"mean{i}"], t[f"var{i}"], p[f"s{i}"], p[f"b{i}"],
                                     acLEAKY, t["avg"])
                h = None
            else:
                hip.bnForward(n, f, B, y, xn, out, t[f"mean{i}"], t[f"var{i}"], p[f"s{i}"], p[f"b{i}"], acLEAKY)
                h = out
        F, hw = BLOCKS[-1][1], self.final_hw
        self.truth = truth
        # softmax backward: net.delta (zeroed each forward) += delta; t - p is
        # never -0, so writing it straight into the zeroed delta is exact
        if self.fused_head:
            hip.softmaxHeadForward(B, F, hw * hw, CLASSES, h, t["avg"], p["fw"], p["fb"], truth, t["logits"],
                                   t["prob"], t["fc_delta"], t["err"])
            return
        hip.avgPoolForward(B, F, hw, hw, h, t["avg"])
        hip.gemm(False, True, B, CLASSES, F, 1.0, t["avg"], 0, F, p["fw"], 0, F, 0.0, t["logits"], 0, CLASSES)
        hip.forwardBias(B * CLASSES, t["logits"], 0, CLASSES, p["fb"], 1, B)
        hip.softmaxBatch(CLASSES, t["logits"], 0, B, CLASSES, 1, CLASSES, 1, 1.0, t["prob"], 0)
        hip.crossEntropySoftmax(B * CLASSES, t["prob"], truth, t["fc_delta"], t["err"])

    # ------------------------------------------------------------ backward
    def backward(self):
        hip, p, t, B = self.hip, self.p, self.t, self.B
        F, hw = BLOCKS[-1][1], self.final_hw
        nfc = B * CLASSES
        # pool backwards and col2im accumulate into zeroed deltas; the conv
        # input deltas and the pool backwards formed in the batch-norm
        # backward write every element
        if not (self.fused_pool_bwd and self.conv_dgrad):
            hip.fill(self.zero_arena.numel(), self.zero_arena, 0, 0.0, 1)
        last = len(self.dims) - 1
        d = t[f"delta{last}"]
        if self.fused_head:
            # connected backward (and the avgpool backward into the last
            # block's zeroed delta unless the batch-norm backward forms it),
            # one launch
            hip.softmaxHeadBackward(B, F, hw * hw, CLASSES, 1.0, t["fc_delta"], t["avg"], p["fw"], p["u_fw"],
                                    p["u_fb"], t["avg_delta"], None if self.fused_pool_bwd else d)
        else:
            hip.clamp(nfc, 1.0, t["fc_delta"], t["fc_delta"])
            hip.backwardBias(CLASSES, p["u_fb"], nfc, t["fc_delta"], 0, 1, B)
            hip.gemm(True, False, CLASSES, F, B, 1.0, t["fc_delta"], 0, CLASSES, t["avg"], 0, F, 1.0, p["u_fw"], 0, F)
            hip.gemm(False, False, B, F, CLASSES, 1.0, t["fc_delta"], 0, CLASSES, p["fw"], 0, F, 0.0, t["avg_delta"],
                     0, F)
            if not self.fused_pool_bwd:
                hip.avgPoolBackward(B, F, hw, hw, t["avg_delta"], d)
        col = t["col"]
        for i in range(last, -1, -1):
            c, hh, f = self.dims[i]
            n = B * f * hh * hh
            d = t[f"delta{i}"]
            # leaky gradient, batchNormBack's dgamma (addDots) and delta *=
            # gamma (forwardScale) in one pass, then the mean / variance
            # deltas and normalizeDelta (four launches)
            bn = (n, f, B)
            out_i = t[f"out{i}"] if self._out_stored[i] else None
            xn_i = t[f"xn{i}"] if self.store_bn_outputs else None
            rest = (out_i, acLEAKY, xn_i, t[f"x{i}"], p[f"s{i}"], t[f"mean{i}"], t[f"var{i}"], d, p[f"u_s{i}"],
                    t[f"md{i}"], t[f"vd{i}"], p[f"b{i}"])
            if not self.fused_pool_bwd:
                hip.bnBackward(*bn, *rest)
            elif i == last:
                # ... the first pass forming the average pool's backward
                hip.bnBackwardAvgPool(*bn, t["avg_delta"], *rest)
            else:
                # ... the first pass forming the 2x2 maxpool's backward of
                # the next block's input delta
                hip.bnBackwardMaxPool(*bn, hh, hh, t[f"pidx{i}"], t[f"dx{i + 1}"], *rest)
            # conv weight gradient: sum_b delta_b * im2col(input_b)^T
            src = self.input if i == 0 else t[f"pool{i - 1}"]
            K, L = c * 9, hh * hh
            if self.pieces[i] is not None:
                buf, _ = self.pieces[i]
                hip.convWeightGradientPieces(B, c, hh, hh, f, 3, 3, 1, 1, 1, 1, 1, 1, src, c * hh * hh, d, f * L, buf,
                                             buf.numel())
            elif self.fused_wgrad:
                hip.convWeightGradient(B, c, hh, hh, f, 3, 3, 1, 1, 1, 1, 1, 1, src, c * hh * hh, d, f * L, 1.0, 1.0,
                                       p[f"u_w{i}"])
            else:
                hip.im2colStridedBatched(c, hh, hh, 3, 3, 1, 1, 1, 1, 1, 1, src, c * hh * hh, 0, col, K * L, 0, B)
                hip.gemmNTBatchReduce(f, K, L, 1.0, d, 0, L, f * L, col, 0, L, K * L, 1.0, p[f"u_w{i}"], 0, K, B)
            if i == 0:
                break  # state.delta is nil for the first layer
            dx = t[f"dx{i}"]
            if self.conv_dgrad:
                # input delta: the output delta convolved with the flipped,
                # transposed weights (f channels in, c filters out, pad 1)
                hip.conv2dForward(B, f, hh, hh, c, 3, 1, 1, d, 0, self.flipped[i], None, acLINEAR, dx, 0,
                                  weightLayout=WEIGHTS_TAP_MAJOR)
            else:
                # input delta: col_b = W^T * delta_b, then col2im into a zeroed delta
                hip.gemmStridedBatched(True, False, K, L, f, 1.0, p[f"w{i}"], 0, K, 0, d, 0, L, f * L, 0.0, col, 0,
                                       L, K * L, B)
                hip.col2imStridedBatched(c, hh, hh, 3, 3, 1, 1, 1, 1, 1, 1, col, K * L, 0, dx, c * hh * hh, 0, B)
            if not self.fused_pool_bwd:
                # maxpool backward into the previous block's zeroed delta
                pc, phh, pf = self.dims[i - 1]
                prev = t[f"delta{i - 1}"]
                hip.backwardMaxPool(B, pf, phh // 2, phh // 2, prev, t[f"pidx{i - 1}"], dx)

    # -------------------------------------------------------------- update
    def update(self):
        """SGD with momentum and decay on every weight (conv and connected),
        momentum only on biases and scales (nConvolutionLayer.pas:673-710,
        nconnectedlayer.pas:324-355), one launch per arena."""
        hip, B = self.hip, self.B
        lr, m, dec = self.lr, self.momentum, self.decay
        w, uw = self.arena["w"]
        q, uq = self.arena["p"]
        # the update's pass also writes the conv weights' tap-major (and
        # flipped) copies the next forward and backward read, and updates the
        # biases and scales
        hip.sgdUpdatePack(w.numel(), lr, B, m, dec, w, uw, self._pack_layers(), q.numel(), q, uq,
                          pieces=self.pieces if self.defer_wgrad_sum else None)

    def step(self, x, truth):
        self.forward(x, truth)
        self.backward()
        self.update()

    def capture(self, x, truth):
        """Records one step (forward, backward, update) over the fixed input
        buffers into a HIP graph on the library's own stream.  It first runs
        one eager step on that stream (so the parameters advance by one
        step): scratch of the weight-gradient split sums cannot be allocated
        while a stream is being captured, and without it the captured step
        would sum without splits (slower, and in another order than the
        eager steps).  Each replay() then trains on the same buffers
        (contents may change)."""
        hip = self.hip
        hip.finish()
        hip.resetStream()
        self.step(x, truth)
        hip.finish()
        hip.graphBegin()
        try:
            self.step(x, truth)
        finally:
            self.graph = hip.graphEnd()

    def replay(self):
        self.hip.graphLaunch(self.graph)

    def release_graph(self):
        if getattr(self, "graph", None):
            self.hip.graphDestroy(self.graph)
            self.graph = None

    def cost(self):
        """Sum of the softmax cross-entropy errors of the last forward
        (TSoftmaxLayer cost[0] = loss.Sum(), read by TNNet.cost)."""
        self.hip.finish()
        err = self.t["err"].numpy()
        return np.float32(err.astype(np.float64).sum())

    def host(self, name):
        self.hip.finish()
        src = self.p if name in self.p else self.t
        return src[name].numpy()
