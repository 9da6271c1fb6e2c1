"""Benchmark: YOLOv3-416 fp32 inference on one MI355X through libtensorium_hip.

A step is one forward pass of YOLOv3-416 (75 convolutions, shortcuts,
routes, upsamples, yolo heads) over a batch of synthetic images already
resident in HBM.  Prints ONE JSON line (rank 0):

  value          images/s at the configured batch (default 16)
  roofline       the dominant kernel (most GPU time) from a separate pass that
                 brackets every launch with HIP events on the library stream:
                 achieved = its algorithmic conv FLOP (2*M*N*K) / its time,
                 against the 157.3 TFLOP/s fp32 MFMA peak
  cpu_baseline   the CPU oracle (C restatement of the reference's AVX2 path)
                 on the host, a bounded sample of batch-1 images

Usage: python bench.py [--gpus 1] [--steps 20] [--warmup 3] [--batch 16]
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "conv im2col+SGEMM GFLOP/s (% fp32 MFMA peak); YOLOv3-416 img/s at batch 1/16"
PEAK_FP32_MFMA = 157.3e12
LAYOUT = ["auto"]  # activation layout of the networks bench.py builds (--layout)


def layout_for(batch):
    """--layout auto: channels-last between layers from batch 2 up (measured
    faster at batch 4 and 16), NCHW at batch 1 (faster there)."""
    if LAYOUT[0] != "auto":
        return LAYOUT[0]
    return "nhwc" if batch > 1 else "nchw"
PEAK_HBM = 8.0e12
# HBM bytes per launch of the dominant kernel family (tap-major 3x3 conv,
# channels-last conv_nhwc_kernel or NCHW conv_lean_kernel, incl. its
# reductions) from two rocprofv3 --pmc runs
# of `bench.py --counter-pass` (FETCH_SIZE then WRITE_SIZE, KiB per dispatch,
# scaled by a 64 MiB copy: read = 2.0 x FETCH_SIZE, write = 1.0 x WRITE_SIZE);
# profiles/yolov3_416_b16_conv_{nhwc,lean}_kernel.md hold the figures and commands.
TRAFFIC_TAP3X3_B16 = {"conv_lean_kernel<tap3x3>": (2.0 * 168517.7 + 40664.9) * 1024,
                      "conv_nhwc_kernel<tap3x3>": (2.0 * 68422.7 + 39756.1) * 1024}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def kernel_kind(L, batch, layout):
    """Kernel family a conv layer launches: the lean implicit GEMM over
    tap-major 3x3 or 1x1 operands (conv_nhwc_kernel for channels-last
    activations, conv_lean_kernel for NCHW; conv_lean.hpp), or the per-pixel
    kernel for few input channels (conv_smallc_kernel)."""
    lean = "conv_nhwc_kernel" if layout == "nhwc" else "conv_lean_kernel"
    if L["size"] == 1 and L["stride"] == 1 and L["pad"] == 0:
        return f"{lean}<1x1>"
    if L["size"] == 3 and L["in"][0] <= 4:
        return "conv_smallc_kernel<3x3>"
    if L["size"] == 3 and L["in"][0] % 16 == 0:
        return f"{lean}<tap3x3>"
    return f"conv_kernel<gather{L['size']}x{L['size']}>"


def time_forward(hip, net, x, steps, warmup, graph=True):
    """Warm-up steps run eagerly (the first one autotunes every layer shape);
    the forward is then captured into a HIP graph and the timed steps replay
    it (graph=False times eager launches instead)."""
    import torch

    for _ in range(warmup):
        net.forward(x)
    torch.cuda.synchronize()
    hip.finish()
    if graph:
        net.capture(x)
        net.replay()
        hip.finish()
    e0, e1 = hip.eventCreate(), hip.eventCreate()
    t0 = time.perf_counter()
    hip.eventRecord(e0)
    for _ in range(steps):
        if graph:
            net.replay()
        else:
            net.forward(x)
    hip.eventRecord(e1)
    hip.finish()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = hip.eventElapsed(e0, e1)
    hip.eventDestroy(e0)
    hip.eventDestroy(e1)
    if graph:
        net.release_graph()
        hip.useTorchStream()
    return ms, wall


def profile_kernels(hip, net, layers, x, reps=3):
    """Per-layer GPU durations from HIP events recorded on the library stream
    around each layer's launches; conv layers are grouped by kernel family."""
    evs = {L["index"]: (hip.eventCreate(), hip.eventCreate()) for L in layers}

    def hook(i, begin):
        hip.eventRecord(evs[i][0 if begin else 1])

    stats = {}
    try:
        for _ in range(reps):
            net.forward(x, on_layer=hook)
            hip.finish()
            for L in layers:
                i = L["index"]
                ms = hip.eventElapsed(*evs[i])
                if L["type"] == "convolutional":
                    kind = kernel_kind(L, net.batch, net.layout)
                    F, oh, ow = L["out"]
                    flop = 2 * F * L["in"][0] * L["size"] ** 2 * oh * ow * net.batch
                else:
                    kind, flop = L["type"], 0
                s = stats.setdefault(kind, {"ms": 0.0, "flop": 0.0, "launches": 0.0})
                s["ms"] += ms / reps
                s["flop"] += flop / reps
                s["launches"] += 1.0 / reps
    finally:
        for a, b in evs.values():
            hip.eventDestroy(a)
            hip.eventDestroy(b)
    return stats


def cpu_baseline(layers, weights, budget_s=12.0):
    """Oracle YOLOv3-416 forward at batch 1 on the host cores, repeated until
    ~budget_s of work; returns (img/s, threads, images)."""
    import numpy as np

    from oracle import netref
    from oracle import refcpu as R
    from tensorium_amd import synth

    threads = min(16, os.cpu_count() or 4)
    R.set_threads(threads)
    x = synth.uniform(7, (1, 3, 416, 416))
    netref.forward(layers, weights, x)  # warm-up
    n, t0 = 0, time.perf_counter()
    while True:
        netref.forward(layers, weights, x)
        n += 1
        if time.perf_counter() - t0 >= budget_s:
            break
    dt = time.perf_counter() - t0
    del np
    return n / dt, threads, n


COPY_BYTES = 64 << 20


def time_events(hip, fn, reps):
    """Average ms of fn() over reps calls, HIP events on the library stream."""
    e0, e1 = hip.eventCreate(), hip.eventCreate()
    hip.eventRecord(e0)
    for _ in range(reps):
        fn()
    hip.eventRecord(e1)
    ms = hip.eventElapsed(e0, e1) / reps
    hip.eventDestroy(e0)
    hip.eventDestroy(e1)
    return ms


def time_graph(hip, fn, reps):
    """Average ms of fn() as replayed from a HIP graph of `reps` calls (no
    host launch cost in the timed region: small kernels are not launch-bound).
    The capture runs on the library's own stream (the null stream that bench
    shares with torch cannot be captured); the caller has synchronized."""
    hip.finish()
    hip.resetStream()
    hip.graphBegin()
    for _ in range(reps):
        fn()
    g = hip.graphEnd()
    hip.graphLaunch(g)
    hip.finish()
    e0, e1 = hip.eventCreate(), hip.eventCreate()
    best = 1e30
    for _ in range(2):
        hip.eventRecord(e0)
        hip.graphLaunch(g)
        hip.eventRecord(e1)
        best = min(best, hip.eventElapsed(e0, e1) / reps)
    hip.eventDestroy(e0)
    hip.eventDestroy(e1)
    hip.graphDestroy(g)
    hip.finish()
    hip.useTorchStream()
    return best


def extra_single_conv(hip):
    """Config 1: one conv layer forward, batch 1, 3x416x416 -> 16 filters 3x3
    s1 p1, weights N(0, 0.05), bias 0, leaky 0.1 (GEMM M=16, N=173056, K=27)."""
    import numpy as np
    import torch

    from tensorium_amd import synth
    from tensorium_amd.nnhip import acLEAKY

    x = torch.from_numpy(synth.uniform(1, (1, 3, 416, 416))).cuda()
    w = torch.from_numpy(synth.normal(2, (16, 27), 0.05)).cuda()
    b = torch.zeros(16, dtype=torch.float32, device="cuda")
    out = torch.empty((1, 16, 416, 416), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()

    def fn():
        hip.conv2dForward(1, 3, 416, 416, 16, 3, 1, 1, x, 0, w, b, acLEAKY, out, 0)

    for _ in range(3):
        fn()
    ms = time_events(hip, fn, 50)
    flop = 2.0 * 16 * 27 * 416 * 416
    byts = 4.0 * (3 * 416 * 416 + 16 * 416 * 416 + 16 * 27)
    del np
    return {"workload": "conv 3->16 3x3 s1 p1 + bias + leaky, 1x3x416x416", "us": round(ms * 1e3, 2),
            "gflops": round(flop / ms / 1e6, 1), "gb_s": round(byts / ms / 1e6, 1),
            "hbm_frac": round(byts / ms * 1e3 / PEAK_HBM, 4)}


def extra_sgemm(hip):
    """Config 2: C = op(A)*op(B) (beta 0), A and B ~ U[-1, 1): NN at 512^3 ..
    8192^3, the four variants at 4096^3 and the YOLOv3 conv-shaped skinny
    GEMMs, each timed as a graph replay after the first (tuning) call."""
    import torch

    from tensorium_amd import synth

    cases = [("NN", 512, 512, 512), ("NN", 1024, 1024, 1024), ("NN", 2048, 2048, 2048),
             ("NN", 4096, 4096, 4096), ("NT", 4096, 4096, 4096), ("TN", 4096, 4096, 4096),
             ("TT", 4096, 4096, 4096), ("NN", 8192, 8192, 8192), ("NN", 64, 692224, 288),
             ("NN", 256, 43264, 1152), ("NN", 1024, 2704, 4608)]
    res = []
    for var, M, N, K in cases:
        ta, tb = var[0] == "T", var[1] == "T"
        A = torch.from_numpy(synth.uniform(11, (M * K,), -1, 1)).cuda()
        B = torch.from_numpy(synth.uniform(12, (K * N,), -1, 1)).cuda()
        C = torch.empty(M * N, dtype=torch.float32, device="cuda")
        torch.cuda.synchronize()
        lda, ldb = (M if ta else K), (K if tb else N)

        def fn():
            hip.gemm(ta, tb, M, N, K, 1.0, A, 0, lda, B, 0, ldb, 0.0, C, 0, N)

        fn()
        reps = 3 if M * N * K >= 8192 ** 3 else (10 if M * N * K >= 1024 ** 3 else 50)
        ms = time_graph(hip, fn, reps)
        res.append({"variant": var, "M": M, "N": N, "K": K, "ms": round(ms, 4),
                    "tflops": round(2.0 * M * N * K / ms / 1e9, 2),
                    "frac": round(2.0 * M * N * K / ms * 1e3 / PEAK_FP32_MFMA, 4)})
        del A, B, C
        torch.cuda.empty_cache()
    return res


def extra_train(hip, steps, warmup, cpu_steps):
    """Config 3: one training step (forward + backward + SGD update) of the
    conv-BN-leaky x3 / pool / connected / softmax-CE network on synthetic
    3x32x32 U[0,1) images with one-hot labels, batch 128, replayed from a HIP
    graph; the CPU oracle's step timed beside it."""
    import numpy as np
    import torch

    from tensorium_amd import synth, trainnet

    B = 128
    x = synth.uniform(21, (B, 3, 32, 32))
    lab = (synth.splitmix64(22, B) % np.uint64(10)).astype(np.int64)
    truth = np.zeros((B, 10), np.float32)
    truth[np.arange(B), lab] = 1
    params = trainnet.init_params()
    tr = trainnet.CifarTrainer(hip, params, B)
    dx, dt = torch.from_numpy(x).cuda(), torch.from_numpy(truth).cuda()
    torch.cuda.synchronize()
    for _ in range(max(1, warmup)):
        tr.step(dx, dt)
    loss0 = float(tr.cost())
    tr.capture(dx, dt)
    tr.replay()
    tr.hip.finish()
    ms = time_events(hip, tr.replay, steps)
    loss1 = float(tr.cost())
    tr.release_graph()
    hip.useTorchStream()
    flop = 0
    for (c, f), hw in zip(trainnet.BLOCKS, (32, 16, 8)):
        flop += 2 * f * 9 * c * hw * hw * B * (2 if c == 3 else 3)  # fwd + dW (+ dX except layer 0)
    out = {"workload": "config-3 CNN train step (fwd+bwd+SGD), batch 128, 3x32x32", "ms_per_step": round(ms, 4),
           "img_s": round(B / ms * 1e3, 1), "gflop_per_step": round(flop / 1e9, 3),
           "gflops": round(flop / ms / 1e6, 1), "launch": "hip_graph",
           "loss_first": round(loss0, 3), "loss_after": round(loss1, 3)}
    if cpu_steps:
        from oracle import refcpu as R
        from oracle import trainref as T

        R.set_threads(min(16, os.cpu_count() or 4))
        ref = T.CifarStep(params)
        ref.step(x, truth)
        t0 = time.perf_counter()
        for _ in range(cpu_steps):
            ref.step(x, truth)
        cms = (time.perf_counter() - t0) / cpu_steps * 1e3
        out["cpu_baseline"] = {"value": round(cms, 1), "unit": "ms/step", "cores": R.get_threads(), "kind": "port",
                               "sample": f"{cpu_steps} oracle steps (C AVX2 GEMM/im2col/col2im + numpy BN/softmax)"}
    return out


def extra_yolo(hip, layers608, weights608, steps, warmup, batch=32, size=608):
    """Config 5: YOLOv3-608 inference at batch 32 (HIP graph replay)."""
    import torch

    from tensorium_amd import darknet, synth

    net = darknet.Network(hip, layers608, batch, weights608, layout=layout_for(batch))
    x = torch.from_numpy(synth.uniform(9, (batch, 3, size, size))).cuda()
    torch.cuda.synchronize()
    ms, _ = time_forward(hip, net, x, steps, warmup, graph=True)
    ms /= steps
    flop = darknet.conv_flops(layers608) * batch
    del net, x
    torch.cuda.empty_cache()
    return {"workload": f"YOLOv3-{size} fp32 inference, batch {batch}", "ms_per_step": round(ms, 3),
            "img_s": round(batch / ms * 1e3, 1), "conv_frac_fp32_mfma_peak": round(flop / ms * 1e3 / PEAK_FP32_MFMA, 4)}


def extra_detect(hip, layers, weights, batch=16, thresh=0.5, nms=0.45):
    """YOLO detection list + per-class NMS on the device (the reference's
    TNNet.Detections, nnet.pas:584, and doNMSSort, ntypes.pas:1612) after a YOLOv3-416
    forward at batch 16 (tnh_yolo_detections +
    tnh_yolo_nms_sort, device time; the list stays in HBM)."""
    import torch

    from tensorium_amd import darknet, synth

    net = darknet.Network(hip, layers, batch, weights, layout=layout_for(batch))
    x = torch.from_numpy(synth.uniform(7, (batch, 3, 416, 416))).cuda()
    torch.cuda.synchronize()
    net.forward(x)
    dets = net.detect(thresh=thresh, nms=nms)  # allocates the buffers, checks capacity
    yl = [L for L in layers if L["type"] == "yolo"]
    _, boxes, obj, prob, counts = net._det_bufs
    cap = boxes.shape[1]

    def fn():
        hip.yoloDetections(batch, [net.out[L["index"]] for L in yl], [L["out"][1:] for L in yl], yl[0]["n"],
                           yl[0]["classes"], [L["anchors"] for L in yl], 416, 416, 416, 416, thresh, False, False,
                           cap, boxes, obj, prob, counts)
        hip.yoloNmsSort(batch, yl[0]["classes"], cap, boxes, prob, counts, nms)

    for _ in range(2):
        fn()
    ms = time_events(hip, fn, 10)
    nd = sum(len(d[1]) for d in dets)
    kept = sum(int((d[2] > 0).sum()) for d in dets)
    del net, x
    return {"workload": f"YOLOv3-416 detections + per-class NMS on device, batch {batch}, thresh {thresh}, nms {nms}",
            "us": round(ms * 1e3, 1), "detections": nd, "kept_class_scores": kept}


def counter_pass(hip, net, args):
    """Warm-up forwards (autotuning), a fence, then exactly one forward and one
    copy of COPY_BYTES: the dispatches a counter run attributes.  The copy
    calibrates FETCH_SIZE / WRITE_SIZE (KiB per dispatch) against a kernel whose
    HBM traffic is known (COPY_BYTES read + COPY_BYTES written)."""
    import torch

    from tensorium_amd import synth

    x = torch.from_numpy(synth.uniform(7, (args.batch, 3, args.size, args.size))).cuda()
    src = torch.rand(COPY_BYTES // 4, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(max(1, args.warmup)):
        net.forward(x)
    hip.finish()
    torch.cuda.synchronize()
    marker = torch.zeros(64, dtype=torch.float32, device="cuda")
    hip.fill(1, marker, 0, 0.0, 1)  # fill_kernel: marks the start of the attributed region
    log("counter pass: timed region starts")
    net.forward(x)
    hip.copy(COPY_BYTES // 4, src, 0, 1, dst, 0, 1)
    hip.finish()
    torch.cuda.synchronize()
    log("counter pass: done")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--batch", type=int, default=16)
    ap.add_argument("--size", type=int, default=416)
    ap.add_argument("--cpu-budget", type=float, default=12.0)
    ap.add_argument("--weights", default=None,
                    help="darknet .weights file for the YOLOv3 network (batch norm folded on the host); default: "
                         "the seeded He-normal random weights of the benchmark configuration")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-batch1", action="store_true")
    ap.add_argument("--eager", action="store_true", help="time eager launches instead of a HIP graph replay")
    ap.add_argument("--layout", choices=("auto", "nhwc", "nchw"), default="auto",
                    help="activation layout between layers (the image and the yolo heads stay NCHW); auto: "
                         "channels-last from batch 2 up, NCHW at batch 1")
    ap.add_argument("--no-extras", action="store_true",
                    help="skip the other BASELINE configurations (single conv, SGEMM sweep, training step, "
                         "YOLOv3-608 batch 32)")
    ap.add_argument("--counter-pass", action="store_true",
                    help="for rocprofv3 --pmc: tune, then run ONE eager forward and a 64 MiB copy "
                         "(the calibration kernel), print nothing else")
    args = ap.parse_args()
    LAYOUT[0] = args.layout
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU only (the YOLOv3 inference path shards by image "
              "with no communication, one process per GPU). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    from tensorium_amd import darknet, synth
    from tensorium_amd.nnhip import TNNHip

    hip = TNNHip(0)
    hip.useTorchStream()  # one ordered stream for torch's buffers and the kernels
    _, layers = darknet.load_cfg("yolov3.cfg", args.size, args.size)
    if args.weights:
        from tensorium_amd import weights as WT

        weights = WT.load_weights(args.weights, layers)
    else:
        weights = darknet.synthetic_weights(layers)
    flop_img = darknet.conv_flops(layers)

    if args.counter_pass:
        counter_pass(hip, darknet.Network(hip, layers, args.batch, weights, layout=layout_for(args.batch)), args)
        return

    def run(batch, steps, warmup):
        net = darknet.Network(hip, layers, batch, weights, layout=layout_for(batch))
        x = torch.from_numpy(synth.uniform(7, (batch, 3, args.size, args.size))).cuda()
        torch.cuda.synchronize()
        ms, wall = time_forward(hip, net, x, steps, warmup, graph=not args.eager)
        return net, x, ms, wall

    net, x, ms, wall = run(args.batch, args.steps, args.warmup)
    ms_step = ms / args.steps
    img_s = args.batch * args.steps / (ms / 1e3)
    gflops = flop_img * args.batch / (ms_step / 1e3) / 1e9
    log(f"batch {args.batch}: {ms_step:.3f} ms/step (event), wall {wall / args.steps * 1e3:.3f} ms/step, "
        f"{img_s:.1f} img/s, {gflops:.0f} GFLOP/s")

    stats = profile_kernels(hip, net, layers, x)
    conv_kinds = [k for k in stats if k.startswith("conv")]
    dom = max(conv_kinds, key=lambda k: stats[k]["ms"])
    d = stats[dom]
    achieved = d["flop"] / (d["ms"] / 1e3)
    for k, s in sorted(stats.items(), key=lambda kv: -kv[1]["ms"]):
        log(f"  {k}: {s['ms']:.3f} ms over {s['launches']:.0f} launches, "
            f"{s['flop'] / (s['ms'] / 1e3) / 1e12:.1f} TFLOP/s")
    conv_ms = sum(stats[k]["ms"] for k in conv_kinds)
    del net, x
    torch.cuda.empty_cache()

    b1 = None
    if not args.no_batch1 and args.batch != 1:
        _, _, ms1, _ = run(1, max(args.steps, 20), args.warmup)
        b1 = 1 * max(args.steps, 20) / (ms1 / 1e3)
        log(f"batch 1: {ms1 / max(args.steps, 20):.3f} ms/img, {b1:.1f} img/s")

    cpu = None
    if not args.no_cpu_baseline:
        v, threads, n = cpu_baseline(layers, weights, args.cpu_budget)
        cpu = {"value": round(v, 4), "unit": "img/s", "cores": threads, "kind": "port",
               "sample": f"YOLOv3-416 batch-1 forward x{n} on the CPU oracle (C AVX2+FMA restatement of the "
                         f"reference path, {threads} threads, BN folded)"}
        log(f"cpu baseline: {v:.3f} img/s on {threads} threads")

    extras = None
    if not args.no_extras:
        extras = {}

        def guarded(name, fn):
            try:
                extras[name] = fn()
                log(f"{name}: {extras[name]}")
            except Exception as e:  # an extra must not hide the headline figure
                extras[name] = {"error": f"{type(e).__name__}: {e}"}
                log(f"{name} failed: {e}")
            torch.cuda.synchronize()
            torch.cuda.empty_cache()

        guarded("single_conv_416", lambda: extra_single_conv(hip))
        guarded("sgemm", lambda: extra_sgemm(hip))
        guarded("train_cifar_b128", lambda: extra_train(hip, 50, 2, 0 if args.no_cpu_baseline else 2))
        _, l608 = darknet.load_cfg("yolov3.cfg", 608, 608)
        guarded("yolov3_608_b32", lambda: extra_yolo(hip, l608, weights, 5, 2))
        guarded("yolo_detect_nms_b16", lambda: extra_detect(hip, layers, weights))

    out = {
        "metric": METRIC,
        "value": round(img_s, 2),
        "unit": "img/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "launch": "eager" if args.eager else "hip_graph",
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": ("synthetic (seeded splitmix64 U[0,1) images, He-normal random weights, BN folded)" if not args.weights
                 else f"synthetic images, weights from {os.path.basename(args.weights)} (BN folded)"),
        "config": {"workload": f"YOLOv3-{args.size} fp32 inference, batch {args.batch}, 1 GPU",
                   "global_batch": args.batch, "image": [3, args.size, args.size],
                   "activation_layout": layout_for(args.batch)},
        "conv_gflops": round(gflops, 1),
        "conv_frac_fp32_mfma_peak": round(gflops * 1e9 / PEAK_FP32_MFMA, 4),
        "conv_kernel_ms_per_step": round(conv_ms, 4),
        "img_s_batch1": None if b1 is None else round(b1, 2),
        "roofline": {"bound": "mfma", "kernel": dom, "achieved": round(achieved / 1e12, 3),
                     "peak": PEAK_FP32_MFMA / 1e12, "unit": "TFLOP/s",
                     "frac": round(achieved / PEAK_FP32_MFMA, 4),
                     "traffic": (round(TRAFFIC_TAP3X3_B16[dom]) if dom in TRAFFIC_TAP3X3_B16 and args.batch == 16
                                 and args.size == 416 else None),
                     "traffic_unit": "bytes/launch",
                     "launches_per_step": round(d["launches"]),
                     "flop_per_launch": round(d["flop"] / max(d["launches"], 1))},
        "cpu_baseline": cpu,
        "other_configs": extras,
    }
    print(json.dumps(out), flush=True)
    del np


if __name__ == "__main__":
    main()
