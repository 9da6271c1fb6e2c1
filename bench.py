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
    """--layout auto: channels-last between layers at every batch size
    (measured faster at batch 1, 4 and 16; at batch 1 through the wave-split
    tiles, 1.19 against 1.35 ms for NCHW)."""
    if LAYOUT[0] != "auto":
        return LAYOUT[0]
    return "nhwc"
PEAK_HBM = 8.0e12
# HBM bytes per launch of the dominant kernel family at batch 16 (tap-major
# 3x3 conv, channels-last conv_nhwc_kernel, incl. its in-kernel tail sums) from two
# rocprofv3 --pmc runs of `bench.py --counter-pass` (FETCH_SIZE then
# WRITE_SIZE, KiB per dispatch, scaled by a 64 MiB copy: read = 2.0 x
# FETCH_SIZE, write = 1.0 x WRITE_SIZE); profiles/yolov3_416_b16_conv_nhwc_kernel.md
# holds the figures and the commands.  Other layouts / batches: null.
TRAFFIC_TAP3X3_B16 = {"conv_nhwc_kernel<tap3x3>": (2.0 * 93274.8 + 53472.5) * 1024}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def kernel_kind(L, batch, layout):
    """Kernel family of a conv layer, by layer shape: the implicit GEMM over
    tap-major 3x3 or 1x1 operands (named after the lean kernel,
    conv_nhwc_kernel for channels-last activations, conv_lean_kernel for
    NCHW, conv_lean.hpp; the tuner may run a layer of the family with the
    wave-split tiles, conv_wsplit.hip), or the first layer over few input
    channels (conv_first.hip / conv_smallc_kernel)."""
    lean = "conv_nhwc_kernel" if layout == "nhwc" else "conv_lean_kernel"
    if L["size"] == 1 and L["stride"] == 1 and L["pad"] == 0:
        return f"{lean}<1x1>"
    if L["size"] == 3 and L["in"][0] <= 4:
        return "first_layer<3x3>"  # conv_first_mfma_kernel (channels-last from 262K pixels) or conv_smallc_kernel
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


CPU_SHARE = 16  # host CPUs the GPU pool grants one GPU's jobs (worker pools are sized to it)


def host_cpus():
    """What the host offers the CPU baseline: nproc (online CPUs), the CPUs
    this process may run on (affinity, cut by a cgroup CPU quota), and the
    CPU model name (lscpu's "Model name", read from /proc/cpuinfo)."""
    nproc = os.cpu_count() or 1
    try:
        avail = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        avail = nproc
    try:
        quota, period = open("/sys/fs/cgroup/cpu.max").read().split()[:2]
        if quota != "max":
            avail = min(avail, max(1, int(int(quota) // int(period))))
    except (OSError, ValueError):
        pass
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return nproc, avail, model


def baseline_threads():
    """P of the reference's worker pool: GetSystemThreadCount =
    max(TThread.ProcessorCount, 4) (steroids.pas:281-296), with the processor
    count taken as the CPUs this process may use, bounded by the pool's
    per-GPU share (threads beyond the CPUs available only time-slice)."""
    nproc, avail, model = host_cpus()
    return max(min(avail, CPU_SHARE), 4), nproc, avail, model


HEADS = (81, 93, 105)  # the pre-logistic head convolutions (darknet layer indices)
PARITY_TOL = 1e-5  # per tensor: max|gpu - oracle| / max|oracle|


def cpu_baseline(layers, weights, budget_s=12.0, size=416):
    """Oracle YOLOv3-416 forward at batch 1 on the host cores, repeated until
    ~budget_s of work, on image 0 of the timed batch (synth.uniform(7) draws
    the batch image by image, so its first 3x416x416 values are this image);
    returns (img/s, threads, images, host description, the oracle's head
    convolutions of that image)."""
    import numpy as np

    from oracle import netref
    from oracle import refcpu as R
    from tensorium_amd import synth

    threads, nproc, avail, model = baseline_threads()
    R.set_threads(threads)
    x = synth.uniform(7, (1, 3, size, size))
    outs = netref.forward(layers, weights, x)  # warm-up
    heads = {i: outs[i] for i in HEADS}
    del outs
    n, t0 = 0, time.perf_counter()
    while True:
        netref.forward(layers, weights, x)
        n += 1
        if time.perf_counter() - t0 >= budget_s:
            break
    dt = time.perf_counter() - t0
    del np
    return n / dt, threads, n, {"nproc": nproc, "cpus_available": avail, "cpu_model": model, "P": threads}, heads


def head_parity(gpu_heads, ref_heads):
    """Per-tensor relative error (max|g - r| / max|r|) of the timed network's
    head convolutions for image 0 against the CPU oracle's forward of the
    same image."""
    from oracle import refcpu as R

    errs = {f"head{i}": float(R.rel_err(gpu_heads[i], ref_heads[i])) for i in HEADS}
    worst = max(errs.values())
    return {**{k: float(f"{v:.3e}") for k, v in errs.items()}, "tolerance": PARITY_TOL,
            "pass": bool(worst <= PARITY_TOL), "image": 0,
            "against": "CPU oracle forward of the same image (batch 1, per-image route concat)",
            "metric": "max|gpu - oracle| / max|oracle| per head tensor (pre-logistic conv output)"}


def cpu_timed(fn, budget_s):
    """Calls fn() once to warm up, then until ~budget_s have passed; returns
    (seconds per call, calls)."""
    fn()
    n, t0 = 0, time.perf_counter()
    while True:
        fn()
        n += 1
        if time.perf_counter() - t0 >= budget_s:
            break
    return (time.perf_counter() - t0) / n, n


def cpu_info(threads):
    _, nproc, avail, model = baseline_threads()
    return {"cores": threads, "kind": "port", "nproc": nproc, "cpus_available": avail, "cpu_model": model,
            "P": threads}


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


def extra_single_conv(hip, cpu_budget=0.0):
    """Config 1: one conv layer forward, batch 1, 3x416x416 -> 16 filters 3x3
    s1 p1, weights N(0, 0.05), bias 0, leaky 0.1 (GEMM M=16, N=173056, K=27);
    with cpu_budget > 0 the CPU oracle's forward of the same layer (im2col,
    sgemm, bias, leaky) timed beside it."""
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
    eager = time_events(hip, fn, 50)
    ms = time_graph(hip, fn, 50)
    flop = 2.0 * 16 * 27 * 416 * 416
    byts = 4.0 * (3 * 416 * 416 + 16 * 416 * 416 + 16 * 27)
    # floors at this size, timed the same way: writing the 11.1 MB output
    # alone (a fill) and moving the layer's bytes as one copy of that size
    nout = 16 * 416 * 416
    fill_ms = time_graph(hip, lambda: hip.fill(nout, out, 0, 0.5, 1), 50)
    half = int(byts / 8)  # floats read = floats written = the layer's bytes / 2
    src = torch.empty(half, dtype=torch.float32, device="cuda")
    dst = torch.empty(half, dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    copy_ms = time_graph(hip, lambda: hip.copy(half, src, 0, 1, dst, 0, 1), 50)
    out = {"workload": "conv 3->16 3x3 s1 p1 + bias + leaky, 1x3x416x416", "launch": "hip_graph",
           "us": round(ms * 1e3, 2), "us_eager": round(eager * 1e3, 2),
           "gflops": round(flop / ms / 1e6, 1), "gb_s": round(byts / ms / 1e6, 1),
           "hbm_frac": round(byts / ms * 1e3 / PEAK_HBM, 4),
           "floor": {"fill_output_us": round(fill_ms * 1e3, 2), "copy_same_bytes_us": round(copy_ms * 1e3, 2),
                     "conv_over_copy": round(ms / copy_ms, 3),
                     "note": "one launch of this size, graph-timed like the conv: the output fill alone, and a "
                             "device copy moving the layer's algorithmic bytes (half read, half written)"}}
    del src, dst
    if cpu_budget > 0:
        from oracle import refcpu as R
        from tensorium_amd import synth as S
        from tensorium_amd.nnhip import acLEAKY as LK

        threads = baseline_threads()[0]
        R.set_threads(threads)
        xh, wh = S.uniform(1, (1, 3, 416, 416)), S.normal(2, (16, 27), 0.05)
        bh = np.zeros(16, np.float32)
        sec, n = cpu_timed(lambda: R.conv_forward(xh, wh, bh, 3, 1, 1, LK), cpu_budget)
        out["cpu_baseline"] = {"value": round(sec * 1e6, 1), "unit": "us/layer", "gflops": round(flop / sec / 1e9, 2),
                               "sample": f"the same layer x{n} on the CPU oracle (im2col + AVX2 sgemm + bias + leaky)",
                               **cpu_info(threads)}
    del np
    return out


SGEMM_SQUARES = (512, 1024, 2048, 4096, 8192)
# the conv-shaped skinny GEMMs of config 2: M = F, N = OH*OW*16, K = 9*C
SGEMM_SKINNY = ((64, 692224, 288), (128, 173056, 576), (256, 43264, 1152), (512, 10816, 2304),
                (1024, 2704, 4608))


def extra_sgemm(hip, cpu_budget=0.0):
    """Config 2: C = alpha*op(A)*op(B) + beta*C with A and B ~ U[-1, 1):
    the four NN/NT/TN/TT variants at M = N = K in 512 .. 8192 (beta 0), the
    conv-shaped skinny GEMMs (NN, beta 0) and one alpha = 0.5 / beta = 1 run
    at 4096^3, each timed as a graph replay after the first (tuning) call.
    Operands are cut from one seeded U[-1, 1) pool of 2^26 floats (copied
    on the device where a matrix is larger)."""
    import numpy as np
    import torch

    from tensorium_amd import synth

    pool = torch.from_numpy(synth.uniform(11, (1 << 26,), -1, 1)).cuda()

    def operand(n):
        t = torch.empty(n, dtype=torch.float32, device="cuda")
        for o in range(0, n, pool.numel()):
            k = min(pool.numel(), n - o)
            t[o:o + k].copy_(pool[:k])
        return t

    cases = [(v, n, n, n, 1.0, 0.0) for n in SGEMM_SQUARES for v in ("NN", "NT", "TN", "TT")]
    cases += [("NN", M, N, K, 1.0, 0.0) for M, N, K in SGEMM_SKINNY]
    cases += [("NN", 4096, 4096, 4096, 0.5, 1.0)]
    res = []
    bufs = {}
    for var, M, N, K, alpha, beta in cases:
        ta, tb = var[0] == "T", var[1] == "T"
        key = (M, N, K)
        if key not in bufs:
            bufs.clear()
            torch.cuda.empty_cache()
            bufs[key] = (operand(M * K), operand(K * N), operand(M * N))
        A, B, C = bufs[key]
        torch.cuda.synchronize()
        lda, ldb = (M if ta else K), (K if tb else N)

        def fn():
            hip.gemm(ta, tb, M, N, K, alpha, A, 0, lda, B, 0, ldb, beta, C, 0, N)

        fn()
        reps = 3 if M * N * K >= 8192 ** 3 else (10 if M * N * K >= 1024 ** 3 else 50)
        ms = time_graph(hip, fn, reps)
        r = {"variant": var, "M": M, "N": N, "K": K, "ms": round(ms, 4),
             "tflops": round(2.0 * M * N * K / ms / 1e9, 2),
             "frac": round(2.0 * M * N * K / ms * 1e3 / PEAK_FP32_MFMA, 4)}
        if alpha != 1.0 or beta != 0.0:
            r.update(alpha=alpha, beta=beta)
        res.append(r)
    bufs.clear()
    del pool
    torch.cuda.empty_cache()
    if cpu_budget <= 0:
        return res
    # the CPU oracle's sgemm (saxpy_avx2 row workers, rows chunked over P
    # threads) on a row sample of the 4096^3 NN product: every row of C is
    # the same work, so the sample's rate is the whole product's rate
    from oracle import refcpu as R

    threads = baseline_threads()[0]
    R.set_threads(threads)
    n, rows = 4096, 4 * threads
    A = synth.uniform(11, (rows, n), -1, 1)
    Bm = synth.uniform(12, (n, n), -1, 1)
    Cm = np.zeros((rows, n), np.float32)
    sec, calls = cpu_timed(lambda: R.sgemm(0, 0, rows, n, n, 1.0, A, n, Bm, n, 0.0, Cm, n), cpu_budget)
    gf = 2.0 * rows * n * n / sec / 1e9
    cpu = {"value": round(gf, 2), "unit": "GFLOP/s", "full_gemm_s": round(2.0 * n ** 3 / (gf * 1e9), 2),
           "sample": f"NN sgemm, {rows} of 4096 rows of A (M={rows}, N=K=4096) x{calls} on the CPU oracle; "
                     "full_gemm_s = the 4096^3 product at that rate (rows are independent and equal work)",
           **cpu_info(threads)}
    return {"cases": res, "cpu_baseline": cpu}


def extra_train(hip, steps, warmup, cpu_steps):
    """Config 3: one training step (forward + backward + SGD update) of the
    conv-BN-leaky x3 / pool / connected / softmax-CE network on synthetic
    3x32x32 U[0,1) images with one-hot labels, batch 128, replayed from a HIP
    graph; the CPU oracle's step timed beside it."""
    import numpy as np

    from tensorium_amd import synth, trainnet
    from tensorium_amd.nnhip import DeviceArray

    B = 128
    x = synth.uniform(21, (B, 3, 32, 32))
    lab = (synth.splitmix64(22, B) % np.uint64(10)).astype(np.int64)
    truth = np.zeros((B, 10), np.float32)
    truth[np.arange(B), lab] = 1
    params = trainnet.init_params()
    tr = trainnet.CifarTrainer(hip, params, B)
    # the trainer and its inputs on the library's own memory (no torch)
    dx, dt = DeviceArray.from_numpy(x), DeviceArray.from_numpy(truth)
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

        threads, nproc, avail, model = baseline_threads()
        R.set_threads(threads)
        ref = T.CifarStep(params, form="avx2")  # the reference's routines on an AVX2 host
        ref.step(x, truth)
        t0 = time.perf_counter()
        for _ in range(cpu_steps):
            ref.step(x, truth)
        cms = (time.perf_counter() - t0) / cpu_steps * 1e3
        out["cpu_baseline"] = {"value": round(cms, 1), "unit": "ms/step", "cores": R.get_threads(), "kind": "port",
                               "sample": f"{cpu_steps} oracle steps (C restatement: AVX2 GEMM, im2col/col2im, the AVX2 host's "
                                         "batch-norm reductions, softmax)",
                               "nproc": nproc, "cpus_available": avail, "cpu_model": model, "P": threads}
    return out


def extra_yolo(hip, layers608, weights608, steps, warmup, batch=32, size=608, name="YOLOv3", cpu_budget=0.0):
    """Config 5: YOLOv3-608 inference at batch 32 (HIP graph replay); also
    YOLOv3-tiny-416 at batch 16 (channels-last with maxpools and a
    16-channel convolution input).  With cpu_budget > 0 the CPU oracle's
    forward of image 0 (batch 1) is timed beside it."""
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
    out = {"workload": f"{name}-{size} fp32 inference, batch {batch}", "ms_per_step": round(ms, 3),
           "img_s": round(batch / ms * 1e3, 1), "conv_frac_fp32_mfma_peak": round(flop / ms * 1e3 / PEAK_FP32_MFMA, 4)}
    if cpu_budget > 0:
        from oracle import netref
        from oracle import refcpu as R

        threads = baseline_threads()[0]
        R.set_threads(threads)
        x1 = synth.uniform(9, (1, 3, size, size))
        sec, n = cpu_timed(lambda: netref.forward(layers608, weights608, x1), cpu_budget)
        out["cpu_baseline"] = {"value": round(1.0 / sec, 4), "unit": "img/s",
                               "sample": f"{name}-{size} batch-1 forward (image 0 of the batch) x{n} on the CPU "
                                         "oracle, BN folded; measured at batch 1, not extrapolated",
                               **cpu_info(threads)}
    return out


def extra_batch1(hip, layers, weights, steps, warmup):
    """YOLOv3-416 at batch 1 (the other half of the metric), HIP graph replay."""
    import torch

    from tensorium_amd import darknet, synth

    net = darknet.Network(hip, layers, 1, weights, layout=layout_for(1))
    x = torch.from_numpy(synth.uniform(7, (1, 3, 416, 416))).cuda()
    torch.cuda.synchronize()
    ms, _ = time_forward(hip, net, x, steps, warmup, graph=True)
    ms /= steps
    flop = darknet.conv_flops(layers)
    del net, x
    torch.cuda.empty_cache()
    return {"workload": "YOLOv3-416 fp32 inference, batch 1", "ms_per_step": round(ms, 4),
            "img_s": round(1e3 / ms, 2), "conv_frac_fp32_mfma_peak": round(flop / ms * 1e3 / PEAK_FP32_MFMA, 4)}


def extra_dropin(hip, layers, weights, steps, warmup, batch=16):
    """YOLOv3-416 at batch 16 through the per-layer calls a Tensorium build
    with the USE_HIP branches makes (TConvolutionalLayer.forwardGPU and the
    shortcut, route, upsample and yolo GPU hooks): NCHW activations, one
    tnh_conv2d_fwd per convolution with bias and activation fused, and a
    separate launch for every shortcut (addvv), route copy, upsample and yolo
    layer.  Three weight arrangements, each as a HIP graph replay:
      reference_layout  the layer's weights as stored ([F][C][k][k],
                        TNH_WEIGHTS_REFERENCE), as forwardGPU passes them;
      packed_in_layer   a tap-major copy the layer packs once after
                        fuseBatchNorm / each update (TNH_WEIGHTS_TAP_MAJOR);
      packed_fused      the same with each shortcut folded into the preceding
                        convolution's epilogue (darknet.Network's NCHW plan)."""
    import torch

    from tensorium_amd import darknet, synth

    x = torch.from_numpy(synth.uniform(7, (batch, 3, 416, 416))).cuda()
    flop = darknet.conv_flops(layers) * batch
    out = {"workload": f"YOLOv3-416 fp32 inference, batch {batch}, NCHW, per-layer TNNHip calls"}
    for name, fuse, pack in (("reference_layout", False, False), ("packed_in_layer", False, True),
                             ("packed_fused", True, True)):
        net = darknet.Network(hip, layers, batch, weights, fuse=fuse, pack=pack, layout="nchw")
        torch.cuda.synchronize()
        ms, _ = time_forward(hip, net, x, steps, warmup, graph=True)
        ms /= steps
        out[name] = {"ms_per_step": round(ms, 3), "img_s": round(batch / ms * 1e3, 1),
                     "conv_frac_fp32_mfma_peak": round(flop / ms * 1e3 / PEAK_FP32_MFMA, 4)}
        del net
        torch.cuda.empty_cache()
    del x
    return out


def _bw_entry(name, ms, byts, copy_gbs):
    gbs = byts / ms / 1e6
    return {"kernel": name, "us": round(ms * 1e3, 2), "bytes": int(byts), "gb_s": round(gbs, 1),
            "hbm_frac": round(gbs * 1e9 / PEAK_HBM, 4),
            "copy_frac": None if copy_gbs is None else round(gbs / copy_gbs, 4)}


def extra_bandwidth(hip):
    """The memory-bound kernels of the path at config-3 and YOLOv3 sizes, each
    timed as a graph replay: achieved GB/s of the algorithmic bytes
    (compulsory fp32 reads + writes, 8-byte indices) against the 8 TB/s
    datasheet peak and against a plain device copy measured in the same run."""
    import torch

    from tensorium_amd import synth
    from tensorium_amd.nnhip import acLEAKY

    def dev(shape, seed, dtype=torch.float32):
        t = torch.from_numpy(synth.uniform(seed, shape, -1, 1)).cuda()
        return t if dtype == torch.float32 else t.to(dtype)

    out = []
    n = 64 << 20  # floats: a 256 MiB copy
    src, dst = dev((n,), 1), torch.empty(n, dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    ms = time_graph(hip, lambda: hip.copy(n, src, 0, 1, dst, 0, 1), 20)
    copy_gbs = 8.0 * n / ms / 1e6
    out.append(_bw_entry("copy 256 MiB", ms, 8.0 * n, None))
    # writes only: the bound of a store-dominated kernel (the first conv layer)
    ms = time_graph(hip, lambda: hip.fill(n, dst, 0, 0.5, 1), 20)
    out.append(_bw_entry("fill 256 MiB (writes only)", ms, 4.0 * n, copy_gbs))
    del src, dst

    def im2col_case(label, B, C, H, k, p, s):
        OH = (H + 2 * p - k) // s + 1
        x = dev((B, C, H, H), 2)
        col = torch.empty(B * C * k * k * OH * OH, dtype=torch.float32, device="cuda")
        torch.cuda.synchronize()
        t = time_graph(hip, lambda: hip.im2colStridedBatched(C, H, H, k, k, p, p, s, s, 1, 1, x, C * H * H, 0, col,
                                                             C * k * k * OH * OH, 0, B), 20)
        out.append(_bw_entry(f"im2col {label} B{B} C{C} {H}x{H} k{k}", t,
                             4.0 * B * (C * H * H + C * k * k * OH * OH), copy_gbs))
        t = time_graph(hip, lambda: hip.col2imStridedBatched(C, H, H, k, k, p, p, s, s, 1, 1, col,
                                                             C * k * k * OH * OH, 0, x, C * H * H, 0, B), 20)
        out.append(_bw_entry(f"col2im {label} B{B} C{C} {H}x{H} k{k}", t,
                             4.0 * B * (C * k * k * OH * OH + 2 * C * H * H), copy_gbs))

    im2col_case("config-3 conv2", 128, 32, 16, 3, 1, 1)
    im2col_case("config-3 conv3", 128, 64, 8, 3, 1, 1)
    im2col_case("yolov3 52x52", 16, 128, 52, 3, 1, 1)

    def pool_case(label, B, C, H):
        OH = H // 2
        x = dev((B, C, H, H), 3)
        y = torch.empty((B, C, OH, OH), dtype=torch.float32, device="cuda")
        idx = torch.empty((B, C, OH, OH), dtype=torch.int64, device="cuda")
        dIn = torch.zeros((B, C, H, H), dtype=torch.float32, device="cuda")
        torch.cuda.synchronize()
        t = time_graph(hip, lambda: hip.forwardMaxPool(B, C, OH, OH, x, C, H, H, 2, 2, 0, 2, idx, y), 20)
        out.append(_bw_entry(f"maxpool fwd {label} B{B} C{C} {H}x{H} 2/2 +idx", t,
                             4.0 * B * C * (H * H + OH * OH) + 8.0 * B * C * OH * OH, copy_gbs))
        t = time_graph(hip, lambda: hip.backwardMaxPool(B, C, OH, OH, dIn, idx, y), 20)
        # dOut + indices read, and the touched (one per window) dIn elements read and written
        out.append(_bw_entry(f"maxpool bwd {label} B{B} C{C} {H}x{H} 2/2", t,
                             (4.0 + 8.0 + 8.0) * B * C * OH * OH, copy_gbs))

    pool_case("config-3 pool1", 128, 32, 32)
    pool_case("config-3 pool2", 128, 64, 16)

    def up_case(label, B, C, H):
        x = dev((B, C, H, H), 4)
        y = torch.empty((B, C, 2 * H, 2 * H), dtype=torch.float32, device="cuda")
        torch.cuda.synchronize()
        t = time_graph(hip, lambda: hip.upSample(B, C, H, H, x, 2, 1, 1.0, y), 20)
        out.append(_bw_entry(f"upsample fwd {label} B{B} C{C} {H}->{2 * H}", t, 4.0 * B * C * H * H * 5, copy_gbs))

    up_case("yolov3-416 first", 16, 256, 13)
    up_case("yolov3-416 second", 16, 128, 26)

    B, F, Hh = 128, 32, 32
    nel = B * F * Hh * Hh
    y = dev((B, F, Hh, Hh), 5)
    b = dev((F,), 6)
    torch.cuda.synchronize()

    def bias_leaky():
        hip.forwardBias(nel, y, 0, F, b, 1, B)
        hip.ActivateArray(nel, y, 0, acLEAKY)

    t = time_graph(hip, bias_leaky, 20)
    out.append(_bw_entry(f"bias + leaky (unfused, 2 passes) B{B} C{F} {Hh}x{Hh}", t, 2 * 8.0 * nel, copy_gbs))
    del y, b
    torch.cuda.empty_cache()
    return {"copy_gb_s": round(copy_gbs, 1), "kernels": out}


# YOLOv3-416 layer shapes at batch 16 (label, C, H, F, k, stride)
IM2COL_VS_FUSED = (("416->208 3x3 s2", 32, 416, 64, 3, 2), ("104x104 3x3", 64, 104, 128, 3, 1),
                   ("52x52 3x3", 128, 52, 256, 3, 1), ("26x26 3x3", 256, 26, 512, 3, 1),
                   ("13x13 3x3", 512, 13, 1024, 3, 1), ("52x52 1x1", 256, 52, 128, 1, 1))


def extra_im2col_vs_fused(hip, batch=16):
    """The two ways to run a conv layer on the GPU, on YOLOv3-416 layer shapes
    at batch 16 (NCHW, leaky): (a) the sequence of TConvolutionalLayer's GPU
    forward (nConvolutionLayer.pas:1047-1097) as separate launches -- im2col
    of every image into a materialised column matrix (one batched launch
    here; a 1x1 stride-1 layer skips it and reads the input directly), one
    gemmStridedBatched W x col_b, forwardBias, then the activation -- and (b)
    the implicit-GEMM conv (tnh_conv2d_fwd: the gather inside the GEMM's
    operand loader, bias and leaky in its epilogue).  Each is timed as a
    graph replay after an eager (tuning) call."""
    import torch

    from tensorium_amd import synth
    from tensorium_amd.nnhip import WEIGHTS_TAP_MAJOR, acLEAKY

    out = []
    for label, C, H, F, k, s in IM2COL_VS_FUSED:
        p = k // 2
        OH = (H + 2 * p - k) // s + 1
        HW, K = OH * OH, C * k * k
        x = torch.from_numpy(synth.uniform(11, (batch, C, H, H))).cuda()
        w = torch.from_numpy(synth.normal(12, (F, K), (2.0 / K) ** 0.5)).cuda()
        wt = torch.empty_like(w)
        hip.packConvWeights(F, C, k, w, wt)
        b = torch.from_numpy(synth.normal(13, (F,), 0.1)).cuda()
        y = torch.empty((batch, F, OH, OH), dtype=torch.float32, device="cuda")
        col = torch.empty(batch * K * HW, dtype=torch.float32, device="cuda") if k > 1 else None
        torch.cuda.synchronize()

        def fused():
            hip.conv2dForward(batch, C, H, H, F, k, s, p, x, 0, wt if k > 1 else w, b, acLEAKY, y, 0,
                              weightLayout=WEIGHTS_TAP_MAJOR if k > 1 else 0)

        def im2col():
            hip.im2colStridedBatched(C, H, H, k, k, p, p, s, s, 1, 1, x, C * H * H, 0, col, K * HW, 0, batch)

        def gemm():
            src, stride = (col, K * HW) if k > 1 else (x, C * H * H)
            hip.gemmStridedBatched(False, False, F, HW, K, 1.0, w, 0, K, 0, src, 0, HW, stride, 0.0, y, 0, HW,
                                   F * HW, batch)

        def epilogue():
            hip.forwardBias(batch * F * HW, y, 0, F, b, 1, batch)
            hip.ActivateArray(batch * F * HW, y, 0, acLEAKY)

        def sequence():
            if k > 1:
                im2col()
            gemm()
            epilogue()

        for f in (fused, sequence):
            f()
        t_fused = time_graph(hip, fused, 10)
        t_seq = time_graph(hip, sequence, 10)
        t_i2c = time_graph(hip, im2col, 10) if k > 1 else 0.0
        t_gemm = time_graph(hip, gemm, 10)
        t_epi = time_graph(hip, epilogue, 10)
        flop = 2.0 * batch * F * HW * K
        out.append({"layer": f"{label} C{C}->F{F} B{batch}", "fused_us": round(t_fused * 1e3, 1),
                    "sequence_us": round(t_seq * 1e3, 1), "im2col_us": round(t_i2c * 1e3, 1),
                    "gemm_us": round(t_gemm * 1e3, 1), "bias_act_us": round(t_epi * 1e3, 1),
                    "fused_tflops": round(flop / t_fused / 1e9, 1), "speedup": round(t_seq / t_fused, 3)})
        del x, w, wt, b, y, col
        torch.cuda.empty_cache()
    return {"workload": "YOLOv3-416 conv layers at batch 16, NCHW: implicit GEMM against im2col + SGEMM + "
                        "bias + leaky", "layers": out}


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
    ap.add_argument("--deterministic", action="store_true",
                    help="tnh_set_deterministic(1): every conv and SGEMM shape takes a fixed tiling with no split-K "
                         "or tail split, so results do not depend on what the autotuner timed")
    ap.add_argument("--layout", choices=("auto", "nhwc", "nchw"), default="auto",
                    help="activation layout between layers (the image and the yolo heads stay NCHW); auto: "
                         "channels-last")
    ap.add_argument("--no-extras", action="store_true",
                    help="skip the other BASELINE configurations (single conv, SGEMM sweep, training step, "
                         "YOLOv3-608 batch 32) and the YOLOv3-tiny / detection / bandwidth figures")
    ap.add_argument("--only", choices=("single_conv_416", "sgemm", "train_cifar_b128", "yolov3_608_b32",
                                       "yolo_detect_nms_b16", "bandwidth", "batch1", "yolov3_tiny_416_b16",
                                       "im2col_vs_fused", "yolov3_416_b16_dropin"),
                    default=None,
                    help="run one secondary configuration alone and print its figures (for profiling runs)")
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
    from tensorium_amd.nnhip import DeviceArray, TNNHip

    hip = TNNHip(0)
    hip.useTorchStream()  # one ordered stream for torch's buffers and the kernels
    if args.deterministic:
        TNNHip.setDeterministic(True)
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
    if args.only:
        tiny = darknet.load_cfg("yolov3-tiny.cfg")[1]
        only = {
            "single_conv_416": lambda: extra_single_conv(hip),
            "sgemm": lambda: extra_sgemm(hip),
            "train_cifar_b128": lambda: extra_train(hip, args.steps, args.warmup, 0),
            "yolov3_608_b32": lambda: extra_yolo(hip, darknet.load_cfg("yolov3.cfg", 608, 608)[1], weights,
                                                 args.steps, args.warmup),
            "yolo_detect_nms_b16": lambda: extra_detect(hip, layers, weights),
            "bandwidth": lambda: extra_bandwidth(hip),
            "im2col_vs_fused": lambda: extra_im2col_vs_fused(hip),
            "yolov3_416_b16_dropin": lambda: extra_dropin(hip, layers, weights, args.steps, args.warmup),
            "batch1": lambda: extra_batch1(hip, layers, weights, args.steps, args.warmup),
            "yolov3_tiny_416_b16": lambda: extra_yolo(hip, tiny, darknet.synthetic_weights(tiny), args.steps,
                                                      args.warmup, batch=16, size=416, name="YOLOv3-tiny"),
        }[args.only]
        print(json.dumps({args.only: only()}), flush=True)
        return

    def run(batch, steps, warmup):
        net = darknet.Network(hip, layers, batch, weights, layout=layout_for(batch))
        x = DeviceArray.from_numpy(synth.uniform(7, (batch, 3, args.size, args.size)))
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
    # image 0's head convolutions as the timed network computed them (the
    # profile pass above is one more eager forward of the same input)
    gpu_heads = {i: net.output(i)[0:1] for i in HEADS}
    del net, x
    torch.cuda.empty_cache()

    b1 = None
    if not args.no_batch1 and args.batch != 1:
        _, _, ms1, _ = run(1, max(args.steps, 20), args.warmup)
        b1 = 1 * max(args.steps, 20) / (ms1 / 1e3)
        log(f"batch 1: {ms1 / max(args.steps, 20):.3f} ms/img, {b1:.1f} img/s")

    cpu = None
    parity = None
    if not args.no_cpu_baseline:
        v, threads, n, hostd, ref_heads = cpu_baseline(layers, weights, args.cpu_budget, args.size)
        parity = head_parity(gpu_heads, ref_heads)
        log(f"parity (image 0 heads vs the oracle): {parity}")
        del ref_heads
        cpu = {"value": round(v, 4), "unit": "img/s", "cores": threads, "kind": "port",
               "sample": f"YOLOv3-{args.size} batch-1 forward x{n} on the CPU oracle (C AVX2+FMA restatement of the "
                         f"reference path, P = {threads} worker threads, BN folded); measured at batch 1, "
                         f"not extrapolated",
               **hostd}
        log(f"cpu baseline: {v:.3f} img/s on {threads} threads ({hostd})")

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

        cb = 0.0 if args.no_cpu_baseline else 3.0
        guarded("single_conv_416", lambda: extra_single_conv(hip, cb))
        guarded("sgemm", lambda: extra_sgemm(hip, cb))
        guarded("train_cifar_b128", lambda: extra_train(hip, 50, 2, 0 if args.no_cpu_baseline else 2))
        _, l608 = darknet.load_cfg("yolov3.cfg", 608, 608)
        guarded("yolov3_608_b32", lambda: extra_yolo(hip, l608, weights, 5, 2, cpu_budget=cb))
        _, ltiny = darknet.load_cfg("yolov3-tiny.cfg")
        guarded("yolov3_tiny_416_b16", lambda: extra_yolo(hip, ltiny, darknet.synthetic_weights(ltiny), 20, 3,
                                                          batch=16, size=416, name="YOLOv3-tiny"))
        guarded("yolo_detect_nms_b16", lambda: extra_detect(hip, layers, weights))
        guarded("bandwidth", lambda: extra_bandwidth(hip))
        guarded("im2col_vs_fused", lambda: extra_im2col_vs_fused(hip))
        guarded("yolov3_416_b16_dropin", lambda: extra_dropin(hip, layers, weights, 10, 2))

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
                   "activation_layout": layout_for(args.batch),
                   "tiling": ("deterministic (fixed tiling, no split-K or tail split)" if args.deterministic
                              else "autotuned (split-K / tail splits chosen by time; the sum order may differ "
                                   "between processes)")},
        "conv_gflops": round(gflops, 1),
        "conv_frac_fp32_mfma_peak": round(gflops * 1e9 / PEAK_FP32_MFMA, 4),
        # the per-layer event brackets of one eager pass (each includes its
        # launch gaps), summed over the conv layers: a breakdown of an eager
        # forward, not a part of ms_per_step (a graph replay)
        "conv_ms_eager_layer_events": round(conv_ms, 4),
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
        "parity": parity,
        "other_configs": extras,
    }
    print(json.dumps(out), flush=True)
    del np


if __name__ == "__main__":
    main()
