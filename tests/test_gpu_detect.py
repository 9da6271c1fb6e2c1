"""YOLO detections and NMS on the device (tnh_yolo_detections /
tnh_yolo_nms_sort) against the CPU restatement of the reference
(oracle/detref.py).  Detection order, counts, objectness and probabilities
are exact; x and y are exact float operations; w and h go through exp and
are compared within 4 ulp.  NMS runs on the oracle's own boxes and must zero
exactly the same (detection, class) probabilities."""
import numpy as np
import pytest
import torch

from oracle import detref as DR
from tensorium_amd import darknet, synth

pytestmark = pytest.mark.gpu

ANCH = [[(116, 90), (156, 198), (373, 326)], [(30, 61), (62, 45), (59, 119)], [(10, 13), (16, 30), (33, 23)]]


def random_heads(seed, B, sizes, n=3, classes=80):
    heads = []
    for s, hw in enumerate(sizes):
        x = synth.uniform(seed + s, (B, n, classes + 5, hw, hw))
        x[:, :, 2:4] = synth.normal(seed + 100 + s, (B, n, 2, hw, hw), 0.5)  # raw tw, th
        heads.append(x)
    return heads


def run_detect(hip, heads, classes, thresh, netw, neth, imgw, imgh, relative, letter, cap, nms=None):
    B = heads[0].shape[0]
    dh = [torch.from_numpy(h).cuda() for h in heads]
    boxes = torch.empty((B, cap, 4), dtype=torch.float32, device="cuda")
    obj = torch.empty((B, cap), dtype=torch.float32, device="cuda")
    prob = torch.empty((B, cap, classes), dtype=torch.float32, device="cuda")
    counts = torch.empty(B, dtype=torch.int32, device="cuda")
    torch.cuda.synchronize()
    hip.yoloDetections(B, dh, [h.shape[-2:] for h in heads], 3, classes, ANCH[:len(heads)], netw, neth, imgw, imgh,
                       thresh, relative, letter, cap, boxes, obj, prob, counts)
    if nms is not None:
        hip.yoloNmsSort(B, classes, cap, boxes, prob, counts, nms)
    hip.finish()
    torch.cuda.synchronize()
    return boxes.cpu().numpy(), obj.cpu().numpy(), prob.cpu().numpy(), counts.cpu().numpy()


def ulps(a, b):
    ia = a.view(np.int32).astype(np.int64)
    ib = b.view(np.int32).astype(np.int64)
    return np.abs(ia - ib)


@pytest.mark.parametrize("relative,letter,imgw,imgh", [(False, False, 640, 480), (True, False, 416, 416),
                                                       (False, True, 640, 480), (True, True, 500, 700)])
def test_detections_vs_oracle(hip, relative, letter, imgw, imgh):
    print(f"[case] yolo detections rel={relative} letter={letter} img={imgw}x{imgh}", flush=True)
    heads = random_heads(80, 2, (13, 26, 52))
    thresh = 0.8
    bx, ob, pr, cnt = run_detect(hip, heads, 80, thresh, 416, 416, imgw, imgh, relative, letter, 8192)
    for b in range(2):
        rb, ro, rp = DR.detections(heads, ANCH, 416, 416, imgw, imgh, thresh, relative, letter, b)
        assert cnt[b] == len(ro) > 0
        n = cnt[b]
        assert np.array_equal(ob[b, :n], ro)
        assert np.array_equal(pr[b, :n], rp)
        assert np.array_equal(bx[b, :n, :2], rb[:, :2])
        assert ulps(bx[b, :n, 2:], rb[:, 2:]).max() <= 4


def test_capacity_overflow_reports_count(hip):
    print("[case] yolo detections capacity overflow", flush=True)
    heads = random_heads(90, 1, (13,))
    bx, ob, pr, cnt = run_detect(hip, heads, 80, 0.3, 416, 416, 416, 416, False, False, 16)
    rb, ro, rp = DR.detections(heads, ANCH, 416, 416, 416, 416, 0.3, False, False, 0)
    assert cnt[0] == len(ro) > 16
    assert np.array_equal(ob[0, :16], ro[:16])  # the first capacity detections are written, in order


@pytest.mark.parametrize("thresh", [0.45, 0.3])
def test_nms_sort_vs_oracle(hip, thresh):
    """NMS on the oracle's own detection list (boxes, probabilities, counts
    uploaded), so only the suppression is compared."""
    print(f"[case] yolo nms_sort thresh {thresh}", flush=True)
    heads = random_heads(95, 2, (13, 26))
    cap, C = 4096, 80
    boxes = np.zeros((2, cap, 4), np.float32)
    prob = np.zeros((2, cap, C), np.float32)
    counts = np.zeros(2, np.int32)
    ref = []
    for b in range(2):
        rb, ro, rp = DR.detections(heads, ANCH, 416, 416, 416, 416, 0.6, False, False, b)
        n = len(ro)
        boxes[b, :n], prob[b, :n], counts[b] = rb, rp, n
        ref.append(DR.nms_sort(rb, rp.copy(), thresh))
    db, dp, dc = (torch.from_numpy(a).cuda() for a in (boxes, prob, counts))
    torch.cuda.synchronize()
    hip.yoloNmsSort(2, C, cap, db, dp, dc, thresh)
    hip.finish()
    got = dp.cpu().numpy()
    for b in range(2):
        n = counts[b]
        assert np.array_equal(got[b, :n], ref[b])
        assert (ref[b] == 0).sum() > (prob[b, :n] == 0).sum()  # the case suppresses something


def test_yolov3_detect_end_to_end(hip):
    """YOLOv3-416 forward at batch 2 then Network.detect: the device's list
    equals the oracle's list built from the device's own yolo outputs."""
    print("[case] yolov3-416 b2 forward + detect", flush=True)
    _, layers = darknet.load_cfg("yolov3.cfg")
    W = darknet.synthetic_weights(layers)
    net = darknet.Network(hip, layers, 2, W)
    x = torch.from_numpy(synth.uniform(7, (2, 3, 416, 416))).cuda()
    torch.cuda.synchronize()
    net.forward(x)
    hip.finish()
    yl = [L for L in layers if L["type"] == "yolo"]
    heads = [net.out[L["index"]].numpy().reshape((2, L["n"], L["classes"] + 5) + L["out"][1:]) for L in yl]
    anchors = [L["anchors"] for L in yl]
    dets = net.detect(thresh=0.995, nms=0.45, img_w=640, img_h=480)
    for b in range(2):
        rb, ro, rp = DR.detections(heads, anchors, 416, 416, 640, 480, 0.995, False, False, b)
        gb, go, gp = dets[b]
        assert len(go) == len(ro) > 0
        assert np.array_equal(go, ro)
        assert np.array_equal(gb[:, :2], rb[:, :2]) and ulps(gb[:, 2:], rb[:, 2:]).max() <= 4
        assert np.array_equal(gp, DR.nms_sort(gb, rp.copy(), 0.45))
