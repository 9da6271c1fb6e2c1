"""CPU restatement of the reference's YOLO detection list and NMS (TEST
INFRASTRUCTURE ONLY: the parity checker of tnh_yolo_detections /
tnh_yolo_nms_sort).

detections()  TNNet.Detections (nnet.pas:584-680) -> TYoloLayer.getDetections
              (nyololayer.pas:399-450): location outer, anchor inner; getBox
              (nyololayer.pas:105-122, new_coords = 0); correctBoxes
              (nyololayer.pas:452-498).  Float32 operations in the
              reference's order; exp is numpy's float32 exp.
nms_sort()    TDetectionsHelper.doNMSSort (ntypes.pas:1612-1649) with box_iou
              (ntypes.pas:1059-1107).  The reference orders each class with an
              unstable quicksort (ntensors.pas:2483); ties in probability are
              ordered here by detection index (the same rule the GPU uses), so
              only tie order is a choice of this restatement.

Pins (tests/test_detect_oracle.py): closed-form boxes for hand-built heads,
the letterbox correction by hand, hand-made NMS cases with known IoUs, box_iou
special cases, and agreement with an independent float64 greedy NMS on random
boxes whose IoUs keep clear of the threshold."""
import numpy as np

f32 = np.float32


def correct_params(netw, neth, imgw, imgh, letter):
    """correctBoxes' (deltaw, deltah, ratiow, ratioh) as float32 (nyololayer.pas:458-476)."""
    new_w, new_h = netw, neth
    if letter:
        if netw / imgw < neth / imgh:
            new_w, new_h = netw, (imgh * netw) // imgw
        else:
            new_h, new_w = neth, (imgw * neth) // imgh
    return f32(netw - new_w), f32(neth - new_h), f32(new_w / netw), f32(new_h / neth)


def detections(heads, anchors, netw, neth, imgw, imgh, thresh, relative=False, letter=False, b=0):
    """heads: list of float32 [B, n, classes+5, h, w] yolo outputs (after the
    logistic); anchors: per head, n (w, h) pairs.  Returns (boxes [D, 4],
    objectness [D], prob [D, classes]) for image b in detection order."""
    thresh = f32(thresh)
    dw, dh, rw, rh = correct_params(netw, neth, imgw, imgh, letter)
    boxes, objs, probs = [], [], []
    for head, anc in zip(heads, anchors):
        _, n, E, h, w = head.shape
        out = head[b]
        for i in range(h * w):
            row, col = i // w, i % w
            for a in range(n):
                o = out[a, :, row, col]
                obj = o[4]
                if not obj > thresh:
                    continue
                x = (f32(col) + o[0]) / f32(w)
                y = (f32(row) + o[1]) / f32(h)
                bw = np.exp(o[2]) * f32(anc[a][0]) / f32(netw)
                bh = np.exp(o[3]) * f32(anc[a][1]) / f32(neth)
                x = (x - dw / f32(2.0) / f32(netw)) / rw
                y = (y - dh / f32(2.0) / f32(neth)) / rh
                bw = bw * (f32(1.0) / rw)
                bh = bh * (f32(1.0) / rh)
                if not relative:
                    x, bw = x * f32(imgw), bw * f32(imgw)
                    y, bh = y * f32(imgh), bh * f32(imgh)
                p = (obj * o[5:]).astype(np.float32)
                boxes.append(np.array([x, y, bw, bh], np.float32))
                objs.append(obj)
                probs.append(np.where(p > thresh, p, f32(0)).astype(np.float32))
    C = heads[0].shape[2] - 5
    if not boxes:
        return np.zeros((0, 4), np.float32), np.zeros(0, np.float32), np.zeros((0, C), np.float32)
    return np.stack(boxes), np.array(objs, np.float32), np.stack(probs)


def _overlap(x1, w1, x2, w2):
    l1 = x1 - w1 / f32(2)
    l2 = x2 - w2 / f32(2)
    left = np.where(l1 > l2, l1, l2)
    r1 = x1 + w1 / f32(2)
    r2 = x2 + w2 / f32(2)
    right = np.where(r1 < r2, r1, r2)
    return right - left


def box_iou(a, B):
    """box_iou of box a [4] against boxes B [m, 4] in float32."""
    a = a.astype(np.float32)
    B = np.asarray(B, np.float32).reshape(-1, 4)
    w = _overlap(a[0], a[2], B[:, 0], B[:, 2])
    h = _overlap(a[1], a[3], B[:, 1], B[:, 3])
    inter = np.where((w < 0) | (h < 0), f32(0), w * h).astype(np.float32)
    uni = (a[2] * a[3] + B[:, 2] * B[:, 3] - inter).astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        iou = np.where((inter == 0) | (uni == 0), f32(0), inter / uni)
    return iou.astype(np.float32)


def nms_sort(boxes, prob, thresh):
    """doNMSSort in place on prob [D, classes]; returns prob."""
    thresh = f32(thresh)
    D, C = prob.shape
    for k in range(C):
        cand = np.nonzero(prob[:, k] != 0)[0]
        if cand.size < 2:
            continue
        order = cand[np.argsort(-prob[cand, k], kind="stable")]
        alive = np.ones(order.size, bool)
        for i in range(order.size):
            if not alive[i]:
                continue
            if i + 1 < order.size:
                iou = box_iou(boxes[order[i]], boxes[order[i + 1:]])
                alive[i + 1:] &= ~(iou > thresh)
        prob[order[~alive], k] = 0
    return prob
