"""Pins of the detection / NMS oracle (oracle/detref.py) by closed forms and an
independent implementation (CPU)."""
import numpy as np

from oracle import detref as DR


def head(h, w, n, classes, fill_obj=0.1):
    return np.full((1, n, classes + 5, h, w), 0.0, np.float32) + np.float32(fill_obj) * \
        (np.arange(classes + 5)[None, None, :, None, None] == 4)


def test_decode_closed_form():
    hd = head(2, 3, 1, 2)
    o = hd[0, 0, :, 1, 2]
    o[:] = [0.25, 0.5, 0.0, 0.0, 0.75, 0.9, 0.2]  # tx, ty, tw, th, obj, class0, class1
    boxes, obj, prob = DR.detections([hd], [[(32.0, 16.0)]], 64, 32, 640, 480, 0.5, relative=True)
    assert boxes.shape == (1, 4)
    # x = (col + tx)/w = 2.25/3, y = (row + ty)/h = 1.5/2, w = exp(0)*32/64, h = exp(0)*16/32
    assert boxes[0].tolist() == [0.75, 0.75, 0.5, 0.5]
    assert obj[0] == np.float32(0.75)
    assert prob[0, 0] == np.float32(0.75) * np.float32(0.9) and prob[0, 1] == 0  # 0.15 is below thresh
    abs_boxes, _, _ = DR.detections([hd], [[(32.0, 16.0)]], 64, 32, 640, 480, 0.5, relative=False)
    assert abs_boxes[0].tolist() == [480.0, 360.0, 320.0, 240.0]


def test_order_location_outer_anchor_inner():
    hd = head(1, 2, 2, 1, fill_obj=0.9)  # all four (location, anchor) pairs pass
    hd[0, 0, 0] = 0.1  # tx of anchor 0
    hd[0, 1, 0] = 0.2  # tx of anchor 1
    boxes, _, _ = DR.detections([hd], [[(1, 1), (1, 1)]], 8, 8, 8, 8, 0.5, relative=True)
    xs = boxes[:, 0] * 2  # (col + tx)
    assert np.allclose(xs, [0.1, 0.2, 1.1, 1.2])


def test_letterbox_keeps_center():
    dw, dh, rw, rh = DR.correct_params(416, 416, 640, 480, letter=True)
    assert (dw, dh, rw, rh) == (0.0, 104.0, 1.0, 0.75)  # new size 416 x 312
    hd = head(1, 1, 1, 1)
    hd[0, 0, :, 0, 0] = [0.5, 0.5, 0.0, 0.0, 0.9, 0.9]
    boxes, _, _ = DR.detections([hd], [[(104.0, 78.0)]], 416, 416, 640, 480, 0.5, relative=True, letter=True)
    assert boxes[0, 0] == 0.5 and boxes[0, 1] == 0.5
    assert boxes[0, 2] == np.float32(0.25) and boxes[0, 3] == np.float32(78.0 / 416) / np.float32(0.75)


def test_box_iou_cases():
    a = np.array([10, 10, 10, 10], np.float32)
    B = np.array([[10, 10, 10, 10], [12, 10, 10, 10], [20, 10, 10, 10], [40, 40, 2, 2], [10, 10, 0, 10]], np.float32)
    iou = DR.box_iou(a, B)
    assert iou[0] == 1.0
    assert iou[1] == np.float32(80) / np.float32(120)
    assert iou[2] == 0.0  # touching edges: intersection 0
    assert iou[3] == 0.0  # disjoint
    assert iou[4] == 0.0  # zero-area box


def test_nms_greedy_semantics():
    boxes = np.array([[10, 10, 10, 10], [12, 10, 10, 10], [14, 10, 10, 10], [50, 50, 10, 10]], np.float32)
    prob = np.array([[0.9, 0.3], [0.8, 0.0], [0.7, 0.6], [0.6, 0.5]], np.float32)
    out = DR.nms_sort(boxes, prob.copy(), 0.45)
    # class 0: A keeps, B (IoU 0.667 with A) goes, C (IoU 0.43 with A; its overlap with B does not
    # count, B is suppressed) stays, D is far away
    assert out[:, 0].tolist() == [np.float32(0.9), 0.0, np.float32(0.7), np.float32(0.6)]
    # class 1: C (0.6) keeps, D (0.5) far, A (0.3): IoU(C, A) = 0.43 < 0.45 stays
    assert out[:, 1].tolist() == [np.float32(0.3), 0.0, np.float32(0.6), np.float32(0.5)]


def _greedy64(boxes, p, thresh):
    keep = []
    idx = [i for i in np.argsort(-p, kind="stable") if p[i] != 0]
    alive = {i: True for i in idx}
    b = boxes.astype(np.float64)

    def iou(a, c):
        w = min(a[0] + a[2] / 2, c[0] + c[2] / 2) - max(a[0] - a[2] / 2, c[0] - c[2] / 2)
        h = min(a[1] + a[3] / 2, c[1] + c[3] / 2) - max(a[1] - a[3] / 2, c[1] - c[3] / 2)
        inter = 0.0 if (w < 0 or h < 0) else w * h
        u = a[2] * a[3] + c[2] * c[3] - inter
        return 0.0 if inter == 0 or u == 0 else inter / u

    for n, i in enumerate(idx):
        if not alive[i]:
            continue
        keep.append(i)
        for j in idx[n + 1:]:
            if alive[j] and iou(b[i], b[j]) > thresh:
                alive[j] = False
    return sorted(keep)


def test_nms_matches_independent_float64():
    rng = np.random.default_rng(9)
    D, C = 300, 4
    boxes = np.concatenate([rng.uniform(0, 200, (D, 2)), rng.uniform(5, 40, (D, 2))], 1).astype(np.float32)
    prob = np.where(rng.random((D, C)) < 0.6, rng.random((D, C)), 0).astype(np.float32)
    # keep clear of the threshold: no pair's IoU within 1e-4 of it
    for i in range(D):
        iou = DR.box_iou(boxes[i], boxes)
        assert not (np.abs(iou.astype(np.float64) - 0.45) < 1e-4).any()
    out = DR.nms_sort(boxes, prob.copy(), 0.45)
    for k in range(C):
        assert sorted(np.nonzero(out[:, k])[0].tolist()) == _greedy64(boxes, prob[:, k], 0.45)
