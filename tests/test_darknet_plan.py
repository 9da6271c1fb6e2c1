"""Host-side planning of darknet.Network (CPU): how a batch is split into
passes so that no kernel call addresses more than 2 GiB."""
import pytest

from tensorium_amd import darknet


def test_pass_batch_yolov3():
    """YOLOv3's largest activation is layer 0's output, 32 channels at the
    input resolution: 416 x 416 x 32 x 4 B = 22 151 168 B per image, so a
    pass holds floor((2^31 - 16) / that) = 96 images; at 608, 47 316 992 B
    per image, 45."""
    _, l416 = darknet.load_cfg("yolov3.cfg")
    assert 416 * 416 * 32 * 4 * 96 <= darknet.MAX_CALL_BYTES < 416 * 416 * 32 * 4 * 97
    assert darknet.pass_batch(l416, 16) == 16
    assert darknet.pass_batch(l416, 96) == 96
    assert darknet.pass_batch(l416, 200) == 96
    assert darknet.pass_batch(l416, 200, max_pass_batch=7) == 7
    assert darknet.pass_batch(l416, 5, max_pass_batch=7) == 5
    assert darknet.pass_batch(l416, 5, max_pass_batch=0) == 1
    _, l608 = darknet.load_cfg("yolov3.cfg", 608, 608)
    assert darknet.pass_batch(l608, 32) == 32
    assert darknet.pass_batch(l608, 64) == 45


def test_reference_route_mode_is_not_split():
    """The reference's whole-tensor route concat mixes images across the
    batch: a batch that needs several passes is refused, before anything
    touches the GPU."""
    _, layers = darknet.load_cfg("yolov3.cfg", 64, 64)
    with pytest.raises(NotImplementedError, match="route_mode='reference'"):
        darknet.Network(None, layers, 4, {}, route_mode="reference", max_pass_batch=2)
