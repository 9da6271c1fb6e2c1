"""tensorium_amd: MI355X (gfx950) backend for Tensorium's fp32 convolution path.

The compute lives in libtensorium_hip.so (HIP kernels + C ABI declared in
include/tensorium_hip.h).  ``nnhip.TNNHip`` mirrors the reference's TNNCuda
backend object; ``synth`` generates the seeded synthetic inputs; ``yolo``
builds and runs a YOLOv3 network through the C ABI.
"""
from . import synth  # noqa: F401

__all__ = ["synth"]
