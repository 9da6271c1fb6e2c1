"""Host-side mirror of Tensorium's GPU backend object over libtensorium_hip.

``TNNHip`` has the method names, argument order and argument meaning of
``TNNCuda<T>`` (source/nncuda.pas:35-200), so code written against the
reference backend (``cuda.gemm(...)``, ``cuda.im2col(...)``, ...) reads the
same against this one (``hip.gemm(...)``).  Buffers are ``(buffer, offset)``
pairs exactly as in the reference; a buffer may be a ``DeviceBuffer`` from
``createDeviceBuffer``, a device ``torch.Tensor`` or a raw device address.

Errors: every C call returns a status; a non-zero status raises
``TNHError`` carrying ``tnh_last_error()``.  This is the analogue of the
reference's ``SAFE_CALL`` assertion (nncuda.pas:237-275).

The library must be built (``python tensorium_amd/build.py``); importing this
module fails loudly if ``libtensorium_hip.so`` is missing -- there is no CPU
fallback.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libtensorium_hip.so")

# TActivationType ordinals (ntypes.pas:66)
acLOGISTIC, acLINEAR, acLEAKY = 0, 4, 9
# conv weight layouts
WEIGHTS_REFERENCE, WEIGHTS_TAP_MAJOR = 0, 1
# number of compiled conv tile configurations (tnh_conv2d_set_autotune ids
# 0..NUM_CONV_CFGS-1: 0-5 LDS-staged, 11-19 lean software-pipelined, 20-26
# wave-split; 6-10 retired); CONV_NCHW_CFGS serve tnh_conv2d_fwd,
# CONV_LEAN_CFGS and CONV_WSPLIT_CFGS
# tnh_conv2d_fwd_nhwc; a forced id is
# tile + CONV_SPLIT_UNIT * splits (uniform split-K, up to 16), or, for a lean
# tile, tile + CONV_SPLIT_UNIT * (base + pieces) (tail split; base
# CONV_TAIL_BASE: rounds of one tile per CU, CONV_TAIL_SLOT_BASE: rounds of
# one tile per resident workgroup slot)
NUM_CONV_CFGS = 27
NUM_CONV_NCHW_CFGS = 27
CONV_RETIRED_CFGS = range(6, 11)
CONV_NCHW_CFGS = [c for c in range(NUM_CONV_NCHW_CFGS) if c not in CONV_RETIRED_CFGS]
CONV_LEAN_CFGS = range(11, 20)
CONV_WSPLIT_CFGS = range(20, 27)
CONV_SPLIT_UNIT = 64
CONV_TAIL_BASE = 16
CONV_TAIL_SLOT_BASE = 32
# SGEMM tile configurations (tnh_sgemm_set_autotune): 0, 1 general, 2..5 lean,
# 6..8 wave-split
NUM_SGEMM_CFGS = 9

i32, i64, f32, vp = C.c_int32, C.c_int64, C.c_float, C.c_void_p

# name -> argtypes (restype is int32 status unless listed in _RESTYPES)
_PROTOS = {
    "tnh_init": [i32],
    "tnh_finalize": [],
    "tnh_device_count": [C.POINTER(i32)],
    "tnh_synchronize": [],
    "tnh_last_error": [],
    "tnh_get_stream": [C.POINTER(vp)],
    "tnh_set_stream": [vp],
    "tnh_reset_stream": [],
    "tnh_cu_count": [C.POINTER(i32)],
    "tnh_set_deterministic": [i32],
    "tnh_graph_begin": [],
    "tnh_graph_end": [C.POINTER(vp)],
    "tnh_graph_launch": [vp],
    "tnh_graph_destroy": [vp],
    "tnh_malloc": [i64, C.POINTER(vp)],
    "tnh_free": [vp],
    "tnh_h2d": [vp, vp, i64],
    "tnh_d2h": [vp, vp, i64],
    "tnh_event_create": [C.POINTER(vp)],
    "tnh_event_destroy": [vp],
    "tnh_event_record": [vp],
    "tnh_stream_wait_event": [vp],
    "tnh_stream_create": [C.POINTER(vp)],
    "tnh_stream_destroy": [vp],
    "tnh_event_elapsed_ms": [vp, vp, C.POINTER(f32)],
    "tnh_sgemm": [i32, i32, i64, i64, i64, f32, vp, i64, i64, vp, i64, i64, f32, vp, i64, i64],
    "tnh_sgemm_strided_batched": [i32, i32, i64, i64, i64, f32, vp, i64, i64, i64, vp, i64, i64, i64,
                                  f32, vp, i64, i64, i64, i64],
    "tnh_im2col": [i64] * 11 + [vp, i64, vp, i64],
    "tnh_im2col_batched": [i64] * 11 + [vp, i64, i64, vp, i64, i64, i64],
    "tnh_col2im": [i64] * 11 + [vp, i64, vp, i64],
    "tnh_col2im_batched": [i64] * 11 + [vp, i64, i64, vp, i64, i64, i64],
    "tnh_conv2d_fwd": [i64] * 11 + [vp, i64, i64, vp, i64, i32, vp, i64, i32, vp, i64, i64, vp, i64, i64],
    "tnh_conv2d_pack_weights": [i64, i64, i64, i64, vp, vp],
    "tnh_conv2d_set_autotune": [i32, i32],
    "tnh_conv2d_fwd_nhwc": [i64, i64, i64, i64, i64, i64, i64, i64, i64, i64, i64, vp, i64, i64, vp, i64, vp, i64,
                            i32, vp, i64, i64, vp, i64, i64],
    "tnh_conv2d_fwd_nhwc_noalloc": [i64, i64, i64, i64, i64, i64, i64, i64, i64, i64, i64, vp, i64, i64, vp, i64,
                                    vp, i64, i32, vp, i64, i64, vp, i64, i64],
    "tnh_conv2d_fwd_nhwc_upsample": [i64, i64, i64, i64, i64, i64, i64, i64, i64, i64, i64, vp, i64, i64, vp, i64,
                                     vp, i64, i32, i64, f32, vp, i64, i64],
    "tnh_conv2d_fwd_nhwc_yolo": [i64, i64, i64, i64, i64, i64, i64, i64, i64, i64, i64, vp, i64, i64, vp, i64, vp,
                                 i64, i32, vp, i64, i64, i64, i64, vp, i64],
    "tnh_conv2d_noalloc_scratch_bytes": [C.POINTER(i64)],
    "tnh_sgemm_set_autotune": [i32, i32],
    "tnh_yolo_fwd_nhwc": [i64, i64, i64, i64, i64, vp, i64, i64, vp],
    "tnh_copy_channels": [i64, i64, vp, i64, i64, vp, i64, i64],
    "tnh_upsample_nhwc": [i64, i64, i64, i64, i64, f32, vp, i64, i64, vp, i64, i64],
    "tnh_maxpool_fwd_nhwc": [i64] * 10 + [vp, i64, i64, vp, i64, i64],
    "tnh_conv2d_out_dims": [i64] * 8 + [C.POINTER(i64), C.POINTER(i64)],
    "tnh_forward_bias": [i64, vp, i64, i64, vp, i64, i64],
    "tnh_forward_scale": [i64, vp, i64, i64, vp, i64, i64],
    "tnh_backward_bias": [i64, vp, i64, vp, i64, i64, i64],
    "tnh_activate": [i64, vp, i64, i32],
    "tnh_derive": [i64, vp, i64, i32, vp],
    "tnh_addvv": [i64, vp, i64, i64, vp, i64, i64, vp, i64, i64],
    "tnh_axpy": [i64, f32, vp, i64, i64, vp, i64, i64],
    "tnh_scale": [i64, f32, vp, i64],
    "tnh_fill": [i64, vp, i64, f32, i64],
    "tnh_copy": [i64, vp, i64, i64, vp, i64, i64],
    "tnh_route": [i64, i32, C.POINTER(vp), C.POINTER(i64), vp],
    "tnh_maxpool_fwd": [i64] * 4 + [vp] + [i64] * 7 + [vp, vp],
    "tnh_maxpool_bwd": [i64] * 4 + [vp, vp, vp],
    "tnh_maxpool_bwd_geom": [i64] * 4 + [vp, vp, vp] + [i64] * 6,
    "tnh_upsample": [i64, i64, i64, i64, vp, i64, i32, f32, vp, i32],
    "tnh_bn_normalize": [i64, vp, i64, i64, vp, vp, i64],
    "tnh_normalize": [i64, i64, i64, vp, i64, vp, i64, vp, i64],
    "tnh_forward_scale_add": [i64, vp, i64, i64, vp, vp, i64, i64],
    "tnh_bn_forward": [i64, i64, i64, vp, vp, vp, vp, vp, vp, vp, i32],
    "tnh_bn_forward_maxpool": [i64, i64, i64, i64, vp, vp, vp, vp, vp, vp, vp, i32, vp, vp],
    "tnh_bn_forward_avgpool": [i64, i64, i64, vp, vp, vp, vp, vp, vp, vp, i32, vp],
    "tnh_bn_train_forward_maxpool": [i64, i64, i64, i64, vp, vp, vp, vp, vp, vp, vp, f32, vp, vp, i32, vp, vp],
    "tnh_bn_train_forward_avgpool": [i64, i64, i64, vp, vp, vp, vp, vp, vp, vp, f32, vp, vp, i32, vp],
    "tnh_yolo_fwd": [i64] * 5 + [vp, vp],
    "tnh_yolo_detections": [i64, i32, C.POINTER(vp), C.POINTER(i64), i64, i64, C.POINTER(f32), i64, i64, i64, i64,
                            f32, i32, i32, i64, vp, vp, vp, vp],
    "tnh_yolo_nms_sort": [i64, i64, i64, vp, vp, vp, f32],
    "tnh_means_vars": [i64, i64, i64, vp, i64, vp, vp],
    "tnh_means": [i64, i64, i64, vp, i64, vp],
    "tnh_bn_backward_scale": [i64, i64, i64, vp, i32, vp, vp, vp, vp],
    "tnh_bn_backward": [i64, i64, i64, vp, i32, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp],
    "tnh_bn_backward_maxpool": [i64, i64, i64, i64, i64, vp, vp, vp, i32, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp],
    "tnh_bn_backward_avgpool": [i64, i64, i64, vp, vp, i32, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp],
    "tnh_variances": [i64, i64, i64, vp, i64, vp, vp],
    "tnh_bn_statistics": [i64, i64, i64, vp, i64, vp, vp, vp, vp, f32],
    "tnh_means_vars_delta": [i64, i64, i64, vp, vp, i64, vp, vp, vp, vp],
    "tnh_normalize_delta": [i64, i64, i64, vp, vp, i64, vp, vp, vp, vp],
    "tnh_add_dots": [i64, i64, i64, vp, vp, i64, vp],
    "tnh_softmax_batch": [i64, vp, i64, i64, i64, i64, i64, i64, f32, vp, i64],
    "tnh_cross_entropy_softmax": [i64, vp, vp, vp, vp],
    "tnh_softmax_head_forward": [i64, i64, i64, i64, vp, vp, vp, vp, vp, vp, vp, vp, vp],
    "tnh_softmax_head_backward": [i64, i64, i64, i64, f32, vp, vp, vp, vp, vp, vp, vp],
    "tnh_clamp": [i64, f32, vp, vp, i64, i64],
    "tnh_subvv": [i64, vp, i64, i64, vp, i64, i64, vp, i64, i64],
    "tnh_mulvv": [i64, vp, i64, i64, vp, i64, i64, vp, i64, i64],
    "tnh_fmavv": [i64, vp, i64, i64, vp, i64, i64, vp, i64, i64, vp, i64, i64],
    "tnh_power": [i64, vp, i64, i64, f32, vp, i64, i64],
    "tnh_fmavss": [i64, vp, i64, f32, f32, vp],
    "tnh_cross_entropy_logistic": [i64, vp, vp, vp, vp],
    "tnh_cost_l2": [i64, vp, vp, vp, vp],
    "tnh_inverse_sqrt": [i64, f32, vp, vp, i64, i64],
    "tnh_activate_swish": [i64, vp, i64, vp, vp],
    "tnh_dropout_fwd": [i64, vp, f32, f32, i64, vp, vp],
    "tnh_dropout_bwd": [i64, vp, f32, f32, vp, vp],
    "tnh_avgpool_fwd": [i64, i64, i64, i64, vp, vp],
    "tnh_avgpool_bwd": [i64, i64, i64, i64, vp, vp],
    "tnh_sgd_update": [i64, f32, i64, f32, f32, vp, vp],
    "tnh_sgd_update_pack": [i64, f32, i64, f32, f32, vp, vp, i32, C.POINTER(i64), C.POINTER(i64), C.POINTER(i64),
                            C.POINTER(i64), C.POINTER(vp), C.POINTER(vp), i64, vp, vp],
    "tnh_sgd_update_pack_pieces": [i64, f32, i64, f32, f32, vp, vp, i32, C.POINTER(i64), C.POINTER(i64),
                                   C.POINTER(i64), C.POINTER(i64), C.POINTER(vp), C.POINTER(vp), C.POINTER(vp),
                                   C.POINTER(i32), i64, vp, vp],
    "tnh_param_update": [i64, f32, i64, f32, vp, vp],
    "tnh_conv2d_pack_weights_dgrad": [i64, i64, i64, i64, vp, vp, vp],
    "tnh_conv2d_wgrad": [i64] * 13 + [vp, i64, vp, i64, f32, f32, vp],
    "tnh_conv2d_wgrad_pieces": [i64] * 13 + [vp, i64, vp, i64, vp, i64, C.POINTER(i32)],
    "tnh_sgemm_nt_batch_reduce": [i64, i64, i64, f32, vp, i64, i64, i64, vp, i64, i64, i64, f32, vp, i64, i64,
                                  i64],
}
_RESTYPES = {"tnh_last_error": C.c_char_p}

_lib = None


class TNHError(RuntimeError):
    """A libtensorium_hip call returned a non-zero status."""

    def __init__(self, fn, status, message):
        super().__init__(f"{fn} failed with status {status}: {message}")
        self.status = status
        self.message = message


def lib():
    """Loads libtensorium_hip.so once; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is missing: build it with `python tensorium_amd/build.py` "
                              "(there is no CPU fallback)")
        L = C.CDLL(LIB_PATH)
        for name, args in _PROTOS.items():
            f = getattr(L, name)
            f.argtypes = args
            f.restype = _RESTYPES.get(name, i32)
        _lib = L
    return _lib


def exported_symbols():
    return list(_PROTOS)


def call(name, *args):
    """Calls a tnh_* entry point and raises TNHError on a non-zero status."""
    L = lib()
    st = getattr(L, name)(*args)
    if st != 0:
        raise TNHError(name, st, L.tnh_last_error().decode(errors="replace"))
    return st


def last_error():
    return lib().tnh_last_error().decode(errors="replace")


class DeviceBuffer:
    """A device allocation made through tnh_malloc (TCUMem of the reference)."""

    __slots__ = ("ptr", "count", "itemsize")

    def __init__(self, ptr, count, itemsize=4):
        self.ptr, self.count, self.itemsize = ptr, count, itemsize

    def __int__(self):
        return self.ptr or 0


def _free_device(ptr):
    """Finalizer of a DeviceArray's allocation (the library may already be
    gone at interpreter exit; then the process releases the memory)."""
    if _lib is not None and ptr:
        _lib.tnh_free(ptr)


def release_stream(stream, events=()):
    """Finalizer for a stream from streamCreate and events from eventCreate
    (statuses ignored: at interpreter exit the context may already be gone,
    and a stream still selected is refused and left to the process end)."""
    if _lib is None:
        return
    for ev in events:
        _lib.tnh_event_destroy(ev)
    if stream:
        _lib.tnh_stream_destroy(stream)


class DeviceArray:
    """A shaped, typed device array in memory from tnh_malloc (the library's
    own allocator, TNNCuda.createDeviceBuffer), for Python callers that use
    no other GPU framework: flat slices and reshaped views share the memory,
    uploads and downloads go through tnh_h2d / tnh_d2h, which are ordered on
    the context stream.  Any entry point that takes a device buffer takes
    it (data_ptr)."""

    is_cuda = True

    def __init__(self, shape, dtype=np.float32, _base=None, _ptr=None):
        import weakref

        self.shape = (int(shape),) if np.isscalar(shape) else tuple(int(d) for d in shape)
        self.dtype = np.dtype(dtype)
        self._base = _base  # keeps the owning allocation alive
        if _ptr is not None:
            self.ptr = _ptr
            return
        p = vp()
        call("tnh_malloc", max(self.numel(), 1) * self.dtype.itemsize, C.byref(p))
        self.ptr = p.value
        weakref.finalize(self, _free_device, self.ptr)

    @classmethod
    def from_numpy(cls, a):
        a = np.ascontiguousarray(a)
        d = cls(a.shape, a.dtype)
        d.copy_from(a)
        return d

    def numel(self):
        return int(np.prod(self.shape))

    def data_ptr(self):
        return self.ptr

    def view(self, *shape):
        """The same memory with another shape of as many elements."""
        shape = tuple(shape[0]) if len(shape) == 1 and not np.isscalar(shape[0]) else shape
        if int(np.prod(shape)) != self.numel():
            raise ValueError(f"view {shape} of {self.shape}")
        return DeviceArray(shape, self.dtype, self._base or self, self.ptr)

    def __getitem__(self, key):
        """A contiguous block sharing the memory: integers on some axes, one
        range on one axis, with every axis the block spans after it whole
        (a[b], a[c0:c1], a[b, :n], a[:, lo:hi] of a batch of one)."""
        key = key if isinstance(key, tuple) else (key,)
        if len(key) > len(self.shape):
            raise IndexError(f"{len(key)} indexes into {len(self.shape)} axes")
        key = key + (slice(None),) * (len(self.shape) - len(key))
        strides = [int(np.prod(self.shape[a + 1:])) for a in range(len(self.shape))]
        off, shape, outer = 0, [], 1
        for n, st, k in zip(self.shape, strides, key):
            if isinstance(k, (int, np.integer)):
                i = int(k) + n if k < 0 else int(k)
                if not 0 <= i < n:
                    raise IndexError(f"index {k} of an axis of {n}")
                if outer > 1 and n > 1:
                    raise TypeError("the selected block is not contiguous")
                off += i * st
            elif isinstance(k, slice) and k.step in (None, 1):
                lo, hi, _ = k.indices(n)
                m = max(hi - lo, 0)
                if outer > 1 and m != n:
                    raise TypeError("the selected block is not contiguous")
                off += lo * st
                shape.append(m)
                outer *= m
            else:
                raise TypeError(f"unsupported index {k!r}")
        return DeviceArray(tuple(shape), self.dtype, self._base or self, self.ptr + off * self.dtype.itemsize)

    def copy_from(self, a):
        a = np.ascontiguousarray(a, dtype=self.dtype)
        if a.size != self.numel():
            raise ValueError(f"copy of {a.size} elements into {self.numel()}")
        call("tnh_h2d", self.ptr, a.ctypes.data, a.nbytes)

    def numpy(self):
        out = np.empty(self.shape, self.dtype)
        call("tnh_d2h", out.ctypes.data, self.ptr, out.nbytes)
        return out


def addr(buf):
    """Device address of a buffer argument (None -> NULL)."""
    if buf is None:
        return None
    if isinstance(buf, int):
        return buf
    if isinstance(buf, DeviceBuffer):
        return buf.ptr
    if hasattr(buf, "data_ptr"):
        if getattr(buf, "is_cuda", False) is False:
            raise TypeError("host torch.Tensor passed where a device buffer is required")
        return buf.data_ptr()
    raise TypeError(f"not a device buffer: {type(buf)!r}")


def _b(flag):
    return 1 if flag else 0


class TNNHip:
    """MI355X backend object; method surface of TNNCuda<single>."""

    NUM_THREADS = 0x200

    @staticmethod
    def deviceCount():
        n = i32(0)
        st = lib().tnh_device_count(C.byref(n))
        return n.value if st == 0 else 0

    def __init__(self, deviceIndex=0):
        call("tnh_init", deviceIndex)
        self.deviceIndex = deviceIndex

    # -- lifecycle -------------------------------------------------------
    def Destroy(self):
        call("tnh_finalize")

    def finish(self):
        call("tnh_synchronize")

    @property
    def stream(self):
        s = vp()
        call("tnh_get_stream", C.byref(s))
        return s.value

    def setStream(self, stream):
        """Enqueue on `stream` (a hipStream_t; 0/None = the null stream)."""
        call("tnh_set_stream", stream or None)

    def useTorchStream(self):
        """Share torch's current stream so torch and library work stay ordered."""
        import torch

        self.setStream(torch.cuda.current_stream().cuda_stream)

    def resetStream(self):
        call("tnh_reset_stream")

    def cuCount(self):
        n = i32(0)
        call("tnh_cu_count", C.byref(n))
        return n.value

    # -- graphs --------------------------------------------------------------
    def graphBegin(self):
        """Start capturing the context's own stream (call resetStream first)."""
        call("tnh_graph_begin")

    def graphEnd(self):
        g = vp()
        call("tnh_graph_end", C.byref(g))
        return g.value

    def graphLaunch(self, graph):
        call("tnh_graph_launch", graph)

    def graphDestroy(self, graph):
        call("tnh_graph_destroy", graph)

    # -- memory ------------------------------------------------------------
    def createDeviceBuffer(self, N):
        p = vp()
        call("tnh_malloc", 4 * N, C.byref(p))
        return DeviceBuffer(p.value, N)

    def freeDeviceBuffer(self, cudaMem):
        call("tnh_free", addr(cudaMem))

    def writeBuffer(self, cudaMem, bufferSize, buffer):
        a = np.ascontiguousarray(buffer)
        assert a.nbytes >= bufferSize
        call("tnh_h2d", addr(cudaMem), a.ctypes.data, bufferSize)

    def readBuffer(self, cudaMem, bufferSize, buffer):
        assert isinstance(buffer, np.ndarray) and buffer.flags.c_contiguous and buffer.nbytes >= bufferSize
        call("tnh_d2h", buffer.ctypes.data, addr(cudaMem), bufferSize)

    # -- GEMM ----------------------------------------------------------------
    def gemm(self, transA, transB, M, N, K, ALPHA, A, aOffset, lda, B, bOffset, ldb, BETA, C_, cOffset, ldc):
        call("tnh_sgemm", _b(transA), _b(transB), M, N, K, ALPHA, addr(A), aOffset, lda, addr(B), bOffset, ldb,
             BETA, addr(C_), cOffset, ldc)

    def gemmStridedBatched(self, transA, transB, M, N, K, ALPHA, A, aOffset, lda, strideA, B, bOffset, ldb,
                           strideB, BETA, C_, cOffset, ldc, strideC, batchCount):
        call("tnh_sgemm_strided_batched", _b(transA), _b(transB), M, N, K, ALPHA, addr(A), aOffset, lda, strideA,
             addr(B), bOffset, ldb, strideB, BETA, addr(C_), cOffset, ldc, strideC, batchCount)

    # -- im2col / col2im -----------------------------------------------------
    def im2col(self, aChannels, aHeight, aWidth, kernelHeight, kernelWidth, padHeight, padWidth, strideY, strideX,
               dilationY, dilationX, im, imOffset, col, colOffset):
        call("tnh_im2col", aChannels, aHeight, aWidth, kernelHeight, kernelWidth, padHeight, padWidth, strideY,
             strideX, dilationY, dilationX, addr(im), imOffset, addr(col), colOffset)

    def im2colStridedBatched(self, aChannels, aHeight, aWidth, kernelHeight, kernelWidth, padHeight, padWidth,
                             strideY, strideX, dilationY, dilationX, im, imStride, imOffset, col, colStride,
                             colOffset, batchCount):
        """sim2colStridedBatched (ntensors.pas:11493) argument order."""
        call("tnh_im2col_batched", aChannels, aHeight, aWidth, kernelHeight, kernelWidth, padHeight, padWidth,
             strideY, strideX, dilationY, dilationX, addr(im), imOffset, imStride, addr(col), colOffset, colStride,
             batchCount)

    def col2im(self, aChannels, aHeight, aWidth, kernelHeight, kernelWidth, padHeight, padWidth, strideY, strideX,
               dilationY, dilationX, col, colOffset, im, imOffset):
        call("tnh_col2im", aChannels, aHeight, aWidth, kernelHeight, kernelWidth, padHeight, padWidth, strideY,
             strideX, dilationY, dilationX, addr(col), colOffset, addr(im), imOffset)

    def col2imStridedBatched(self, aChannels, aHeight, aWidth, kernelHeight, kernelWidth, padHeight, padWidth,
                             strideY, strideX, dilationY, dilationX, col, colStride, colOffset, im, imStride,
                             imOffset, batchCount):
        """scol2imStridedBatched (ntensors.pas:11833) argument order."""
        call("tnh_col2im_batched", aChannels, aHeight, aWidth, kernelHeight, kernelWidth, padHeight, padWidth,
             strideY, strideX, dilationY, dilationX, addr(col), colOffset, colStride, addr(im), imOffset, imStride,
             batchCount)

    # -- fused convolution (new: replaces im2col+gemm+bias+activate) ---------
    def conv2dForward(self, batch, c, h, w, filters, kernelSize, stride, padding, input, inOffset, weights,
                      biases, activation, output, outOffset, inBatchStride=None, outBatchStride=None,
                      residual=None, resOffset=0, resBatchStride=None, weightLayout=WEIGHTS_REFERENCE,
                      kernelWidth=None, padWidth=None):
        """Fused conv + bias + activation (+ shortcut add); kernelSize and
        padding are the height ones, kernelWidth / padWidth default to them.
        Returns (outH, outW)."""
        kw = kernelSize if kernelWidth is None else kernelWidth
        pw = padding if padWidth is None else padWidth
        oh = (h + 2 * padding - kernelSize) // stride + 1
        ow = (w + 2 * pw - kw) // stride + 1
        xs = c * h * w if inBatchStride is None else inBatchStride
        os_ = filters * oh * ow if outBatchStride is None else outBatchStride
        rs = filters * oh * ow if resBatchStride is None else resBatchStride
        call("tnh_conv2d_fwd", batch, c, h, w, filters, kernelSize, kw, padding, pw, stride, stride,
             addr(input), inOffset, xs, addr(weights), 0, weightLayout, addr(biases), 0, activation, addr(residual),
             resOffset, rs, addr(output), outOffset, os_)
        return oh, ow

    def conv2dForwardNHWC(self, batch, c, h, w, filters, kernelSize, stride, padding, input, inOffset, weights,
                          biases, activation, output, outOffset, inPix=None, outPix=None, residual=None, resOffset=0,
                          resPix=None, nchwInput=False, noAlloc=False):
        """Channels-last fused conv (tap-major weights); pixel strides default
        to the channel counts; nchwInput reads a C <= 4 image as NCHW;
        noAlloc calls tnh_conv2d_fwd_nhwc_noalloc (no device allocation:
        split pieces in the library's static scratch, no autotuning).
        Returns (outH, outW)."""
        oh = (h + 2 * padding - kernelSize) // stride + 1
        ow = (w + 2 * padding - kernelSize) // stride + 1
        xp = 0 if nchwInput else (c if inPix is None else inPix)
        op_ = filters if outPix is None else outPix
        rp = filters if resPix is None else resPix
        call("tnh_conv2d_fwd_nhwc_noalloc" if noAlloc else "tnh_conv2d_fwd_nhwc", batch, c, h, w, filters,
             kernelSize, kernelSize, padding, padding, stride, stride, addr(input), inOffset, xp, addr(weights), 0,
             addr(biases), 0, activation, addr(residual), resOffset, rp, addr(output), outOffset, op_)
        return oh, ow

    def conv2dForwardNHWCUpsample(self, batch, c, h, w, filters, kernelSize, stride, padding, input, inOffset,
                                  weights, biases, activation, upStride, upScale, output, outOffset, inPix=None,
                                  outPix=None):
        """Channels-last fused conv whose result is stored only as its nearest
        upsample (factor upStride, times upScale) into output, the next
        TUpSampleLayer's tensor (tnh_conv2d_fwd_nhwc_upsample)."""
        xp = c if inPix is None else inPix
        op_ = filters if outPix is None else outPix
        call("tnh_conv2d_fwd_nhwc_upsample", batch, c, h, w, filters, kernelSize, kernelSize, padding, padding, stride,
             stride, addr(input), inOffset, xp, addr(weights), 0, addr(biases), 0, activation, upStride, upScale,
             addr(output), outOffset, op_)

    def conv2dForwardNHWCYolo(self, batch, c, h, w, filters, kernelSize, stride, padding, input, inOffset, weights,
                              biases, activation, output, outOffset, n, classes, yoloOutput, inPix=None,
                              outPix=None, yoloOffset=0):
        """Channels-last fused conv that also writes the yolo head (NCHW) of its
        result (tnh_conv2d_fwd_nhwc_yolo)."""
        xp = c if inPix is None else inPix
        op_ = filters if outPix is None else outPix
        call("tnh_conv2d_fwd_nhwc_yolo", batch, c, h, w, filters, kernelSize, kernelSize, padding, padding, stride,
             stride, addr(input), inOffset, xp, addr(weights), 0, addr(biases), 0, activation, addr(output), outOffset,
             op_, n, classes, addr(yoloOutput), yoloOffset)

    @staticmethod
    def noAllocScratchBytes():
        """Bytes of the static scratch behind conv2dForwardNHWC(noAlloc=True)."""
        v = C.c_int64(0)
        call("tnh_conv2d_noalloc_scratch_bytes", C.byref(v))
        return v.value

    def yoloForwardNHWC(self, batch, n, classes, h, w, input, inOffset, inPix, output):
        """YOLO head on a channels-last input, NCHW head output."""
        call("tnh_yolo_fwd_nhwc", batch, n, classes, h, w, addr(input), inOffset, inPix, addr(output))

    def copyChannels(self, pixels, channels, src, srcOffset, srcPix, dst, dstOffset, dstPix):
        call("tnh_copy_channels", pixels, channels, addr(src), srcOffset, srcPix, addr(dst), dstOffset, dstPix)

    def upSampleNHWC(self, batch, channels, h, w, stride, scale, input, inOffset, inPix, output, outOffset, outPix):
        call("tnh_upsample_nhwc", batch, channels, h, w, stride, scale, addr(input), inOffset, inPix, addr(output),
             outOffset, outPix)

    def forwardMaxPoolNHWC(self, batch, channels, h, w, outH, outW, strideX, strideY, padding, kernelSize, input,
                           inOffset, inPix, output, outOffset, outPix):
        call("tnh_maxpool_fwd_nhwc", batch, channels, h, w, outH, outW, strideX, strideY, padding, kernelSize,
             addr(input), inOffset, inPix, addr(output), outOffset, outPix)

    def packConvWeights(self, filters, c, kernelSize, src, dst, kernelWidth=None):
        """[F][C][kh][kw] -> tap-major [F][kh][kw][C] (device to device)."""
        call("tnh_conv2d_pack_weights", filters, c, kernelSize, kernelSize if kernelWidth is None else kernelWidth,
             addr(src), addr(dst))

    def packConvWeightsDgrad(self, filters, c, kernelSize, src, tapMajor, flipped, kernelWidth=None):
        """[F][C][kh][kw] -> tap-major [F][kh][kw][C] (tapMajor, may be None)
        and the data gradient's flipped [C][kh][kw][F], one launch."""
        call("tnh_conv2d_pack_weights_dgrad", filters, c, kernelSize, kernelSize if kernelWidth is None else kernelWidth,
             addr(src), addr(tapMajor), addr(flipped))

    @staticmethod
    def setDeterministic(enable=True):
        """Same kernels and bits in every process: no timing-based tiling
        choice, no split-K / tail-split (tnh_set_deterministic)."""
        call("tnh_set_deterministic", 1 if enable else 0)

    def setConvAutotune(self, enable=True, forcedConfig=-1):
        call("tnh_conv2d_set_autotune", 1 if enable else 0, forcedConfig)

    def setSgemmAutotune(self, enable=True, forcedConfig=-1):
        """Pins an SGEMM tile configuration (0..NUM_SGEMM_CFGS-1, -1: the library's choice)."""
        call("tnh_sgemm_set_autotune", 1 if enable else 0, forcedConfig)

    # -- epilogue / element-wise ---------------------------------------------
    def forwardBias(self, dstSize, dst, offset, srcSize, src, incb, batch):
        call("tnh_forward_bias", dstSize, addr(dst), offset, srcSize, addr(src), incb, batch)

    def forwardScale(self, dstSize, dst, offset, scaleSize, scale, incb, batch):
        call("tnh_forward_scale", dstSize, addr(dst), offset, scaleSize, addr(scale), incb, batch)

    def backwardBias(self, dstSize, dst, srcSize, src, srcOffset, incb, batch):
        call("tnh_backward_bias", dstSize, addr(dst), srcSize, addr(src), srcOffset, incb, batch)

    def ActivateArray(self, N, x, offset, activation):
        call("tnh_activate", N, addr(x), offset, activation)

    def DeriveArray(self, N, x, offset, activation, delta):
        call("tnh_derive", N, addr(x), offset, activation, addr(delta))

    def addvv(self, N, src1, src1Offset, inca, src2, src2Offset, incb, dst, dstOffset, incc):
        call("tnh_addvv", N, addr(src1), src1Offset, inca, addr(src2), src2Offset, incb, addr(dst), dstOffset, incc)

    def axpy(self, N, a, x, xOffset, incx, y, yOffset, incy):
        call("tnh_axpy", N, a, addr(x), xOffset, incx, addr(y), yOffset, incy)

    def scale(self, N, a, x, stride):
        call("tnh_scale", N, a, addr(x), stride)

    def fill(self, N, x, offset, val, stride):
        call("tnh_fill", N, addr(x), offset, val, stride)

    def copy(self, N, src, srcOffset, inca, dst, dstOffset, incb):
        call("tnh_copy", N, addr(src), srcOffset, inca, addr(dst), dstOffset, incb)

    def concat(self, batch, srcs, sizes, dst):
        """Per-image route concat: dst[b] = [src0[b] | src1[b] | ...]."""
        n = len(srcs)
        ptrs = (vp * n)(*[addr(s) for s in srcs])
        szs = (i64 * n)(*sizes)
        call("tnh_route", batch, n, ptrs, szs, addr(dst))

    # -- pooling / resampling ------------------------------------------------
    def forwardMaxPool(self, aBatch, outC, outH, outW, input, c, h, w, stride_x, stride_y, padding, kernelSize,
                       indexes, output):
        call("tnh_maxpool_fwd", aBatch, outC, outH, outW, addr(input), c, h, w, stride_x, stride_y, padding,
             kernelSize, addr(indexes), addr(output))

    def backwardMaxPool(self, aBatch, outC, outH, outW, output, indexes, delta, geometry=None):
        """output = delta of the layer input (accumulated), as in the reference.

        The library gathers in the reference's order with the geometry of the
        forwardMaxPool call that wrote ``indexes``; ``geometry=(h, w,
        stride_x, stride_y, padding, kernelSize)`` gives it explicitly
        (tnh_maxpool_bwd_geom) for indexes written elsewhere.
        """
        if geometry is None:
            call("tnh_maxpool_bwd", aBatch, outC, outH, outW, addr(output), addr(indexes), addr(delta))
            return
        h, w, sx, sy, pad, k = geometry
        call("tnh_maxpool_bwd_geom", aBatch, outC, outH, outW, addr(output), addr(indexes), addr(delta), h, w, sx,
             sy, pad, k)

    def upSample(self, aBatch, aChannels, outHeight, outWidth, in_, stride, isForward, scale, out, zeroIn=0):
        call("tnh_upsample", aBatch, aChannels, outHeight, outWidth, addr(in_), stride, isForward, scale, addr(out),
             zeroIn)

    def yoloForward(self, batch, n, classes, h, w, input, output):
        """TYoloLayer.forward inference: copy + logistic on x, y, obj, classes."""
        call("tnh_yolo_fwd", batch, n, classes, h, w, addr(input), addr(output))

    def yoloDetections(self, batch, heads, hw, n, classes, anchors, netW, netH, imgW, imgH, thresh, relative,
                       letter, capacity, boxes, objectness, prob, counts):
        """TNNet.Detections over yolo heads on the device: heads = device
        tensors (after yoloForward), hw = [(h, w)] per head, anchors =
        [[(w, h)] * n] per head (the mask's anchors); fills boxes
        [batch][capacity][4], objectness [batch][capacity], prob
        [batch][capacity][classes] and counts [batch] (int32; a count above
        capacity means the buffers were too small)."""
        nh = len(heads)
        hp = (vp * nh)(*[addr(h) for h in heads])
        hwa = (i64 * (2 * nh))(*[v for p in hw for v in p])
        flat = [float(v) for head in anchors for pair in head for v in pair]
        an = (f32 * len(flat))(*flat)
        call("tnh_yolo_detections", batch, nh, hp, hwa, n, classes, an, netW, netH, imgW, imgH, thresh,
             _b(relative), _b(letter), capacity, addr(boxes), addr(objectness), addr(prob), addr(counts))

    def yoloNmsSort(self, batch, classes, capacity, boxes, prob, counts, thresh):
        """TDetectionsHelper.doNMSSort on the device, in place on prob."""
        call("tnh_yolo_nms_sort", batch, classes, capacity, addr(boxes), addr(prob), addr(counts), thresh)

    # -- batch norm ------------------------------------------------------------
    def normalize(self, srcSize, dstSize, groups, means, meansStride, vars, varsStride, dst, dstOffset):
        """TNNCuda.normalize (nncuda.pas:1371) with the CPU clamp."""
        call("tnh_normalize", srcSize, dstSize, groups, addr(means), meansStride, addr(vars), varsStride, addr(dst),
             dstOffset)

    def forwardScaleAdd(self, dstSize, dst, offset, scaleSize, scales, biases, incb, batch):
        """TNNCuda.forwardScaleAdd (nncuda.pas:1490): dst = fl(scale*dst) + bias."""
        call("tnh_forward_scale_add", dstSize, addr(dst), offset, scaleSize, addr(scales), addr(biases), incb, batch)

    def bnForwardAvgPool(self, batch, N, hw, x, xNorm, out, mean, variance, scales, biases, activation, avg):
        """bnForward then avgPoolForward of its output (planes of hw <= 64), one pass."""
        call("tnh_bn_forward_avgpool", batch, N, hw, addr(x), addr(xNorm), addr(out), addr(mean), addr(variance),
             addr(scales), addr(biases), activation, addr(avg))

    def bnTrainForwardMaxPool(self, batch, N, h, w, x, xNorm, out, mean, variance, rollMean, rollVar, momentum,
                              scales, biases, activation, pooled, indexes):
        """bnStatistics then bnForwardMaxPool, three launches (the statistics' final step in the last)."""
        call("tnh_bn_train_forward_maxpool", batch, N, h, w, addr(x), addr(xNorm), addr(out), addr(mean),
             addr(variance), addr(rollMean), addr(rollVar), momentum, addr(scales), addr(biases), activation,
             addr(pooled), addr(indexes))

    def bnTrainForwardAvgPool(self, batch, N, hw, x, xNorm, out, mean, variance, rollMean, rollVar, momentum, scales,
                              biases, activation, avg):
        """bnStatistics then bnForwardAvgPool, three launches."""
        call("tnh_bn_train_forward_avgpool", batch, N, hw, addr(x), addr(xNorm), addr(out), addr(mean),
             addr(variance), addr(rollMean), addr(rollVar), momentum, addr(scales), addr(biases), activation,
             addr(avg))

    def bnForwardMaxPool(self, batch, N, h, w, x, xNorm, out, mean, variance, scales, biases, activation, pooled,
                         indexes):
        """bnForward then forwardMaxPool (2x2, stride 2) of its output, one pass."""
        call("tnh_bn_forward_maxpool", batch, N, h, w, addr(x), addr(xNorm), addr(out), addr(mean), addr(variance),
             addr(scales), addr(biases), activation, addr(pooled), addr(indexes))

    def bnForward(self, dstSize, N, batch, x, xNorm, out, mean, variance, scales, biases, activation):
        """Fused batch-norm forward + activation (tnh_bn_forward)."""
        call("tnh_bn_forward", dstSize, N, batch, addr(x), addr(xNorm), addr(out), addr(mean), addr(variance),
             addr(scales), addr(biases), activation)

    def blockNormalize(self, dstSize, dst, offset, N, mean, variance, batch):
        call("tnh_bn_normalize", dstSize, addr(dst), offset, N, addr(mean), addr(variance), batch)

    # -- training direction ----------------------------------------------------
    def bnStatistics(self, srcSize, dstSize, groups, src, offset, means, vars, rollingMeans, rollingVars,
                     momentum):
        """meansAndVars + the rolling-statistics update in one call (tnh_bn_statistics)."""
        call("tnh_bn_statistics", srcSize, dstSize, groups, addr(src), offset, addr(means), addr(vars),
             addr(rollingMeans), addr(rollingVars), momentum)

    def meansAndVars(self, srcSize, dstSize, groups, src, offset, means, vars):
        call("tnh_means_vars", srcSize, dstSize, groups, addr(src), offset, addr(means), addr(vars))

    def means(self, srcSize, dstSize, groups, src, offset, means):
        call("tnh_means", srcSize, dstSize, groups, addr(src), offset, addr(means))

    def variances(self, srcSize, dstSize, groups, src, offset, means, vars):
        """Unbiased variances about the given means (the CPU path's divisor)."""
        call("tnh_variances", srcSize, dstSize, groups, addr(src), offset, addr(means), addr(vars))

    def bnBackward(self, N, dstSize, groups, output, activation, xNorm, x, scales, mean, variance, delta,
                   scaleUpdates, mean_delta, variance_delta, biases=None):
        """The batch-norm backward with the activation derivative before it:
        bnBackwardScale, meansAndVarsDelta and normalizeDelta in four launches."""
        call("tnh_bn_backward", N, dstSize, groups, addr(output), activation, addr(xNorm), addr(x), addr(scales),
             addr(mean), addr(variance), addr(delta), addr(scaleUpdates), addr(mean_delta), addr(variance_delta),
             addr(biases))

    def bnBackwardMaxPool(self, N, dstSize, groups, h, w, poolIndexes, poolDelta, output, activation, xNorm, x,
                          scales, mean, variance, delta, scaleUpdates, mean_delta, variance_delta, biases=None):
        """backwardMaxPool (2x2, stride 2) into a zeroed delta, then bnBackward; delta is written in full."""
        call("tnh_bn_backward_maxpool", N, dstSize, groups, h, w, addr(poolIndexes), addr(poolDelta), addr(output),
             activation, addr(xNorm), addr(x), addr(scales), addr(mean), addr(variance), addr(delta),
             addr(scaleUpdates), addr(mean_delta), addr(variance_delta), addr(biases))

    def bnBackwardAvgPool(self, N, dstSize, groups, avgDelta, output, activation, xNorm, x, scales, mean, variance,
                          delta, scaleUpdates, mean_delta, variance_delta, biases=None):
        """avgPoolBackward into a zeroed delta, then bnBackward; delta is written in full."""
        call("tnh_bn_backward_avgpool", N, dstSize, groups, addr(avgDelta), addr(output), activation, addr(xNorm),
             addr(x), addr(scales), addr(mean), addr(variance), addr(delta), addr(scaleUpdates), addr(mean_delta),
             addr(variance_delta), addr(biases))

    def bnBackwardScale(self, N, dstSize, groups, output, activation, xNorm, scales, delta, scaleUpdates):
        """DeriveArray + addDots + forwardScale of batchNormBack in one pass
        (tnh_bn_backward_scale)."""
        call("tnh_bn_backward_scale", N, dstSize, groups, addr(output), activation, addr(xNorm), addr(scales),
             addr(delta), addr(scaleUpdates))

    def meansAndVarsDelta(self, srcSize, dstSize, groups, delta, x, offset, mean, variance, mean_delta,
                          variance_delta):
        call("tnh_means_vars_delta", srcSize, dstSize, groups, addr(delta), addr(x), offset, addr(mean),
             addr(variance), addr(mean_delta), addr(variance_delta))

    def normalizeDelta(self, deltaSize, meanSize, groups, delta, x, offset, mean, variance, mean_delta,
                       variance_delta):
        call("tnh_normalize_delta", deltaSize, meanSize, groups, addr(delta), addr(x), offset, addr(mean),
             addr(variance), addr(mean_delta), addr(variance_delta))

    def addDots(self, N, dstSize, groups, src1, src2, srcOffset, dst):
        call("tnh_add_dots", N, dstSize, groups, addr(src1), addr(src2), srcOffset, addr(dst))

    def softmaxBatch(self, N, input, iOffset, batch, batch_size, groups, group_size, stride, temp, output,
                     oOffset):
        call("tnh_softmax_batch", N, addr(input), iOffset, batch, batch_size, groups, group_size, stride, temp,
             addr(output), oOffset)

    def crossEntropySoftmax(self, N, pred, truth, delta, error):
        call("tnh_cross_entropy_softmax", N, addr(pred), addr(truth), addr(delta), addr(error))

    def softmaxHeadForward(self, batch, F, hw, classes, x, avg, weights, biases, truth, logits, prob, delta,
                           error):
        """avgpool + connected + softmax + cross-entropy forward in two launches (x None: avg is filled)."""
        call("tnh_softmax_head_forward", batch, F, hw, classes, addr(x), addr(avg), addr(weights), addr(biases),
             addr(truth), addr(logits), addr(prob), addr(delta), addr(error))

    def softmaxHeadBackward(self, batch, F, hw, classes, clampAlpha, delta, avg, weights, weightUpdates,
                            biasUpdates, avgDelta, deltaIn):
        """Their backward (clamp, bias / weight gradients, avgpool backward) in one launch."""
        call("tnh_softmax_head_backward", batch, F, hw, classes, clampAlpha, addr(delta), addr(avg), addr(weights),
             addr(weightUpdates), addr(biasUpdates), addr(avgDelta), addr(deltaIn))

    def clamp(self, N, alpha, src, dst, stride=1, offset=0):
        call("tnh_clamp", N, alpha, addr(src), addr(dst), stride, offset)

    def subvv(self, N, src1, src1Offset, inca, src2, src2Offset, incb, dst, dstOffset, incc):
        call("tnh_subvv", N, addr(src1), src1Offset, inca, addr(src2), src2Offset, incb, addr(dst), dstOffset, incc)

    def mulvv(self, N, src1, src1Offset, inca, src2, src2Offset, incb, dst, dstOffset, incc):
        call("tnh_mulvv", N, addr(src1), src1Offset, inca, addr(src2), src2Offset, incb, addr(dst), dstOffset, incc)

    def fmavv(self, N, src1, src1Offset, inca, src2, src2Offset, incb, src3, src3Offset, incc, dst, dstOffset,
              incd):
        call("tnh_fmavv", N, addr(src1), src1Offset, inca, addr(src2), src2Offset, incb, addr(src3), src3Offset,
             incc, addr(dst), dstOffset, incd)

    def power(self, N, x, xOffset, incx, a, y, yOffset, incy):
        call("tnh_power", N, addr(x), xOffset, incx, a, addr(y), yOffset, incy)

    def fmavss(self, N, src, offset, scalar, bias, dst):
        call("tnh_fmavss", N, addr(src), offset, scalar, bias, addr(dst))

    def crossEntropyLogistic(self, N, pred, truth, delta, error):
        call("tnh_cross_entropy_logistic", N, addr(pred), addr(truth), addr(delta), addr(error))

    def costL2(self, N, pred, truth, delta, error):
        call("tnh_cost_l2", N, addr(pred), addr(truth), addr(delta), addr(error))

    def inverseSqrt(self, N, alpha, src, dst, stride=1, offset=0):
        call("tnh_inverse_sqrt", N, alpha, addr(src), addr(dst), stride, offset)

    def activateArraySWISH(self, N, x, offset, output_sigmoid, output):
        call("tnh_activate_swish", N, addr(x), offset, addr(output_sigmoid), addr(output))

    def forwardDropout(self, N, src, probability, scale, rnd, dst, seed=None):
        """rnd receives the per-element draws, dst the dropped/scaled values.
        A fresh seed is drawn per call unless one is given, as TNNCuda
        draws one on the host per call (nncuda.pas:1512)."""
        if seed is None:
            self._dropout_seed = getattr(self, "_dropout_seed", 0x9E3779B9) * 6364136223846793005 + 1442695040888963407
            self._dropout_seed &= (1 << 63) - 1
            seed = self._dropout_seed
        call("tnh_dropout_fwd", N, addr(src), probability, scale, seed, addr(rnd), addr(dst))
        return seed

    def backwardDropout(self, N, src, probability, scale, rnd, dst):
        call("tnh_dropout_bwd", N, addr(src), probability, scale, addr(rnd), addr(dst))

    def avgPoolForward(self, batch, c, h, w, input, output):
        call("tnh_avgpool_fwd", batch, c, h, w, addr(input), addr(output))

    def avgPoolBackward(self, batch, c, h, w, delta, deltaIn):
        call("tnh_avgpool_bwd", batch, c, h, w, addr(delta), addr(deltaIn))

    def sgdUpdate(self, N, learningRate, batch, momentum, decay, weights, weightUpdates):
        call("tnh_sgd_update", N, learningRate, batch, momentum, decay, addr(weights), addr(weightUpdates))

    def sgdUpdatePack(self, N, learningRate, batch, momentum, decay, weights, weightUpdates, layers, nParams=0,
                      params=None, paramUpdates=None, pieces=None):
        """sgdUpdate whose pass also refreshes conv layers' packed copies;
        layers: [(offset, F, C, taps, tapMajor, flipped or None), ...]; then
        paramUpdate(nParams, ..., params, paramUpdates) in the same launch.
        pieces: per layer None or (buffer, count) from convWeightGradientPieces,
        added to the layer's weight updates first (tnh_sgd_update_pack_pieces)."""
        n = len(layers)
        arr = lambda t, xs: (t * max(n, 1))(*xs)  # noqa: E731
        tables = (arr(i64, [l[0] for l in layers]), arr(i64, [l[1] for l in layers]),
                  arr(i64, [l[2] for l in layers]), arr(i64, [l[3] for l in layers]),
                  arr(vp, [addr(l[4]) for l in layers]), arr(vp, [addr(l[5]) for l in layers]))
        if pieces is None:
            call("tnh_sgd_update_pack", N, learningRate, batch, momentum, decay, addr(weights), addr(weightUpdates),
                 n, *tables, nParams, addr(params), addr(paramUpdates))
            return
        if len(pieces) != n:
            raise ValueError("one pieces entry per layer")
        call("tnh_sgd_update_pack_pieces", N, learningRate, batch, momentum, decay, addr(weights),
             addr(weightUpdates), n, *tables, arr(vp, [addr(q[0]) if q else None for q in pieces]),
             arr(i32, [q[1] if q else 0 for q in pieces]), nParams, addr(params), addr(paramUpdates))

    def paramUpdate(self, N, learningRate, batch, momentum, params, paramUpdates):
        call("tnh_param_update", N, learningRate, batch, momentum, addr(params), addr(paramUpdates))

    def convWeightGradient(self, batch, c, h, w, filters, kernelH, kernelW, padH, padW, strideY, strideX, dilY, dilX,
                           input, inBatchStride, delta, deltaBatchStride, alpha, beta, dW):
        """dW = beta*dW + alpha * sum_b delta_b * im2col(input_b)^T (the im2col inside the GEMM)."""
        call("tnh_conv2d_wgrad", batch, c, h, w, filters, kernelH, kernelW, padH, padW, strideY, strideX, dilY, dilX,
             addr(input), inBatchStride, addr(delta), deltaBatchStride, alpha, beta, addr(dW))

    def convWeightGradientPieces(self, batch, c, h, w, filters, kernelH, kernelW, padH, padW, strideY, strideX,
                                 dilY, dilX, input, inBatchStride, delta, deltaBatchStride, pieces=None,
                                 piecesFloats=0):
        """tnh_conv2d_wgrad_pieces: the weight-gradient product's split sums
        into `pieces` (None: only count them); returns the number of pieces."""
        n = i32(0)
        call("tnh_conv2d_wgrad_pieces", batch, c, h, w, filters, kernelH, kernelW, padH, padW, strideY, strideX, dilY,
             dilX, addr(input), inBatchStride, addr(delta), deltaBatchStride, addr(pieces), piecesFloats,
             C.byref(n))
        return n.value

    def gemmNTBatchReduce(self, M, N, L, ALPHA, A, aOffset, lda, strideA, B, bOffset, ldb, strideB, BETA, C_,
                          cOffset, ldc, batch):
        """C = BETA*C + ALPHA * sum_b A_b * B_b^T (conv weight gradient)."""
        call("tnh_sgemm_nt_batch_reduce", M, N, L, ALPHA, addr(A), aOffset, lda, strideA, addr(B), bOffset, ldb,
             strideB, BETA, addr(C_), cOffset, ldc, batch)

    # -- events ----------------------------------------------------------------
    def eventCreate(self):
        e = vp()
        call("tnh_event_create", C.byref(e))
        return e.value

    def eventRecord(self, ev):
        call("tnh_event_record", ev)

    def eventElapsed(self, start, stop):
        ms = f32(0)
        call("tnh_event_elapsed_ms", start, stop, C.byref(ms))
        return ms.value

    def streamWaitEvent(self, ev):
        """The context stream waits for `ev` (recorded on another stream)."""
        call("tnh_stream_wait_event", ev)

    def eventDestroy(self, ev):
        call("tnh_event_destroy", ev)

    def streamCreate(self):
        """A second stream (default priority) to select with setStream."""
        s = vp()
        call("tnh_stream_create", C.byref(s))
        return s.value

    def streamDestroy(self, stream):
        """Waits for the stream's work, then destroys it (not while selected)."""
        call("tnh_stream_destroy", stream)
