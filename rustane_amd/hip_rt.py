"""Minimal ctypes plumbing over the HIP runtime that librustane_hip.so links.

Device buffers, copies and events for callers (the benchmark, the device-
pointer tests) that keep inputs resident in HBM.  It binds the runtime
already loaded by librustane_hip.so, so a process has one HIP runtime.
(PyTorch's wheel carries its own HIP/HSA runtime; loading both in one process
leaves the second one without devices, so GPU code here does not use torch.)
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import hip_bridge

_rt = None


def rt():
    global _rt
    if _rt is None:
        hip_bridge.lib()  # loads /opt/rocm libamdhip64.so.7 as a dependency first
        R = ctypes.CDLL("libamdhip64.so.7")
        vp, sz = ctypes.c_void_p, ctypes.c_size_t
        R.hipMalloc.argtypes = [ctypes.POINTER(vp), sz]
        R.hipFree.argtypes = [vp]
        R.hipMemcpy.argtypes = [vp, vp, sz, ctypes.c_int]
        R.hipMemset.argtypes = [vp, ctypes.c_int, sz]
        R.hipDeviceSynchronize.argtypes = []
        R.hipStreamSynchronize.argtypes = [vp]
        R.hipEventCreate.argtypes = [ctypes.POINTER(vp)]
        R.hipEventRecord.argtypes = [vp, vp]
        R.hipEventSynchronize.argtypes = [vp]
        R.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), vp, vp]
        R.hipEventDestroy.argtypes = [vp]
        R.hipGetErrorString.argtypes = [ctypes.c_int]
        R.hipGetErrorString.restype = ctypes.c_char_p
        R.hipStreamBeginCapture.argtypes = [vp, ctypes.c_int]
        R.hipStreamEndCapture.argtypes = [vp, ctypes.POINTER(vp)]
        R.hipGraphInstantiate.argtypes = [ctypes.POINTER(vp), vp, vp, ctypes.c_char_p, sz]
        R.hipGraphLaunch.argtypes = [vp, vp]
        R.hipGraphExecDestroy.argtypes = [vp]
        R.hipGraphDestroy.argtypes = [vp]
        _rt = R
    return _rt


H2D, D2H, D2D = 1, 2, 3


def _ck(rc, what):
    if rc != 0:
        raise RuntimeError(f"{what}: {rt().hipGetErrorString(rc).decode()}")


class DeviceArray:
    """A device allocation with a dtype and shape (numpy on the host side)."""

    def __init__(self, shape, dtype):
        self.shape = tuple(shape) if isinstance(shape, (tuple, list)) else (int(shape),)
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape)) * self.dtype.itemsize
        p = ctypes.c_void_p()
        _ck(rt().hipMalloc(ctypes.byref(p), max(self.nbytes, 1)), "hipMalloc")
        self.ptr = p.value

    @staticmethod
    def from_numpy(a: np.ndarray) -> "DeviceArray":
        a = np.ascontiguousarray(a)
        d = DeviceArray(a.shape, a.dtype)
        _ck(rt().hipMemcpy(d.ptr, a.ctypes.data, a.nbytes, H2D), "hipMemcpy H2D")
        return d

    def numpy(self) -> np.ndarray:
        out = np.empty(self.shape, self.dtype)
        _ck(rt().hipMemcpy(out.ctypes.data, self.ptr, self.nbytes, D2H), "hipMemcpy D2H")
        return out

    def free(self):
        if self.ptr:
            rt().hipFree(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Event:
    def __init__(self):
        e = ctypes.c_void_p()
        _ck(rt().hipEventCreate(ctypes.byref(e)), "hipEventCreate")
        self.e = e.value

    def record(self, stream: int):
        _ck(rt().hipEventRecord(self.e, stream), "hipEventRecord")

    def synchronize(self):
        _ck(rt().hipEventSynchronize(self.e), "hipEventSynchronize")

    def elapsed_ms(self, end: "Event") -> float:
        ms = ctypes.c_float()
        _ck(rt().hipEventElapsedTime(ctypes.byref(ms), self.e, end.e), "hipEventElapsedTime")
        return ms.value

    def __del__(self):
        try:
            rt().hipEventDestroy(self.e)
        except Exception:
            pass


def copy_d2d(dst: "DeviceArray", src: "DeviceArray", nbytes: int):
    _ck(rt().hipMemcpy(dst.ptr, src.ptr, nbytes, D2D), "hipMemcpy D2D")


def synchronize():
    _ck(rt().hipDeviceSynchronize(), "hipDeviceSynchronize")


CAPTURE_THREAD_LOCAL = 1  # hipStreamCaptureModeThreadLocal


class Graph:
    """A HIP graph captured from the work `fn` enqueues on `stream` (run
    once, under capture; nothing executes until launch)."""

    def __init__(self, stream: int, fn):
        R = rt()
        self.exec, self.stream = None, stream
        _ck(R.hipStreamBeginCapture(stream, CAPTURE_THREAD_LOCAL), "hipStreamBeginCapture")
        err = None
        try:
            fn()
        except Exception as e:  # end the capture before reporting
            err = e
        g = ctypes.c_void_p()
        rc = R.hipStreamEndCapture(stream, ctypes.byref(g))
        if err is not None:
            if g.value:
                R.hipGraphDestroy(g)
            raise err
        _ck(rc, "hipStreamEndCapture")
        ex = ctypes.c_void_p()
        rc = R.hipGraphInstantiate(ctypes.byref(ex), g, None, None, 0)
        R.hipGraphDestroy(g)
        _ck(rc, "hipGraphInstantiate")
        self.exec = ex.value

    def launch(self):
        _ck(rt().hipGraphLaunch(self.exec, self.stream), "hipGraphLaunch")

    def close(self):
        if self.exec:
            rt().hipStreamSynchronize(self.stream)
            rt().hipGraphExecDestroy(self.exec)
            self.exec = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
