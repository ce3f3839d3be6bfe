"""Device buffers for GPU tests, allocated through the HIP runtime that
libanima_hip links (ctypes on libamdhip64; no torch).

PyTorch bundles its own HIP runtime; once libanima_hip's runtime has taken
the GPU in a process, torch reports no GPU.  Tests that need raw device
memory therefore stay on the library's runtime.
"""
import ctypes as ct

import numpy as np

from anima_hip import _lib

_H2D, _D2H = 1, 2
_hip = None


def hip():
    global _hip
    if _hip is None:
        _lib.load()  # resolves libamdhip64.so.7; the dlopen below returns that same object
        h = ct.CDLL("libamdhip64.so.7")
        h.hipMalloc.argtypes = [ct.POINTER(ct.c_void_p), ct.c_size_t]
        h.hipMemcpy.argtypes = [ct.c_void_p, ct.c_void_p, ct.c_size_t, ct.c_int]
        h.hipFree.argtypes = [ct.c_void_p]
        for f in (h.hipMalloc, h.hipMemcpy, h.hipFree, h.hipDeviceSynchronize):
            f.restype = ct.c_int
        _hip = h
    return _hip


def _ok(code, what):
    if code != 0:
        raise RuntimeError(f"{what} failed with hipError {code}")


class DevBuf:
    """`nbytes` of device memory; freed on close() or garbage collection."""

    def __init__(self, nbytes):
        self.nbytes = int(nbytes)
        self.ptr = ct.c_void_p()
        _ok(hip().hipMalloc(ct.byref(self.ptr), max(self.nbytes, 256)), "hipMalloc")

    @property
    def addr(self):
        return self.ptr.value

    @classmethod
    def of(cls, arr):
        arr = np.ascontiguousarray(arr)
        b = cls(arr.nbytes)
        _ok(hip().hipMemcpy(b.addr, arr.ctypes.data, arr.nbytes, _H2D), "hipMemcpy H2D")
        return b

    def put(self, arr, offset):
        """Copy `arr` to bytes [offset, offset + arr.nbytes) of the buffer."""
        arr = np.ascontiguousarray(arr)
        assert 0 <= offset and offset + arr.nbytes <= self.nbytes
        _ok(hip().hipMemcpy(self.addr + offset, arr.ctypes.data, arr.nbytes, _H2D),
            "hipMemcpy H2D")

    def get(self, shape, dtype=np.float32):
        out = np.empty(shape, dtype)
        assert out.nbytes <= self.nbytes
        _ok(hip().hipDeviceSynchronize(), "hipDeviceSynchronize")
        _ok(hip().hipMemcpy(out.ctypes.data, self.addr, out.nbytes, _D2H), "hipMemcpy D2H")
        return out

    def close(self):
        if self.ptr.value:
            hip().hipFree(self.ptr)
            self.ptr = ct.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class CapturedCall:
    """One HIP graph captured on a stream of its own (hipStreamBeginCapture,
    thread-local mode) around `fn(stream)`, instantiated and replayable."""

    MODE_THREAD_LOCAL = 1

    def __init__(self, fn):
        h = hip()
        for f in (h.hipStreamCreate, h.hipStreamBeginCapture, h.hipStreamEndCapture,
                  h.hipGraphInstantiate, h.hipGraphLaunch, h.hipStreamSynchronize,
                  h.hipGraphExecDestroy, h.hipGraphDestroy, h.hipStreamDestroy):
            f.restype = ct.c_int
        self.stream = ct.c_void_p()
        _ok(h.hipStreamCreate(ct.byref(self.stream)), "hipStreamCreate")
        self.graph, self.exec = ct.c_void_p(), ct.c_void_p()
        _ok(h.hipStreamBeginCapture(self.stream, self.MODE_THREAD_LOCAL), "hipStreamBeginCapture")
        try:
            fn(self.stream)
        finally:
            end = h.hipStreamEndCapture(self.stream, ct.byref(self.graph))
        _ok(end, "hipStreamEndCapture")
        _ok(h.hipGraphInstantiate(ct.byref(self.exec), self.graph, None, None, ct.c_size_t(0)),
            "hipGraphInstantiate")

    def replay(self):
        h = hip()
        _ok(h.hipGraphLaunch(self.exec, self.stream), "hipGraphLaunch")
        _ok(h.hipStreamSynchronize(self.stream), "hipStreamSynchronize")

    def close(self):
        h = hip()
        if self.exec.value:
            h.hipGraphExecDestroy(self.exec)
            self.exec = ct.c_void_p()
        if self.graph.value:
            h.hipGraphDestroy(self.graph)
            self.graph = ct.c_void_p()
        if self.stream.value:
            h.hipStreamDestroy(self.stream)
            self.stream = ct.c_void_p()
