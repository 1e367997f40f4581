"""Minimal HIP runtime binding (events, synchronisation) for timing.

Events are recorded on the stream the backend launches its kernels on
(coli_hip_stream), so they bracket exactly that stream's work.
"""
import ctypes as C
import os

_lib = None


def lib():
    global _lib
    if _lib is None:
        for name in ("libamdhip64.so", "/opt/rocm/lib/libamdhip64.so"):
            try:
                _lib = C.CDLL(name, mode=C.RTLD_GLOBAL)
                break
            except OSError:
                continue
        if _lib is None:
            raise RuntimeError("libamdhip64.so not found")
        _lib.hipEventCreate.argtypes = [C.POINTER(C.c_void_p)]
        _lib.hipEventRecord.argtypes = [C.c_void_p, C.c_void_p]
        _lib.hipEventSynchronize.argtypes = [C.c_void_p]
        _lib.hipEventElapsedTime.argtypes = [C.POINTER(C.c_float), C.c_void_p, C.c_void_p]
        _lib.hipEventDestroy.argtypes = [C.c_void_p]
        _lib.hipStreamSynchronize.argtypes = [C.c_void_p]
        _lib.hipDeviceSynchronize.argtypes = []
        _lib.hipMemcpyAsync.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int, C.c_void_p]
        _lib.hipStreamBeginCapture.argtypes = [C.c_void_p, C.c_int]
        _lib.hipStreamEndCapture.argtypes = [C.c_void_p, C.POINTER(C.c_void_p)]
        _lib.hipGraphInstantiate.argtypes = [C.POINTER(C.c_void_p), C.c_void_p, C.c_void_p, C.c_char_p, C.c_size_t]
        _lib.hipGraphLaunch.argtypes = [C.c_void_p, C.c_void_p]
        _lib.hipGraphExecDestroy.argtypes = [C.c_void_p]
        _lib.hipGraphDestroy.argtypes = [C.c_void_p]
    return _lib


def check(err, what):
    if err != 0:
        raise RuntimeError(f"{what} failed: hip error {err}")


class Event:
    def __init__(self):
        self.h = C.c_void_p()
        check(lib().hipEventCreate(C.byref(self.h)), "hipEventCreate")

    def record(self, stream):
        check(lib().hipEventRecord(self.h, stream), "hipEventRecord")

    def elapsed_ms(self, later):
        ms = C.c_float()
        check(lib().hipEventSynchronize(later.h), "hipEventSynchronize")
        check(lib().hipEventElapsedTime(C.byref(ms), self.h, later.h), "hipEventElapsedTime")
        return ms.value

    def __del__(self):
        if _lib is not None and self.h:
            _lib.hipEventDestroy(self.h)


def device_sync():
    check(lib().hipDeviceSynchronize(), "hipDeviceSynchronize")


def stream_sync(stream):
    check(lib().hipStreamSynchronize(stream), "hipStreamSynchronize")


def copy_d2d_async(dst, src, nbytes, stream):
    """Device-to-device copy on `stream` (hipMemcpyDeviceToDevice = 3)."""
    check(lib().hipMemcpyAsync(dst, src, nbytes, 3, stream), "hipMemcpyAsync")


class Graph:
    """A HIP graph captured from everything enqueued on `stream` inside the
    `with` block (thread-local capture mode), then instantiated for replay."""

    def __init__(self, stream):
        self.stream = stream
        self.graph = C.c_void_p()
        self.exec = C.c_void_p()

    def __enter__(self):
        check(lib().hipStreamBeginCapture(self.stream, 1), "hipStreamBeginCapture")
        return self

    def __exit__(self, exc_type, exc, tb):
        err = lib().hipStreamEndCapture(self.stream, C.byref(self.graph))
        if exc_type is None:
            check(err, "hipStreamEndCapture")
            check(lib().hipGraphInstantiate(C.byref(self.exec), self.graph, None, None, 0), "hipGraphInstantiate")
        return False

    def launch(self):
        check(lib().hipGraphLaunch(self.exec, self.stream), "hipGraphLaunch")

    def __del__(self):
        if _lib is not None:
            if self.exec:
                _lib.hipGraphExecDestroy(self.exec)
            if self.graph:
                _lib.hipGraphDestroy(self.graph)
