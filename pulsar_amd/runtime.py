"""The device-runtime pieces of the reference's kernel crate that the hot path
relies on, over the HIP runtime libpulsar_moe.so is linked against:

  sync()          kernels::sync, a device-wide synchronize
                  (crates/kernels/src/lib.rs:742-744)
  Graph.capture   records every launch the callable makes on this thread's
                  per-thread default stream, capture mode thread-local, and
                  instantiates it; Graph.launch replays it on that stream
                  (crates/kernels/src/lib.rs:746-811)
  Event           a HIP event recorded on the per-thread default stream, for
                  timing launches on the stream they run on

Every pulsar_* launch goes to the calling thread's per-thread default stream
(hipStreamPerThread) unless pulsar_set_stream chose another, as the
reference's kernels compile with --default-stream=per-thread
(crates/kernels/build.rs:42-48). The HIP functions are looked up through the
library's own handle, so they are those of the runtime it is bound to.
"""
from __future__ import annotations

import ctypes

from . import _lib

STREAM_PER_THREAD = 2  # hipStreamPerThread
CAPTURE_THREAD_LOCAL = 1  # hipStreamCaptureModeThreadLocal

_vp, _int = ctypes.c_void_p, ctypes.c_int
_SIGS = {
    "hipDeviceSynchronize": [],
    "hipStreamSynchronize": [_vp],
    "hipGetErrorString": None,
    "hipEventCreate": [ctypes.POINTER(_vp)],
    "hipEventDestroy": [_vp],
    "hipEventRecord": [_vp, _vp],
    "hipEventSynchronize": [_vp],
    "hipEventElapsedTime": [ctypes.POINTER(ctypes.c_float), _vp, _vp],
    "hipStreamBeginCapture": [_vp, _int],
    "hipStreamEndCapture": [_vp, ctypes.POINTER(_vp)],
    "hipGraphInstantiateWithFlags": [ctypes.POINTER(_vp), _vp, ctypes.c_ulonglong],
    "hipGraphLaunch": [_vp, _vp],
    "hipGraphDestroy": [_vp],
    "hipGraphExecDestroy": [_vp],
}
_rt = None


class HipError(RuntimeError):
    """A HIP runtime call failed (the reference's check_rt error,
    crates/kernels/src/lib.rs:200-210)."""


def _hip():
    global _rt
    if _rt is None:
        lib = _lib.load()
        for name, args in _SIGS.items():
            fn = getattr(lib, name)
            if name == "hipGetErrorString":
                fn.argtypes, fn.restype = [_int], ctypes.c_char_p
            else:
                fn.argtypes, fn.restype = args, _int
        _rt = lib
    return _rt


def _check(err: int, what: str) -> None:
    if err != 0:
        msg = _hip().hipGetErrorString(err).decode(errors="replace")
        raise HipError(f"{what}: {msg} ({err})")


def sync() -> None:
    """Waits for every launch on the device (kernels::sync)."""
    _check(_hip().hipDeviceSynchronize(), "hipDeviceSynchronize")


def stream_sync(stream: int = STREAM_PER_THREAD) -> None:
    _check(_hip().hipStreamSynchronize(stream), "hipStreamSynchronize")


class Event:
    """A timing event recorded on a stream (default: the per-thread one)."""

    def __init__(self):
        h = _vp()
        _check(_hip().hipEventCreate(ctypes.byref(h)), "hipEventCreate")
        self.h = h

    def record(self, stream: int = STREAM_PER_THREAD) -> None:
        _check(_hip().hipEventRecord(self.h, stream), "hipEventRecord")

    def synchronize(self) -> None:
        _check(_hip().hipEventSynchronize(self.h), "hipEventSynchronize")

    def elapsed_ms(self, end: "Event") -> float:
        """Milliseconds from this event to `end` (both recorded and done)."""
        ms = ctypes.c_float()
        _check(_hip().hipEventElapsedTime(ctypes.byref(ms), self.h, end.h), "hipEventElapsedTime")
        return float(ms.value)

    def __del__(self):
        if getattr(self, "h", None) and _rt is not None:
            _rt.hipEventDestroy(self.h)
            self.h = None


class Graph:
    """An instantiated HIP graph of launches made on the per-thread default
    stream (crates/kernels/src/lib.rs:764-811)."""

    def __init__(self, exec_handle):
        self._exec = exec_handle

    @classmethod
    def capture(cls, fn) -> "Graph":
        """Records every pulsar_* launch `fn` makes on this thread's default
        stream (nothing executes during capture) and instantiates it. If `fn`
        raises, the capture is ended and the exception propagates."""
        hip = _hip()
        _check(hip.hipStreamBeginCapture(STREAM_PER_THREAD, CAPTURE_THREAD_LOCAL), "graph begin capture")
        graph = _vp()
        try:
            fn()
        except BaseException:
            if hip.hipStreamEndCapture(STREAM_PER_THREAD, ctypes.byref(graph)) == 0 and graph:
                hip.hipGraphDestroy(graph)
            raise
        _check(hip.hipStreamEndCapture(STREAM_PER_THREAD, ctypes.byref(graph)), "graph end capture")
        exec_h = _vp()
        inst = hip.hipGraphInstantiateWithFlags(ctypes.byref(exec_h), graph, 0)
        hip.hipGraphDestroy(graph)
        _check(inst, "graph instantiate")
        return cls(exec_h)

    def launch(self) -> None:
        """Replays the recorded chain on this thread's default stream."""
        _check(_hip().hipGraphLaunch(self._exec, STREAM_PER_THREAD), "graph launch")

    def __del__(self):
        if getattr(self, "_exec", None) and _rt is not None:
            _rt.hipGraphExecDestroy(self._exec)
            self._exec = None
