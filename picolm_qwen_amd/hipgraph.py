"""Stream capture of library calls into a HIP graph, for callers that replay a
fixed sequence of launches (one decode step of every layer, say) without the
host cost of each launch.

The calls to capture must allocate nothing and synchronise nothing:
pqa_decode_noalloc is the entry point made for this (its split partials live
in a static device array). A captured decode step is tied to its position
(the launch shapes and arguments depend on it), so a caller keeps one graph
per position, or re-captures. Replaying a step appends the same K/V row again
(the same bits), so replays of one graph are idempotent.

This is plain HIP runtime API through ctypes, on the runtime the process has
already loaded (libamdhip64.so.7, the one libpqa.so links)."""
from __future__ import annotations

import ctypes as C

_hip = None

CAPTURE_THREAD_LOCAL = 1  # hipStreamCaptureModeThreadLocal


def hip() -> C.CDLL:
    global _hip
    if _hip is None:
        L = C.CDLL("libamdhip64.so.7")
        vp = C.c_void_p
        L.hipStreamBeginCapture.argtypes = [vp, C.c_int]
        L.hipStreamEndCapture.argtypes = [vp, C.POINTER(vp)]
        L.hipGraphInstantiate.argtypes = [C.POINTER(vp), vp, C.POINTER(vp), C.c_char_p, C.c_size_t]
        L.hipGraphLaunch.argtypes = [vp, vp]
        L.hipGraphExecDestroy.argtypes = [vp]
        L.hipGraphDestroy.argtypes = [vp]
        L.hipGetErrorString.restype = C.c_char_p
        L.hipGetErrorString.argtypes = [C.c_int]
        _hip = L
    return _hip


def _check(rc: int, what: str) -> None:
    if rc != 0:
        raise RuntimeError(f"{what}: hip error {rc} ({hip().hipGetErrorString(rc).decode()})")


class Graph:
    """Captures the launches fn() issues on `stream` (a hipStream_t as an int
    or c_void_p, e.g. PicoAttention's or pqa_stream's) into an instantiated
    graph; launch() replays them on a stream."""

    def __init__(self, stream, fn):
        L = hip()
        self.graph = C.c_void_p()
        self.exec = C.c_void_p()
        s = C.c_void_p(stream.value if isinstance(stream, C.c_void_p) else stream)
        _check(L.hipStreamBeginCapture(s, CAPTURE_THREAD_LOCAL), "hipStreamBeginCapture")
        err = None
        try:
            fn()
        except BaseException as e:  # end the capture before re-raising
            err = e
        rc = L.hipStreamEndCapture(s, C.byref(self.graph))
        if err is not None:
            if self.graph:
                L.hipGraphDestroy(self.graph)
            raise err
        _check(rc, "hipStreamEndCapture")
        _check(L.hipGraphInstantiate(C.byref(self.exec), self.graph, None, None, 0), "hipGraphInstantiate")

    def launch(self, stream) -> None:
        s = C.c_void_p(stream.value if isinstance(stream, C.c_void_p) else stream)
        _check(hip().hipGraphLaunch(self.exec, s), "hipGraphLaunch")

    def close(self) -> None:
        L = hip()
        if self.exec:
            L.hipGraphExecDestroy(self.exec)
            self.exec = C.c_void_p()
        if self.graph:
            L.hipGraphDestroy(self.graph)
            self.graph = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
