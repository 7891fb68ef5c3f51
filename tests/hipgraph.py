"""Stream capture of library calls into a HIP graph, through ctypes on the
HIP runtime (test helper: the library itself never captures).

    with Capture(ctx.stream) as cap:
        ctx.linear(desc)          # recorded, not run
    cap.replay()                  # runs the recorded launches on the stream
"""
from __future__ import annotations

import ctypes

_hip = None

# hipStreamCaptureModeRelaxed: other threads may call unsafe APIs meanwhile;
# the capture itself still refuses allocation on the captured stream.
CAPTURE_MODE_RELAXED = 2


def hip() -> ctypes.CDLL:
    global _hip
    if _hip is None:
        L = ctypes.CDLL("libamdhip64.so")
        vp = ctypes.c_void_p
        L.hipStreamBeginCapture.argtypes = [vp, ctypes.c_int]
        L.hipStreamEndCapture.argtypes = [vp, ctypes.POINTER(vp)]
        L.hipGraphInstantiate.argtypes = [ctypes.POINTER(vp), vp, vp, ctypes.c_char_p, ctypes.c_size_t]
        L.hipGraphLaunch.argtypes = [vp, vp]
        L.hipGraphExecDestroy.argtypes = [vp]
        L.hipGraphDestroy.argtypes = [vp]
        L.hipStreamSynchronize.argtypes = [vp]
        _hip = L
    return _hip


class Capture:
    def __init__(self, stream: int):
        self.stream = ctypes.c_void_p(stream)
        self.graph = ctypes.c_void_p()
        self.exe = ctypes.c_void_p()

    def __enter__(self):
        rc = hip().hipStreamBeginCapture(self.stream, CAPTURE_MODE_RELAXED)
        assert rc == 0, f"hipStreamBeginCapture: {rc}"
        return self

    def __exit__(self, exc_type, exc, tb):
        rc = hip().hipStreamEndCapture(self.stream, ctypes.byref(self.graph))
        if exc_type is None:
            assert rc == 0, f"hipStreamEndCapture: {rc}"
            rc = hip().hipGraphInstantiate(ctypes.byref(self.exe), self.graph, None, None, 0)
            assert rc == 0, f"hipGraphInstantiate: {rc}"
        return False

    def replay(self) -> None:
        assert hip().hipGraphLaunch(self.exe, self.stream) == 0
        assert hip().hipStreamSynchronize(self.stream) == 0

    def close(self) -> None:
        if self.exe:
            hip().hipGraphExecDestroy(self.exe)
            self.exe = ctypes.c_void_p()
        if self.graph:
            hip().hipGraphDestroy(self.graph)
            self.graph = ctypes.c_void_p()
