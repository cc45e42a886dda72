"""Minimal ctypes access to HIP events (libamdhip64) for timing kernels on a given stream."""
from __future__ import annotations

import ctypes as C

_hip = None


def hip() -> C.CDLL:
    global _hip
    if _hip is None:
        lib = C.CDLL("libamdhip64.so")
        lib.hipEventCreate.argtypes = [C.POINTER(C.c_void_p)]
        lib.hipEventRecord.argtypes = [C.c_void_p, C.c_void_p]
        lib.hipEventSynchronize.argtypes = [C.c_void_p]
        lib.hipEventElapsedTime.argtypes = [C.POINTER(C.c_float), C.c_void_p, C.c_void_p]
        lib.hipEventDestroy.argtypes = [C.c_void_p]
        for f in ("hipEventCreate", "hipEventRecord", "hipEventSynchronize",
                  "hipEventElapsedTime", "hipEventDestroy"):
            getattr(lib, f).restype = C.c_int
        _hip = lib
    return _hip


class Event:
    """A HIP event recorded on an explicit stream (torch.cuda.Event only sees torch streams)."""

    def __init__(self) -> None:
        self.h = C.c_void_p()
        rc = hip().hipEventCreate(C.byref(self.h))
        if rc:
            raise RuntimeError(f"hipEventCreate failed ({rc})")

    def record(self, stream: int) -> None:
        rc = hip().hipEventRecord(self.h, C.c_void_p(stream))
        if rc:
            raise RuntimeError(f"hipEventRecord failed ({rc})")

    def synchronize(self) -> None:
        hip().hipEventSynchronize(self.h)

    def elapsed_ms(self, end: "Event") -> float:
        ms = C.c_float()
        rc = hip().hipEventElapsedTime(C.byref(ms), self.h, end.h)
        if rc:
            raise RuntimeError(f"hipEventElapsedTime failed ({rc})")
        return float(ms.value)

    def __del__(self) -> None:
        try:
            if self.h:
                hip().hipEventDestroy(self.h)
        except Exception:
            pass
