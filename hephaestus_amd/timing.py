"""Kernel-boundary timing with HIP events.

heph_profile_next_launch() makes the library launch its next main kernel
with hipExtLaunchKernel, which stamps a start and a stop event at the
kernel's own begin and end on the stream it runs on. KernelTimer keeps a
pool of such event pairs and sums their elapsed times after a sync.

The HIP runtime is reached through the process's already-loaded
libamdhip64 (torch loads it first), so events and streams are shared with
torch and with libhephfp8.so.
"""
from __future__ import annotations

import ctypes

import torch  # noqa: F401  (loads the process's HIP runtime first)

from . import _lib as L

_hip = None


def hip():
    global _hip
    if _hip is None:
        h = ctypes.CDLL("libamdhip64.so.7")
        h.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        h.hipEventCreate.restype = ctypes.c_int
        h.hipEventDestroy.argtypes = [ctypes.c_void_p]
        h.hipEventDestroy.restype = ctypes.c_int
        h.hipEventSynchronize.argtypes = [ctypes.c_void_p]
        h.hipEventSynchronize.restype = ctypes.c_int
        h.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p,
                                          ctypes.c_void_p]
        h.hipEventElapsedTime.restype = ctypes.c_int
        _hip = h
    return _hip


class KernelTimer:
    """Pairs of HIP events attached to successive main-kernel launches."""

    def __init__(self, n: int):
        self.pairs = []
        for _ in range(n):
            a, b = ctypes.c_void_p(), ctypes.c_void_p()
            if hip().hipEventCreate(ctypes.byref(a)) or hip().hipEventCreate(ctypes.byref(b)):
                raise RuntimeError("hipEventCreate failed")
            self.pairs.append((a, b))
        self.used = 0

    def arm(self) -> None:
        """Attach the next event pair to the next main kernel launch."""
        a, b = self.pairs[self.used]
        self.used += 1
        L.lib().heph_profile_next_launch(a, b)

    def durations_ms(self) -> list[float]:
        out = []
        for a, b in self.pairs[: self.used]:
            hip().hipEventSynchronize(b)
            ms = ctypes.c_float()
            if hip().hipEventElapsedTime(ctypes.byref(ms), a, b):
                raise RuntimeError("hipEventElapsedTime failed")
            out.append(ms.value)
        return out

    def reset(self) -> None:
        self.used = 0

    def close(self) -> None:
        for a, b in self.pairs:
            hip().hipEventDestroy(a)
            hip().hipEventDestroy(b)
        self.pairs = []
