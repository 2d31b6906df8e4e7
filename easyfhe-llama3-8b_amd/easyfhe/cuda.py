"""Device module: synchronisation, timing events and allocator control
(reference backend.py:361-390, operators/linear/operator.py:273-291), and the
device queries the reference's Triton bridge reads
(operators/linear/gpu_packer.py:35-45: current device, capability, stream).
This backend drives one GPU, device 0."""

from __future__ import annotations

import ctypes

from . import _native
from ._native import check, lib


def _contexts():
    from .fhe import _live_contexts

    return [c for c in list(_live_contexts) if getattr(c, "_h", None)]


def is_available() -> bool:
    return True


def device_count() -> int:
    return 1


def current_device() -> int:
    return 0


def set_device(index) -> None:
    if int(getattr(index, "index", index) or 0) != 0:
        raise ValueError(f"this backend drives device 0 only, not {index!r}")


def get_device_capability(index=None) -> tuple[int, int]:
    """gfx950 (MI355X) as (major, minor) = (9, 5)."""
    set_device(0 if index is None else index)
    return (9, 5)


class Stream:
    """The current context's HIP stream; ``cuda_stream`` is the hipStream_t."""

    def __init__(self, context=None):
        from .fhe import current_context

        ctx = context if context is not None else current_context()
        h = ctypes.c_void_p()
        check(lib.ckks_context_stream(ctx.handle, ctypes.byref(h)))
        self.cuda_stream = int(h.value or 0)
        self._ctx = ctx

    def synchronize(self) -> None:
        self._ctx.synchronize()


def current_stream(device=None) -> Stream:
    set_device(0 if device is None else device)
    return Stream()


def synchronize() -> None:
    for ctx in _contexts():
        ctx.synchronize()


def empty_cache() -> None:
    for ctx in _contexts():
        ctx.empty_cache()


def memory_info() -> dict[str, int]:
    total = {"live_bytes": 0, "cached_bytes": 0}
    for ctx in _contexts():
        for k, v in ctx.memory_info().items():
            total[k] += v
    return total


class Event:
    """Timing event on the current context's stream."""

    def __init__(self, enable_timing: bool = False, context=None):
        from .fhe import current_context

        self._ctx = context if context is not None else current_context()
        h = ctypes.c_void_p()
        check(lib.ckks_event_create(self._ctx.handle, ctypes.byref(h)))
        self._h = h.value

    def record(self) -> None:
        check(lib.ckks_event_record(self._h))

    def synchronize(self) -> None:
        self._ctx.synchronize()

    def elapsed_time(self, end: "Event") -> float:
        ms = ctypes.c_float()
        check(lib.ckks_event_elapsed_ms(self._h, end._h, ctypes.byref(ms)))
        return float(ms.value)

    def __del__(self):
        try:
            if self._h:
                lib.ckks_event_destroy(self._h)
                self._h = None
        except Exception:
            pass
