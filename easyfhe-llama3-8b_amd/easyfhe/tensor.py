"""Host and device arrays with the few torch-like methods the reference's
weight path uses (``from_numpy(x).to(device)``, ``is_cuda``, ``shape``,
``dtype``, ``ndim``, ``stride(dim)``; reference
llama3fhe/operators/linear/weight.py:186-231, gpu_packer.py:79-97).

A DeviceTensor owns a ``ckks_tensor`` of the current context: raw bytes in
HBM that the diagonal packers read.
"""

from __future__ import annotations

import ctypes

import numpy as np

from . import _native
from ._native import check, lib


class HostTensor:
    """A numpy array that can be moved to the device."""

    is_cuda = False

    def __init__(self, array):
        self._a = np.ascontiguousarray(np.asarray(array))

    def __array__(self, dtype=None, copy=None):
        return self._a if dtype is None else self._a.astype(dtype)

    @property
    def shape(self):
        return self._a.shape

    @property
    def dtype(self):
        return self._a.dtype

    @property
    def ndim(self) -> int:
        return self._a.ndim

    def stride(self, dim: int) -> int:
        return self._a.strides[dim] // self._a.itemsize

    def numpy(self) -> np.ndarray:
        return self._a

    def to(self, device=None, dtype=None, context=None):
        a = self._a if dtype is None else self._a.astype(dtype)
        if device is None or str(device) == "cpu":
            return HostTensor(a)
        return DeviceTensor(a, context=context)


class DeviceTensor:
    """An array resident in the context's HBM."""

    is_cuda = True

    def __init__(self, array, context=None):
        from .fhe import current_context

        a = np.ascontiguousarray(np.asarray(array))
        if a.size == 0:
            raise ValueError("empty tensor")
        self.context = context if context is not None else current_context()
        self._shape = a.shape
        self._dtype = a.dtype
        self._strides = tuple(s // a.itemsize for s in a.strides)
        self.nbytes = int(a.nbytes)
        out = ctypes.c_void_p()
        check(lib.ckks_tensor_upload(self.context.handle, a.ctypes.data_as(ctypes.c_void_p),
                                     self.nbytes, ctypes.byref(out)))
        self._h = out.value

    @property
    def handle(self) -> int:
        if not self._h:
            raise RuntimeError("tensor was released")
        return self._h

    @property
    def shape(self):
        return self._shape

    @property
    def dtype(self):
        return self._dtype

    @property
    def ndim(self) -> int:
        return len(self._shape)

    def stride(self, dim: int) -> int:
        return self._strides[dim]

    def numpy(self) -> np.ndarray:
        out = np.empty(self._shape, dtype=self._dtype)
        check(lib.ckks_tensor_download(self.context.handle, self.handle,
                                       out.ctypes.data_as(ctypes.c_void_p), self.nbytes))
        return out

    cpu = numpy

    def __array__(self, dtype=None, copy=None):
        a = self.numpy()
        return a if dtype is None else a.astype(dtype)

    def to(self, device=None, dtype=None, context=None):
        if device is not None and str(device) == "cpu":
            return HostTensor(self.numpy() if dtype is None else self.numpy().astype(dtype))
        if dtype is not None and np.dtype(dtype) != self._dtype:
            return DeviceTensor(self.numpy().astype(dtype), context=self.context)
        return self

    def release(self) -> None:
        if getattr(self, "_h", None):
            lib.ckks_tensor_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.release()
        except Exception:
            pass


__all__ = ["DeviceTensor", "HostTensor"]
