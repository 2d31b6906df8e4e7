"""MI355X (gfx950) RNS-CKKS backend with the module surface of ``easyfhe``.

The reference's operators import ``easyfhe``, ``easyfhe.fhe``,
``easyfhe.bs.openfhe`` and ``easyfhe.cuda`` (reference llama3fhe/backend.py:17-19,
operators/primitives.py:16); this package provides those names on top of the
C ABI in include/ckks_mi355x.h.  Host arrays are numpy arrays (the tensor
bridge of reference backend.py:274-284 uses ``from_numpy`` and an optional
``.to(device)``).
"""

from __future__ import annotations

import types

import numpy as np

from . import _native  # noqa: F401  (loads the library; raises if it is missing)
from . import bs, cuda, fhe, packing
from .tensor import DeviceTensor, HostTensor

# the reference's Triton bridge reads torch.version.hip (gpu_packer.py:16-19)
version = types.SimpleNamespace(hip="7.2", cuda=None)

complex128 = np.complex128
float64 = np.float64
float32 = np.float32


def from_numpy(array) -> HostTensor:
    """Host tensor; ``.to("cuda")`` moves it to the current context's HBM."""
    return HostTensor(array)


def is_tensor(value) -> bool:
    return isinstance(value, (np.ndarray, HostTensor, DeviceTensor))


def empty(shape, dtype=np.float64, device=None):
    return np.empty(shape, dtype=dtype)


def get_device_module(device: str):
    if str(device).startswith(("cuda", "hip", "gpu")):
        return cuda
    raise ValueError(f"unsupported device {device!r}: this backend runs on the GPU only")


__all__ = ["bs", "complex128", "cuda", "empty", "fhe", "float32", "float64", "from_numpy",
           "get_device_module", "is_tensor", "version"]
