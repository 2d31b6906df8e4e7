"""Feature-major BSGS diagonal packers on the device (counterparts of the
reference's Triton packers, llama3fhe/operators/linear/gpu_packer.py:49-424).

``row(g, b)[slot] = W[(f - (giant_base + g) B) mod D, (f + b) mod D]`` with
``f = slot // token_lanes`` (the layout of reference
operators/linear/weight.py:18-47).  A packer returns a DiagonalChunk: the
diagonals are never materialised in HBM; ConstantBundle.plaintext encodes
them straight from the resident weight (one HIP gather feeding the encoder's
FFT), so pack and encode are one device pass.
"""

from __future__ import annotations

import ctypes

import numpy as np

from . import _native
from ._native import check, lib, ptr_array
from .tensor import DeviceTensor

_DTYPE_CODES = {np.dtype(np.float64): 0, np.dtype(np.float32): 1, np.dtype(np.complex128): 2}


def _geometry(slots, dimension, token_lanes, baby_steps, giant_base, giant_count):
    slots, dimension, token_lanes = int(slots), int(dimension), int(token_lanes)
    baby_steps, giant_base, giant_count = int(baby_steps), int(giant_base), int(giant_count)
    if slots <= 0 or dimension <= 0 or token_lanes <= 0:
        raise ValueError("slots/dimension/token_lanes must be positive.")
    if dimension * token_lanes != slots:
        raise ValueError("token-lane packing requires dimension*token_lanes == slots, got "
                         f"{dimension}*{token_lanes} != {slots}.")
    if baby_steps <= 0 or giant_base < 0 or giant_count <= 0:
        raise ValueError("baby_steps/giant_count must be positive and giant_base non-negative.")
    return slots, dimension, token_lanes, baby_steps, giant_base, giant_count


class DiagonalChunk:
    """``giant_count * baby_steps`` diagonal rows of ``slots`` complex values,
    encoded on demand (``encode``); shape/dtype describe the logical block."""

    dtype = np.dtype(np.complex128)

    def __init__(self, encoder, slots: int, rows: int, keep=()):
        self._encoder = encoder
        self._keep = keep  # device tensors that must outlive the chunk
        self.shape = (int(rows), int(slots))

    def encode(self, context, *, limbs: int, scale: float, is_ext: bool = False) -> list:
        return self._encoder(context, int(limbs), float(scale), bool(is_ext))

    def __array__(self, dtype=None, copy=None):
        raise TypeError("diagonal chunks are encoded on the device; pass them to "
                        "ConstantBundle (PackedRaw / UnpackedRaw)")


def _wrap_outputs(context, handles, rows):
    from .fhe import Ciphertext

    return [Ciphertext(context, handles[i]) for i in range(rows)]


def pack_token_lane_bsgs_weight_chunk(weight, *, slots: int, dimension: int, token_lanes: int,
                                      baby_steps: int, giant_base: int, giant_count: int,
                                      device: str = "cuda", block_size: int = 256):
    """Diagonals of a device-resident square weight (float64, float32 or
    complex128) (reference gpu_packer.py:49-177)."""
    slots, D, lanes, B, g0, G = _geometry(slots, dimension, token_lanes, baby_steps, giant_base,
                                          giant_count)
    if not isinstance(weight, DeviceTensor):
        raise TypeError(f"the token-lane packer expects a device tensor, got {type(weight)}.")
    if tuple(int(v) for v in weight.shape) != (D, D):
        raise ValueError(f"weight must have shape {(D, D)}, got {tuple(weight.shape)}.")
    if weight.stride(0) != D or weight.stride(1) != 1:
        raise ValueError("weight must be row-major contiguous")
    if weight.dtype not in _DTYPE_CODES:
        weight = weight.to(dtype=np.float64)
    code = _DTYPE_CODES[np.dtype(weight.dtype)]
    rows = G * B

    def encoder(context, limbs, scale, is_ext):
        out = (ctypes.c_void_p * rows)()
        check(lib.ckks_encode_token_lane(context.handle, weight.handle, code, D, lanes, B, g0, G,
                                         slots, limbs, scale, int(is_ext), out))
        return _wrap_outputs(context, out, rows)

    return DiagonalChunk(encoder, slots, rows, keep=(weight,))


_METADATA = ("real_source", "real_row", "real_scale", "imag_source", "imag_row", "imag_scale",
             "column", "column_scale")


def pack_structured_token_lane_bsgs_weight_chunk(sources, metadata, *, slots: int,
                                                 dimension: int, token_lanes: int,
                                                 baby_steps: int, giant_base: int,
                                                 giant_count: int, device: str = "cuda",
                                                 block_size: int = 256):
    """Diagonals of a structured physical matrix read from 1..3 device-resident
    real sources through the row/column maps (reference gpu_packer.py:180-424,
    structured_weight.py:1-20); every map index is checked on the host."""
    slots, D, lanes, B, g0, G = _geometry(slots, dimension, token_lanes, baby_steps, giant_base,
                                          giant_count)
    sources = tuple(sources)
    if not 1 <= len(sources) <= 3:
        raise ValueError("the structured packer requires one to three sources.")
    for i, src in enumerate(sources):
        if not isinstance(src, DeviceTensor):
            raise ValueError(f"structured source {i} must be a device tensor.")
        if src.ndim != 2:
            raise ValueError(f"structured source {i} must be rank two, got {src.shape}.")
    dtype = np.dtype(sources[0].dtype)
    if any(np.dtype(s.dtype) != dtype for s in sources):
        raise TypeError("structured sources must use one common dtype.")
    if dtype not in (np.dtype(np.float32), np.dtype(np.float64)):
        raise TypeError(f"structured sources must use float32 or float64, got {dtype}.")
    missing = [k for k in _METADATA if k not in metadata]
    if missing:
        raise ValueError(f"structured metadata is missing {missing}.")
    host = {k: np.asarray(metadata[k]).reshape(-1) for k in _METADATA}
    for k, v in host.items():
        if v.shape != (D,):
            raise ValueError(f"structured metadata {k!r} must have shape {(D,)}, got {v.shape}.")
    index_maps = np.ascontiguousarray(np.stack(
        [host[k].astype(np.int64) for k in ("real_source", "real_row", "imag_source",
                                            "imag_row", "column")]))
    scale_maps = np.ascontiguousarray(np.stack(
        [host[k].astype(np.float64) for k in ("real_scale", "imag_scale", "column_scale")]))
    shapes = np.asarray([[int(s.shape[0]), int(s.shape[1])] for s in sources], dtype=np.int64)
    strides = np.asarray([[s.stride(0), s.stride(1)] for s in sources], dtype=np.int64)
    fp32 = int(dtype == np.dtype(np.float32))
    rows = G * B

    def encoder(context, limbs, scale, is_ext):
        out = (ctypes.c_void_p * rows)()
        check(lib.ckks_encode_structured(
            context.handle, ptr_array([s.handle for s in sources]), len(sources), fp32,
            shapes.ctypes.data_as(_native.I64P), strides.ctypes.data_as(_native.I64P),
            index_maps.ctypes.data_as(_native.I64P), scale_maps.ctypes.data_as(_native.DP),
            D, lanes, B, g0, G, slots, limbs, scale, int(is_ext), out))
        return _wrap_outputs(context, out, rows)

    return DiagonalChunk(encoder, slots, rows, keep=sources)


__all__ = ["DiagonalChunk", "pack_structured_token_lane_bsgs_weight_chunk",
           "pack_token_lane_bsgs_weight_chunk"]
