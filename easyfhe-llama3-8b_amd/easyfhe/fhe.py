"""Homomorphic evaluation surface (the ``easyfhe.fhe`` names the reference calls).

Every function here forwards to the gfx950 library through the C ABI in
include/ckks_mi355x.h; there is no host arithmetic path.  Signatures follow
the reference's call sites (ciphertext arguments first, the native context
last before keyword options, a new owned object returned).  Invalid levels,
slot counts or states raise ``ValueError`` (the reference relies on that,
operators/nonlinear/bootstrap.py:434); other backend failures raise
``RuntimeError``.
"""

from __future__ import annotations

import atexit
import ctypes
import dataclasses
import hashlib
import itertools
import math
import weakref
from dataclasses import dataclass, field
from typing import Any, Iterable, Sequence

import numpy as np

from . import _native
from ._native import check, lib, ptr_array

# ---------------------------------------------------------------------------
# states and specs
# ---------------------------------------------------------------------------


@dataclass(frozen=True)
class CipherState:
    """Level/scale bookkeeping of a ciphertext or plaintext
    (reference operators/primitives.py:89-93, 140-144)."""

    cur_limbs: int
    scale_degree: int = 1
    scaling_factor: float | None = None

    def replace(self, **changes) -> "CipherState":
        return dataclasses.replace(self, **changes)


@dataclass
class CKKSContextSpec:
    """Context parameters (reference application/session.py:31-45)."""

    depth: int
    log_n: int
    dnum: int = 3
    dcrt_bits: int = 59
    first_mod: int = 60
    secret_key_dist: str = "SPARSE_TERNARY"
    scale_mode: str = "fixed"
    rescale_policy: str = "manual"
    rotations: Sequence[int] = ()
    auto_load_keys: bool = True
    seed: int = 0
    special_bits: int = 60
    hamming_weight: int = 192
    relin_key: bool = True


_SECRET_MODES = {"SPARSE_TERNARY": 0, "UNIFORM_TERNARY": 1}

# ---------------------------------------------------------------------------
# native context and objects
# ---------------------------------------------------------------------------

_live_contexts: "weakref.WeakSet[NativeContext]" = weakref.WeakSet()
_current: list = []


class NativeContext:
    """The device context: primes, tables, secret and evaluation keys.

    Attributes mirror the reference's native context: ``L`` (Q limbs),
    ``M`` (= 2N), ``logN``, ``max_slots``, ``device``, ``scale_at(limbs)`` and
    ``rescale_divisor_at(limbs)`` (reference backend.py:214-228,
    operators/nonlinear/polynomial.py:59).
    """

    def __init__(self, spec: CKKSContextSpec, device: str = "cuda"):
        dist = str(spec.secret_key_dist).upper()
        if dist not in _SECRET_MODES:
            raise ValueError(f"unsupported secret_key_dist {spec.secret_key_dist!r}")
        if str(spec.scale_mode) != "fixed":
            raise ValueError("only scale_mode='fixed' is supported")
        params = _native.ckks_params(
            log_n=int(spec.log_n),
            depth=int(spec.depth),
            dnum=int(spec.dnum),
            dcrt_bits=int(spec.dcrt_bits),
            first_mod=int(spec.first_mod),
            special_bits=int(spec.special_bits),
            secret_mode=_SECRET_MODES[dist],
            hamming_weight=int(spec.hamming_weight),
            seed=int(spec.seed) & (2**64 - 1),
        )
        handle = ctypes.c_void_p()
        check(lib.ckks_context_create(ctypes.byref(params), ctypes.byref(handle)))
        self._h = handle.value
        info = _native.ckks_context_info()
        check(lib.ckks_context_info_get(self._h, ctypes.byref(info)))
        self.N = int(info.N)
        self.logN = int(info.log_n)
        self.L = int(info.L)
        self.alpha = int(info.alpha)
        self.digit_size = int(info.digit_size)
        self.max_slots = int(info.max_slots)
        self.M = 2 * self.N
        self.device = str(device)
        self.spec = spec
        self._enc_ids = itertools.count(1)
        _live_contexts.add(self)
        _current.append(weakref.ref(self))

    # -- reference-visible attributes ------------------------------------------
    def scale_at(self, limbs: int) -> float:
        return float(lib.ckks_scale_at(self._h, int(limbs)))

    def rescale_divisor_at(self, limbs: int) -> float:
        return float(lib.ckks_rescale_divisor_at(self._h, int(limbs)))

    def clear_cuda_rotation_cache(self, keep_rotations: Iterable[int] = ()) -> None:
        keep = np.asarray(list(keep_rotations) or [0], dtype=np.int64)
        check(lib.ckks_clear_rotation_keys(self._h, keep.ctypes.data_as(_native.I64P),
                                           len(list(keep_rotations))))

    # -- extras ---------------------------------------------------------------------
    @property
    def handle(self) -> int:
        return self._h

    def primes(self) -> np.ndarray:
        out = np.zeros(self.L + self.alpha, dtype=np.uint64)
        check(lib.ckks_context_primes(self._h, out.ctypes.data_as(_native.U64P)))
        return out

    def secret(self) -> np.ndarray:
        out = np.zeros(self.N, dtype=np.int8)
        check(lib.ckks_context_secret(self._h, out.ctypes.data_as(ctypes.POINTER(ctypes.c_int8))))
        return out

    def galois_element(self, rotation: int) -> int:
        return int(lib.ckks_galois_element(self._h, int(rotation)))

    def generate_rotation_keys(self, rotations: Iterable[int]) -> None:
        rot = np.asarray(sorted({int(r) for r in rotations}), dtype=np.int64)
        if rot.size:
            check(lib.ckks_keygen_rotations(self._h, rot.ctypes.data_as(_native.I64P), rot.size))

    def generate_relin_key(self) -> None:
        check(lib.ckks_keygen_relin(self._h))

    def has_rotation_key(self, rotation: int) -> bool:
        return bool(lib.ckks_has_rotation_key(self._h, int(rotation)))

    def download_key(self, galois: int) -> np.ndarray:
        digits = ctypes.c_int()
        check(lib.ckks_key_download(self._h, int(galois), None, ctypes.byref(digits)))
        out = np.zeros((digits.value, 2, self.L + self.alpha, self.N), dtype=np.uint64)
        check(lib.ckks_key_download(self._h, int(galois), out.ctypes.data_as(_native.U64P), None))
        return out

    def next_encryption_id(self) -> int:
        return next(self._enc_ids)

    def synchronize(self) -> None:
        check(lib.ckks_synchronize(self._h))

    def audit(self, reset: bool = False) -> dict[str, float]:
        """Operation audit since the last reset (ckks_audit_read): key
        switches and their ciphertext / key bytes, plaintext and rescale
        bytes."""
        v = (ctypes.c_double * 5)()
        check(lib.ckks_audit_read(self._h, v, 1 if reset else 0))
        return {"keyswitches": v[0], "keyswitch_ct_bytes": v[1], "key_bytes": v[2],
                "plaintext_bytes": v[3], "rescale_bytes": v[4]}

    def memory_info(self) -> dict[str, int]:
        live, cached = ctypes.c_size_t(), ctypes.c_size_t()
        check(lib.ckks_memory_info(self._h, ctypes.byref(live), ctypes.byref(cached)))
        peak, seg, allocs = ctypes.c_size_t(), ctypes.c_size_t(), ctypes.c_uint64()
        check(lib.ckks_memory_stats(self._h, ctypes.byref(peak), ctypes.byref(seg),
                                    ctypes.byref(allocs)))
        return {"live_bytes": int(live.value), "cached_bytes": int(cached.value),
                "peak_live_bytes": int(peak.value), "segment_bytes": int(seg.value),
                "device_allocations": int(allocs.value)}

    def empty_cache(self) -> None:
        check(lib.ckks_empty_cache(self._h))

    def set_split_parts(self, parts: int) -> None:
        """Streams a batched key switch is split over (1 to the count the
        context was created with; 0 restores that count)."""
        check(lib.ckks_set_split_parts(self._h, int(parts)))

    def profile(self, enable: bool = True) -> None:
        """Start (or stop) recording device time per kernel group."""
        check(lib.ckks_profile_enable(self._h, int(bool(enable))))

    def profile_read(self) -> dict[str, dict[str, float]]:
        """Kernel groups recorded since the last read: launches, device
        milliseconds, algorithmic bytes and modular operations."""
        buf = ctypes.create_string_buffer(1 << 16)
        check(lib.ckks_profile_read(self._h, buf, len(buf)))
        out = {}
        for line in buf.value.decode().splitlines():
            name, calls, ms, nbytes, ops = line.split()
            out[name] = {"launches": int(calls), "ms": float(ms), "bytes": float(nbytes),
                         "ops": float(ops)}
        return out

    def close(self) -> None:
        if getattr(self, "_h", None):
            clear_plaintext_cache(self)
            lib.ckks_context_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def _close_all_contexts() -> None:
    # Destroy device contexts while the HIP runtime is still up; ciphertexts
    # collected later only drop their host records.
    for ctx in list(_live_contexts):
        ctx.close()


atexit.register(_close_all_contexts)


def current_context() -> NativeContext:
    while _current:
        ctx = _current[-1]()
        if ctx is not None and ctx._h:
            return ctx
        _current.pop()
    raise RuntimeError("no live easyfhe context")


class Ciphertext:
    """Owned device object: a ciphertext (2 or 3 polynomials), a plaintext
    (1 polynomial) or a scalar constant (per-limb values).

    ``state``, ``slots``, ``is_ext``, ``deep_copy()`` and ``release()`` follow
    the reference's usage (operators/primitives.py:115-150,
    backend.py:336-351)."""

    __slots__ = ("context", "_h", "_pinned", "__weakref__")

    def __init__(self, context: NativeContext, handle: int):
        self.context = context
        self._h = handle
        self._pinned = False  # held by the context's plaintext cache

    @property
    def handle(self) -> int:
        if not self._h:
            raise RuntimeError("ciphertext was released")
        return self._h

    def _info(self) -> _native.ckks_ct_info:
        info = _native.ckks_ct_info()
        check(lib.ckks_ct_info_get(self.handle, ctypes.byref(info)))
        return info

    @property
    def state(self) -> CipherState:
        info = self._info()
        return CipherState(cur_limbs=int(info.limbs), scale_degree=int(info.scale_degree),
                           scaling_factor=float(info.scale))

    @property
    def slots(self) -> int:
        return int(self._info().slots)

    @property
    def is_ext(self) -> bool:
        return bool(self._info().is_ext)

    @property
    def polys(self) -> int:
        return int(self._info().polys)

    @property
    def degree(self) -> int:
        return self.polys - 1

    def set_scale(self, scale: float, scale_degree: int | None = None) -> None:
        info = self._info()
        check(lib.ckks_ct_set_scale(self.handle, float(scale),
                                    int(info.scale_degree if scale_degree is None else scale_degree)))

    def deep_copy(self) -> "Ciphertext":
        out = ctypes.c_void_p()
        check(lib.ckks_ct_copy(self.context.handle, self.handle, ctypes.byref(out)))
        return Ciphertext(self.context, out.value)

    def download(self) -> np.ndarray:
        info = self._info()
        per = int(info.limbs) + (self.context.alpha if info.is_ext else 0)
        if info.polys == 0:
            out = np.zeros(int(info.limbs), dtype=np.uint64)
        else:
            out = np.zeros((int(info.polys), per, self.context.N), dtype=np.uint64)
        check(lib.ckks_ct_download(self.context.handle, self.handle,
                                   out.ctypes.data_as(_native.U64P)))
        return out

    def release(self) -> None:
        if self._h and not self._pinned:
            lib.ckks_ct_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self._pinned = False
            self.release()
        except Exception:
            pass


Plaintext = Ciphertext


def _wrap(context: NativeContext, handle: ctypes.c_void_p) -> Ciphertext:
    return Ciphertext(context, handle.value)


def _ctx(ct: Ciphertext, context) -> NativeContext:
    if context is not None and context is not ct.context:
        raise ValueError("ciphertext belongs to a different context")
    return ct.context


def upload(context: NativeContext, data: np.ndarray, *, slots: int, scale: float,
           scale_degree: int = 1, is_ext: bool = False) -> Ciphertext:
    """Raw limbs [polys, limbs(+alpha), N] to a device object (tests, batching)."""
    data = np.ascontiguousarray(data, dtype=np.uint64)
    if data.ndim != 3 or data.shape[2] != context.N:
        raise ValueError(f"raw limbs must have shape [polys, limbs, {context.N}], got {data.shape}")
    polys, per = int(data.shape[0]), int(data.shape[1])
    limbs = per - (context.alpha if is_ext else 0)
    out = ctypes.c_void_p()
    check(lib.ckks_ct_upload(context.handle, data.ctypes.data_as(_native.U64P), polys, limbs,
                             int(is_ext), int(slots), float(scale), int(scale_degree),
                             ctypes.byref(out)))
    return _wrap(context, out)


# ---------------------------------------------------------------------------
# client (secret-key side)
# ---------------------------------------------------------------------------


class Client:
    """Encryption and decryption with the context's secret key
    (reference backend.py:221-229, 305-313; application/session.py:71-77)."""

    def __init__(self, context: NativeContext):
        self.context = context

    def encrypt(self, values, device: str | None = None, slots: int | None = None,
                cur_limbs: int | None = None, scaling_factor: float | None = None,
                enc_id: int | None = None) -> Ciphertext:
        ctx = self.context
        slots = ctx.max_slots if slots is None else int(slots)
        limbs = ctx.L if cur_limbs is None else int(cur_limbs)
        scale = ctx.scale_at(limbs) if scaling_factor is None else float(scaling_factor)
        z = np.asarray(values).reshape(-1)
        if z.size > slots:
            raise ValueError(f"{z.size} values do not fit {slots} slots")
        buf = np.zeros(slots, dtype=np.complex128)
        buf[: z.size] = z
        re = np.ascontiguousarray(buf.real)
        im = np.ascontiguousarray(buf.imag)
        eid = ctx.next_encryption_id() if enc_id is None else int(enc_id)
        out = ctypes.c_void_p()
        check(lib.ckks_encrypt(ctx.handle, re.ctypes.data_as(_native.DP),
                               im.ctypes.data_as(_native.DP), slots, limbs, scale,
                               eid & 0xFFFFFFFF, ctypes.byref(out)))
        return _wrap(ctx, out)

    def decrypt_complex(self, ct: Ciphertext) -> np.ndarray:
        slots = ct.slots
        re = np.zeros(slots)
        im = np.zeros(slots)
        check(lib.ckks_decrypt(self.context.handle, ct.handle, re.ctypes.data_as(_native.DP),
                               im.ctypes.data_as(_native.DP)))
        return re + 1j * im

    def decrypt(self, ct: Ciphertext) -> np.ndarray:
        """Real part of the decrypted slots (reference backend.py:305-313)."""
        return np.real(self.decrypt_complex(ct)).copy()


def generate_client_context(spec: CKKSContextSpec, device: str = "cuda"):
    """Create the context, the secret key, the relinearisation key and the
    rotation keys of ``spec.rotations`` (reference application/session.py:31-45)."""
    ctx = NativeContext(spec, device=device)
    if spec.relin_key:
        ctx.generate_relin_key()
    ctx.generate_rotation_keys(int(r) for r in spec.rotations if int(r))
    return Client(ctx), ctx


# ---------------------------------------------------------------------------
# encoding
# ---------------------------------------------------------------------------


def encode_rows(context: NativeContext, rows, *, limbs: int, scale: float, slots: int,
                is_ext: bool = False) -> list[Ciphertext]:
    z = np.asarray(rows)
    if z.ndim == 1:
        z = z[None, :]
    if z.shape[1] != slots:
        raise ValueError(f"row length {z.shape[1]} != slots {slots}")
    z = z.astype(np.complex128)
    re = np.ascontiguousarray(z.real)
    im = np.ascontiguousarray(z.imag)
    n = z.shape[0]
    handles = (ctypes.c_void_p * n)()
    check(lib.ckks_encode_rows(context.handle, re.ctypes.data_as(_native.DP),
                               im.ctypes.data_as(_native.DP), n, int(slots), int(limbs),
                               float(scale), int(is_ext), handles))
    return [Ciphertext(context, handles[i]) for i in range(n)]


# Plaintexts of constant rows (masks, rotation tables, row selectors) that an
# operator encodes on every call: kept per context, keyed by the rows'
# content (xxh3-128 of their bytes), shape, limbs, scale and basis, least
# recently used dropped beyond a byte cap.  The cached objects are pinned:
# release() leaves them alone until the cache drops them.
PLAINTEXT_CACHE_BYTES = 8 << 30


def _rows_digest(z: np.ndarray) -> str:
    try:
        import xxhash

        return xxhash.xxh3_128_hexdigest(z.tobytes())
    except ImportError:  # pragma: no cover - xxhash ships with the image
        import hashlib

        return hashlib.blake2b(z.tobytes(), digest_size=16).hexdigest()


def encode_rows_cached(context: NativeContext, rows, *, limbs: int, scale: float, slots: int,
                       is_ext: bool = False) -> list[Ciphertext]:
    """encode_rows through the context's plaintext cache; the returned
    plaintexts may be released by the caller (a no-op while cached) and must
    not be modified."""
    z = np.ascontiguousarray(np.asarray(rows))
    if z.ndim == 1:
        z = z[None, :]
    key = (_rows_digest(z), z.shape, str(z.dtype), int(limbs), float(scale), int(slots),
           bool(is_ext))
    cache = context.__dict__.setdefault("_pt_cache", {})
    hit = cache.pop(key, None)
    if hit is None:
        pts = encode_rows(context, z, limbs=limbs, scale=scale, slots=slots, is_ext=is_ext)
        width = int(limbs) + (context.alpha if is_ext else 0)
        hit = (pts, 8 * context.N * width * len(pts))
        for p in pts:
            p._pinned = True
        used = context.__dict__.get("_pt_cache_bytes", 0) + hit[1]
        while cache and used > PLAINTEXT_CACHE_BYTES:
            old_key = next(iter(cache))
            old, nbytes = cache.pop(old_key)
            for p in old:
                p._pinned = False
                p.release()
            used -= nbytes
        context.__dict__["_pt_cache_bytes"] = used
    cache[key] = hit  # most recently used last
    return list(hit[0])


def clear_plaintext_cache(context: NativeContext) -> None:
    cache = context.__dict__.pop("_pt_cache", {})
    context.__dict__["_pt_cache_bytes"] = 0
    for pts, _ in cache.values():
        for p in pts:
            p._pinned = False
            p.release()


def decode(pt: Ciphertext) -> np.ndarray:
    slots = pt.slots
    re = np.zeros(slots)
    im = np.zeros(slots)
    check(lib.ckks_decode(pt.context.handle, pt.handle, re.ctypes.data_as(_native.DP),
                          im.ctypes.data_as(_native.DP)))
    return re + 1j * im


class PackedRaw:
    """Already packed ``[rows, slots]`` (or ``[slots]``) values
    (reference backend.py:274-284)."""

    def __init__(self, tensor):
        self.tensor = tensor

    def values(self, slots: int, context):
        from .packing import DiagonalChunk

        if isinstance(self.tensor, DiagonalChunk):
            return self.tensor
        return np.asarray(self.tensor)


class UnpackedRaw:
    """Raw source plus a packer ``packer(source, slots, context) -> [rows, slots]``
    (reference operators/linear/weight.py:309-366)."""

    def __init__(self, source, packer):
        self.source = source
        self.packer = packer

    def values(self, slots: int, context):
        from .packing import DiagonalChunk

        out = self.packer(self.source, slots, context)
        return out if isinstance(out, DiagonalChunk) else np.asarray(out)


class ConstantBundle:
    """Named constant vectors encoded on demand at a requested state
    (reference backend.py:260-297, operators/primitives.py:83-97).

    ``plaintext`` returns one plaintext for a 1-D vector and a list of
    plaintexts (one per row) for a 2-D ``[rows, slots]`` block.
    Cache modes: ``none`` keeps nothing, ``plain``/``both`` keep encoded
    plaintexts per (name, limbs, scale, basis, slots), ``middle`` keeps the
    packed host values."""

    def __init__(self, vectors: dict, cache_mode: str = "none"):
        if cache_mode not in {"none", "middle", "plain", "both"}:
            raise ValueError(f"unknown cache_mode {cache_mode!r}")
        self.vectors = dict(vectors)
        self.cache_mode = cache_mode
        self._plain: dict = {}
        self._middle: dict = {}

    def set_cache_mode(self, mode: str, clear: bool = False) -> None:
        if mode not in {"none", "middle", "plain", "both"}:
            raise ValueError(f"unknown cache_mode {mode!r}")
        if clear:
            self.clear_cache()
        self.cache_mode = mode

    def _values(self, name: str, slots: int, context) -> np.ndarray:
        if name in self._middle:
            return self._middle[name]
        values = self.vectors[name].values(slots, context)
        if self.cache_mode in ("middle", "both"):
            self._middle[name] = values
        return values

    def plaintext(self, name: str, *, state: CipherState, slots: int, context: NativeContext,
                  is_ext: bool = False, cache: bool = False):
        limbs = int(state.cur_limbs)
        scale = float(state.scaling_factor) if state.scaling_factor else context.scale_at(limbs)
        key = (str(name), limbs, scale, bool(is_ext), int(slots))
        if key in self._plain:
            return self._plain[key]
        values = self._values(str(name), int(slots), context)
        from .packing import DiagonalChunk

        if isinstance(values, DiagonalChunk):
            # device-resident weight: gather and encode in one device pass
            result = values.encode(context, limbs=limbs, scale=scale, is_ext=bool(is_ext))
        else:
            arr = np.asarray(values)
            pts = encode_rows(context, arr, limbs=limbs, scale=scale, slots=int(slots),
                              is_ext=bool(is_ext))
            result = pts[0] if arr.ndim == 1 else pts
        if cache or self.cache_mode in ("plain", "both"):
            self._plain[key] = result
        return result

    def cache_info(self) -> dict[str, int]:
        total = 0
        entries = 0
        for value in self._plain.values():
            items = value if isinstance(value, list) else [value]
            for pt in items:
                info = pt._info()
                total += 8 * pt.context.N * (int(info.limbs) +
                                             (pt.context.alpha if info.is_ext else 0))
                entries += 1
        total += sum(int(v.nbytes) for v in self._middle.values() if isinstance(v, np.ndarray))
        return {"entries": entries, "total_bytes": total}

    def clear_cache(self) -> None:
        for value in self._plain.values():
            for pt in (value if isinstance(value, list) else [value]):
                pt.release()
        self._plain.clear()
        self._middle.clear()


def encode_scalar(value: float, cur_limbs: int, scale_degree: int = 1,
                  scaling_factor: float | None = None, mode: str | None = None,
                  context: NativeContext | None = None) -> Ciphertext:
    """Per-limb constant round(value * scale); ``mode="integer"`` encodes the
    value itself (reference operators/nonlinear/polynomial.py:40-67,
    operators/nonlinear/bootstrap.py:330-349)."""
    if context is None:
        context = current_context()
    if mode == "integer":
        scale = 1.0
    else:
        scale = float(scaling_factor) if scaling_factor else context.scale_at(int(cur_limbs))
    out = ctypes.c_void_p()
    check(lib.ckks_encode_scalar(context.handle, float(value), int(cur_limbs), scale,
                                 ctypes.byref(out)))
    return _wrap(context, out)


# ---------------------------------------------------------------------------
# arithmetic
# ---------------------------------------------------------------------------


def _binary(fn, a: Ciphertext, b: Ciphertext, context) -> Ciphertext:
    ctx = _ctx(a, context)
    out = ctypes.c_void_p()
    check(fn(ctx.handle, a.handle, b.handle, ctypes.byref(out)))
    return _wrap(ctx, out)


def homo_add(a, b, context=None):
    return _binary(lib.ckks_add, a, b, context)


def homo_sub(a, b, context=None):
    return _binary(lib.ckks_sub, a, b, context)


def _binary_many(op: int, a: Sequence[Ciphertext], b: Sequence[Ciphertext], context) -> list:
    a, b = list(a), list(b)
    if len(a) != len(b):
        raise ValueError("operand lists differ in length")
    if not a:
        return []
    ctx = _ctx(a[0], context)
    outs = (ctypes.c_void_p * len(a))()
    check(lib.ckks_add_many(ctx.handle, ptr_array([x.handle for x in a]),
                            ptr_array([y.handle for y in b]), len(a), int(op), outs))
    return [Ciphertext(ctx, outs[i]) for i in range(len(a))]


def homo_add_many(a: Sequence[Ciphertext], b: Sequence[Ciphertext], context=None) -> list:
    """[homo_add(x, y) for x, y in zip(a, b)] for pairs of one shape in
    batched launches."""
    return _binary_many(0, a, b, context)


def homo_sub_many(a: Sequence[Ciphertext], b: Sequence[Ciphertext], context=None) -> list:
    return _binary_many(1, a, b, context)


def homo_add_pt(a, pt, context=None):
    return _binary(lib.ckks_add_pt, a, pt, context)


def homo_mul_pt(a, pt, context=None):
    return _binary(lib.ckks_mul_pt, a, pt, context)


def homo_mul_i(a, context=None, negative: bool = False):
    """Multiply slots by +i (or -i): the monomial X^(N/2), level-free
    (reference operators/linear/complex.py:21, attention/codec.py:44)."""
    ctx = _ctx(a, context)
    out = ctypes.c_void_p()
    check(lib.ckks_mul_i(ctx.handle, a.handle, int(bool(negative)), ctypes.byref(out)))
    return _wrap(ctx, out)


def homo_add_scalar(a, scalar, context=None):
    return _binary(lib.ckks_add_scalar, a, scalar, context)


def homo_mul_scalar(a, scalar, context=None):
    return _binary(lib.ckks_mul_scalar, a, scalar, context)


def homo_mul_scalar_rescale(a, scalar, context=None):
    prod = homo_mul_scalar(a, scalar, context)
    try:
        if float(scalar.state.scaling_factor or 1.0) == 1.0:
            return prod.deep_copy()
        return rescale(prod, context)
    finally:
        prod.release()


def homo_mul_no_relin(a, b, context=None):
    return _binary(lib.ckks_mul_no_relin, a, b, context)


def homo_relinearize(a, context=None):
    ctx = _ctx(a, context)
    out = ctypes.c_void_p()
    check(lib.ckks_relinearize(ctx.handle, a.handle, ctypes.byref(out)))
    return _wrap(ctx, out)


def homo_mul_relin(a, b, context=None):
    return _binary(lib.ckks_mul_relin, a, b, context)


def rescale(a, context=None):
    ctx = _ctx(a, context)
    out = ctypes.c_void_p()
    check(lib.ckks_rescale(ctx.handle, a.handle, ctypes.byref(out)))
    return _wrap(ctx, out)


# relative scale differences below this are one scale (float rounding of the
# exact bookkeeping); above it align_to adjusts the scale when it has a level
_SAME_SCALE = 2.0 ** -32
# fixed-scale tolerance of limb-wise sums (the library's check_scales)
_FIXED_SCALE_TOL = 1.0 / 1024.0


def align_to(a, target_state: CipherState, context=None):
    """Bring ``a`` to ``target_state``: its limb count and, when the state
    names one, its scaling factor (reference operators/primitives.py:140-150,
    the Meta-BTS alignments of operators/nonlinear/bootstrap.py:386-424).
    Returns ``a`` itself when nothing changes.

    A limb drop keeps the scale.  A different target scale ``w`` is reached
    exactly up to integer rounding: ``a`` is cut to ``t + D`` limbs, multiplied
    by the integer ``round(w p / s)`` with ``p`` the product of the D primes
    above the target level (D the fewest that make the integer at least
    2^30), and rescaled by those primes; the result's scale is ``w`` to
    within 2^-31 relative, and only levels that the drop would shed are used.
    Without such a level, a scale within the fixed-scale tolerance (2^-10
    relative) is kept and a larger difference raises ``ValueError``."""
    ctx = _ctx(a, context)
    target = int(target_state.cur_limbs)
    info = a._info()
    cur, scale = int(info.limbs), float(info.scale)
    if target > cur:
        raise ValueError(f"cannot align {cur} limbs up to {target} limbs")
    if target < 1:
        raise ValueError("cannot align below one limb")
    want = target_state.scaling_factor
    if want is not None and float(want) <= 0.0:
        raise ValueError("the target scaling factor must be positive")
    if want is None or abs(float(want) - scale) <= scale * _SAME_SCALE:
        return a if target == cur else _drop_limbs(a, target, ctx)
    want = float(want)
    primes = [int(q) for q in ctx.primes()[: ctx.L]]
    prod, D = 1.0, 0
    while target + D < cur and want * prod / scale < 2.0 ** 30:
        prod *= float(primes[target + D])
        D += 1
    k = want * prod / scale
    if D == 0 or k < 2.0 ** 30:
        if abs(want - scale) <= scale * _FIXED_SCALE_TOL:
            return a if target == cur else _drop_limbs(a, target, ctx)
        raise ValueError(
            f"align_to needs a spare level to change the scale by {want / scale:.6g} "
            f"({cur} limbs -> {target})")
    if k >= 2.0 ** 62:
        raise ValueError(f"scale ratio {want / scale:.6g} is too large to adjust in one step")
    work = a if target + D == cur else _drop_limbs(a, target + D, ctx)
    try:
        factor = encode_scalar(1.0, target + D, scaling_factor=float(np.rint(k)), context=ctx)
        try:
            prod_ct = homo_mul_scalar(work, factor, ctx)
        finally:
            factor.release()
        try:
            return rescale_many([prod_ct], ctx, primes=D)[0]
        finally:
            prod_ct.release()
    finally:
        if work is not a:
            work.release()


def _drop_limbs(a, target: int, ctx) -> "Ciphertext":
    out = ctypes.c_void_p()
    check(lib.ckks_drop_limbs(ctx.handle, a.handle, int(target), ctypes.byref(out)))
    return _wrap(ctx, out)


def homo_mul_relin_rescale_postop(left, right, context=None, *, apply_double: bool = False,
                                  sub=None, scalar=None):
    """rescale(relin(l r)), then x2 when ``apply_double``, then ``- sub`` and
    ``+ scalar`` at the output level, as one key switch whose ModDown applies
    the postop (reference operators/nonlinear/polynomial.py:115-203).  The
    operands meet at the lower of their levels first."""
    ctx = _ctx(left, context)
    limbs = min(left.state.cur_limbs, right.state.cur_limbs)
    l2 = align_to(left, left.state.replace(cur_limbs=limbs, scaling_factor=None), ctx)
    r2 = align_to(right, right.state.replace(cur_limbs=limbs, scaling_factor=None), ctx)
    try:
        return homo_mul_relin_rescale_postop_many(
            [l2], [r2], ctx, apply_double=apply_double,
            sub=None if sub is None else [sub], scalar=scalar)[0]
    finally:
        for x, y in ((l2, left), (r2, right)):
            if x is not y:
                x.release()


def homo_mul_relin_rescale_postop_many(left: Sequence[Ciphertext], right: Sequence[Ciphertext],
                                       context=None, *, apply_double: bool = False,
                                       sub: Sequence[Ciphertext] | None = None,
                                       scalar=None) -> list:
    """``homo_mul_relin_rescale_postop`` of n pairs at one level in batched
    launches; ``sub`` holds one ciphertext per pair (or None), ``scalar`` is
    shared by all pairs."""
    left, right = list(left), list(right)
    if len(left) != len(right) or (sub is not None and len(list(sub)) != len(left)):
        raise ValueError("operand lists differ in length")
    if not left:
        return []
    ctx = _ctx(left[0], context)
    outs = (ctypes.c_void_p * len(left))()
    subs = None if sub is None else ptr_array([c.handle for c in sub])
    check(lib.ckks_mul_relin_rescale_postop_many(
        ctx.handle, ptr_array([c.handle for c in left]), ptr_array([c.handle for c in right]),
        len(left), int(bool(apply_double)), subs, None if scalar is None else scalar.handle, outs))
    return [Ciphertext(ctx, outs[i]) for i in range(len(left))]


def homo_rotate(a, rotation: int, context=None):
    """Left rotation by ``rotation`` slots (``np.roll(m, -k)``); ``M - 1``
    conjugates (reference operators/linear/operator.py:333,
    operators/linear/complex.py:47-51)."""
    ctx = _ctx(a, context)
    out = ctypes.c_void_p()
    check(lib.ckks_rotate(ctx.handle, a.handle, int(rotation), ctypes.byref(out)))
    return _wrap(ctx, out)


def mod_raise(a, target_limbs: int, context=None):
    """One-limb ciphertext lifted to ``target_limbs`` limbs (bootstrap ModRaise)."""
    ctx = _ctx(a, context)
    out = ctypes.c_void_p()
    check(lib.ckks_mod_raise(ctx.handle, a.handle, int(target_limbs), ctypes.byref(out)))
    return _wrap(ctx, out)


def linear_combination(terms, weights, constant: float, limbs: int, scale: float,
                       scale_degree: int = 2, context=None) -> list:
    """``out_i = sum_t rint(weights[t]) terms[t][i] + rint(constant)`` for every
    ciphertext i in one launch, on the first ``limbs`` limbs of each term
    (weights already carry their encoding scales); ``terms`` is [T][n]."""
    terms = [list(t) for t in terms]
    T, n = len(terms), len(terms[0])
    if any(len(t) != n for t in terms):
        raise ValueError("every term needs one ciphertext per output")
    ctx = _ctx(terms[0][0], context)
    w = np.ascontiguousarray(np.asarray(weights, dtype=np.float64))
    outs = (ctypes.c_void_p * n)()
    check(lib.ckks_linear_combination(ctx.handle, ptr_array([x.handle for t in terms for x in t]),
                                      T, n, w.ctypes.data_as(_native.DP), float(constant),
                                      int(limbs), float(scale), int(scale_degree), outs))
    return [Ciphertext(ctx, outs[i]) for i in range(n)]


def rescale_many(cts: Sequence[Ciphertext], context=None, primes: int = 1) -> list:
    """fhe.rescale of several ciphertexts of one shape in batched launches;
    ``primes`` > 1 divides by that many last primes in one pass, with the
    words of as many rescales in a row."""
    if not cts:
        return []
    ctx = _ctx(cts[0], context)
    cts, left = list(cts), int(primes)
    if left < 1:
        raise ValueError("rescale divides by at least one prime")
    while left:
        step = min(left, 4)  # primes per launch sequence
        outs = (ctypes.c_void_p * len(cts))()
        check(lib.ckks_rescale_many_by(ctx.handle, ptr_array([c.handle for c in cts]), len(cts),
                                       step, outs))
        cts = [Ciphertext(ctx, outs[i]) for i in range(len(cts))]
        left -= step
    return cts


def hoisted_mac_sum_ext_many(cts: Sequence[Ciphertext], baby_offsets, plaintexts,
                             giant_offset: int, giant_count: int, context=None,
                             strategy: str = "ext_normal") -> list:
    """The extended-basis hoisted_mac_sum of several ciphertexts at one level
    with shared (extended) plaintexts; keys and plaintexts are read once per
    batch of up to 64.  ``strategy`` "ext_double_hoist" rotates the giant
    groups in Q u P (see hoisted_mac_sum)."""
    if strategy not in ("ext_normal", "ext_double_hoist"):
        raise ValueError(f"unknown extended strategy {strategy!r}")
    if not cts:
        return []
    ctx = _ctx(cts[0], context)
    offs = np.asarray([int(o) for o in baby_offsets], dtype=np.int64)
    B = len(offs)
    pts = list(plaintexts)[: B * int(giant_count)]
    if len(pts) < B * int(giant_count):
        raise ValueError(f"need {B * int(giant_count)} plaintexts, got {len(pts)}")
    results: list = []
    for i0 in range(0, len(cts), 64):
        chunk = cts[i0: i0 + 64]
        outs = (ctypes.c_void_p * len(chunk))()
        fn = (lib.ckks_hoisted_mac_sum_double_many if strategy == "ext_double_hoist"
              else lib.ckks_hoisted_mac_sum_ext_many)
        check(fn(ctx.handle, ptr_array([c.handle for c in chunk]), len(chunk),
                 offs.ctypes.data_as(_native.I64P), B, ptr_array([p.handle for p in pts]),
                 int(giant_offset), int(giant_count), outs))
        results.extend(Ciphertext(ctx, outs[i]) for i in range(len(chunk)))
    return results


def homo_rotate_many(cts: Sequence[Ciphertext], rotation: int, context=None) -> list:
    """One rotation of many same-level ciphertexts; the key is streamed once."""
    cts = list(cts)
    if not cts:
        return []
    ctx = _ctx(cts[0], context)
    ins = ptr_array([c.handle for c in cts])
    outs = (ctypes.c_void_p * len(cts))()
    check(lib.ckks_rotate_many(ctx.handle, ins, len(cts), int(rotation), outs))
    return [Ciphertext(ctx, outs[i]) for i in range(len(cts))]


def homo_mul_relin_rescale_many(left: Sequence[Ciphertext], right: Sequence[Ciphertext],
                                context=None, primes: int = 1) -> list:
    """Products, relinearised and rescaled by ``primes`` (1..4) last primes,
    batched: one key switch per product whose ModDown also does the rescales
    (the same words as homo_mul_relin and ``primes`` rescales)."""
    left, right = list(left), list(right)
    if len(left) != len(right):
        raise ValueError("operand lists differ in length")
    if not left:
        return []
    ctx = _ctx(left[0], context)
    if int(primes) < 1:
        raise ValueError("rescale divides by at least one prime")
    first = min(int(primes), 4)  # primes one merged ModDown takes
    outs = (ctypes.c_void_p * len(left))()
    check(lib.ckks_mul_relin_rescale_many_by(ctx.handle, ptr_array([c.handle for c in left]),
                                             ptr_array([c.handle for c in right]), len(left),
                                             first, outs))
    res = [Ciphertext(ctx, outs[i]) for i in range(len(left))]
    return rescale_many(res, ctx, primes=int(primes) - first) if int(primes) > first else res


def _hoisted(ct: Ciphertext, offsets: Sequence[int], ctx: NativeContext) -> list:
    offs = np.asarray([int(o) for o in offsets], dtype=np.int64)
    outs = (ctypes.c_void_p * len(offs))()
    check(lib.ckks_hoisted_rotate(ctx.handle, ct.handle, offs.ctypes.data_as(_native.I64P),
                                  len(offs), outs))
    return [Ciphertext(ctx, outs[i]) for i in range(len(offs))]


def prepare_hoisted_baby_rotations(ct, baby_offsets, context=None, strategy: str = "normal",
                                   baby_anchor_step: int = -1):
    """Rotations of ``ct`` by every baby offset from one shared ModUp
    (reference operators/linear/operator.py:100-117).  With an anchor step
    A < B the babies come in blocks of A: block k starts from the anchor
    rot(ct, offsets[kA]) reached by chaining one anchor key, and covers its
    block with one hoisted call."""
    ctx = _ctx(ct, context)
    offsets = [int(o) for o in baby_offsets]
    if strategy not in {"normal", "ext_normal", "ext_double_hoist"}:
        raise ValueError(f"unknown strategy {strategy!r}")
    B = len(offsets)
    anchor = int(baby_anchor_step)
    if anchor < 2 or anchor >= B:
        return tuple(_hoisted(ct, offsets, ctx))
    result: list = []
    base = ct
    for start in range(0, B, anchor):
        block = offsets[start: start + anchor]
        if start:
            nxt = homo_rotate(base, offsets[start] - offsets[start - anchor], ctx)
            if base is not ct:
                base.release()
            base = nxt
        result.extend(_hoisted(base, [o - offsets[start] for o in block], ctx))
    if base is not ct:
        base.release()
    return tuple(result)


def prepare_hoisted_baby_rotations_many(cts: Sequence[Ciphertext], baby_offsets, context=None,
                                        baby_anchor_step: int = -1) -> list:
    """prepare_hoisted_baby_rotations for several same-level ciphertexts: one
    batched ModUp, each baby key read once for the batch; returns one tuple of
    babies per ciphertext (same words as the single-ciphertext form)."""
    cts = list(cts)
    if not cts:
        return []
    ctx = _ctx(cts[0], context)
    offsets = [int(o) for o in baby_offsets]
    B = len(offsets)

    def hoisted(bases, offs):
        arr = np.asarray(offs, dtype=np.int64)
        outs = (ctypes.c_void_p * (len(bases) * len(offs)))()
        check(lib.ckks_hoisted_rotate_many(ctx.handle, ptr_array([c.handle for c in bases]),
                                           len(bases), arr.ctypes.data_as(_native.I64P),
                                           len(offs), outs))
        return [[Ciphertext(ctx, outs[i * len(offs) + r]) for r in range(len(offs))]
                for i in range(len(bases))]

    anchor = int(baby_anchor_step)
    if anchor < 2 or anchor >= B:
        return [tuple(x) for x in hoisted(cts, offsets)]
    result: list = [[] for _ in cts]
    bases = cts
    for start in range(0, B, anchor):
        block = offsets[start: start + anchor]
        if start:
            nxt = homo_rotate_many(bases, offsets[start] - offsets[start - anchor], ctx)
            if bases is not cts:
                for b in bases:
                    b.release()
            bases = nxt
        for i, part in enumerate(hoisted(bases, [o - offsets[start] for o in block])):
            result[i].extend(part)
    if bases is not cts:
        for b in bases:
            b.release()
    return [tuple(r) for r in result]


def hoisted_mac_sum(ct, baby_offsets, plaintexts, giant_offset: int, giant_count: int,
                    context=None, strategy: str = "normal", baby_anchor_step: int = -1,
                    baby_rotations=None):
    """BSGS diagonal MAC
    ``sum_{g<G} rot_{g giant}( sum_{b<B} pt[g B + b] * rot_{baby_b}(ct) )``
    with a Horner chain over one giant key; unrescaled
    (reference operators/linear/operator.py:320-330, operators/transform.py:108).
    Strategies "ext_normal" and "ext_double_hoist" with extended plaintexts
    keep the babies in the Q u P basis: "ext_normal" takes one ModDown per
    giant group before the Horner chain, "ext_double_hoist" rotates every
    giant group in Q u P with its own key (g * giant_offset) and takes one
    ModDown of the sum (reference operators/linear/config.py:296-305).  With
    Q-basis plaintexts (or precomputed babies or an anchor step) both run
    the normal schedule."""
    ctx = _ctx(ct, context)
    pts = plaintexts if isinstance(plaintexts, (list, tuple)) else [plaintexts]
    B = len(list(baby_offsets))
    if len(pts) < B * int(giant_count):
        raise ValueError(f"need {B * int(giant_count)} plaintexts, got {len(pts)}")
    used = pts[: B * int(giant_count)]
    if (strategy in ("ext_normal", "ext_double_hoist") and baby_rotations is None
            and int(baby_anchor_step) < 2 and all(p.is_ext for p in used)):
        # babies kept in Q u P: one ModDown per giant group, or (double
        # hoisting) giant groups rotated in Q u P and one ModDown of the sum
        offs = np.asarray([int(o) for o in baby_offsets], dtype=np.int64)
        out = ctypes.c_void_p()
        fn = (lib.ckks_hoisted_mac_sum_double if strategy == "ext_double_hoist"
              else lib.ckks_hoisted_mac_sum_ext)
        check(fn(ctx.handle, ct.handle, offs.ctypes.data_as(_native.I64P), B,
                 ptr_array([p.handle for p in used]), int(giant_offset), int(giant_count),
                 ctypes.byref(out)))
        return _wrap(ctx, out)
    babies = baby_rotations
    owned = False
    if babies is None:
        babies = prepare_hoisted_baby_rotations(ct, baby_offsets, ctx, strategy=strategy,
                                                baby_anchor_step=baby_anchor_step)
        owned = True
    try:
        out = ctypes.c_void_p()
        check(lib.ckks_hoisted_mac_sum(ctx.handle, ptr_array([b.handle for b in babies]), B,
                                       ptr_array([p.handle for p in pts[: B * int(giant_count)]]),
                                       int(giant_offset), int(giant_count), ctypes.byref(out)))
        return _wrap(ctx, out)
    finally:
        if owned:
            for b in babies:
                b.release()


def hoisted_mac_sum_many(baby_rotations: Sequence[Sequence[Ciphertext]], plaintexts,
                         giant_offset: int, giant_count: int, context=None) -> list:
    """hoisted_mac_sum with precomputed babies for several ciphertexts that
    share the plaintexts (every input of one linear chunk): ``baby_rotations[i]``
    holds the B babies of ciphertext i.  The plaintexts are read once for the
    batch and the babies once per pass of up to 8 giant groups; results are
    unrescaled and the same words as one hoisted_mac_sum per ciphertext."""
    sets = [list(b) for b in baby_rotations]
    if not sets:
        return []
    B = len(sets[0])
    if B == 0 or any(len(b) != B for b in sets):
        raise ValueError("every ciphertext needs the same number of babies")
    ctx = _ctx(sets[0][0], context)
    pts = plaintexts if isinstance(plaintexts, (list, tuple)) else [plaintexts]
    if len(pts) < B * int(giant_count):
        raise ValueError(f"need {B * int(giant_count)} plaintexts, got {len(pts)}")
    used = ptr_array([p.handle for p in pts[: B * int(giant_count)]])
    per = max(1, 8192 // B - min(8, int(giant_count)))  # the kernel's pointer-table bound
    results: list = []
    for i0 in range(0, len(sets), per):
        part = sets[i0: i0 + per]
        outs = (ctypes.c_void_p * len(part))()
        check(lib.ckks_hoisted_mac_sum_many(ctx.handle, ptr_array([b.handle for bs in part
                                                                   for b in bs]),
                                            len(part), B, used, int(giant_offset),
                                            int(giant_count), outs))
        results.extend(Ciphertext(ctx, outs[i]) for i in range(len(part)))
    return results


# ---------------------------------------------------------------------------
# batches (reference operators/attention/kernel_helpers.py:83-85,
# attention/input.py:792-826)
# ---------------------------------------------------------------------------


class CipherBatch:
    """An ordered group of same-level ciphertexts."""

    def __init__(self, ciphers: Sequence[Ciphertext]):
        self.cv = list(ciphers)

    @property
    def batch_size(self) -> int:
        return len(self.cv)

    def cipher_like(self, cv, batch_size: int | None = None, slots: int | None = None):
        return CipherBatch(list(cv)[: batch_size] if batch_size else list(cv))

    def __iter__(self):
        return iter(self.cv)

    def __len__(self):
        return len(self.cv)

    def release(self) -> None:
        for c in self.cv:
            c.release()


def pack_cipher_batch(ciphers: Iterable[Ciphertext]) -> CipherBatch:
    return CipherBatch([c.deep_copy() for c in ciphers])


def unpack_cipher_batch(batch: CipherBatch) -> tuple:
    return tuple(batch.cv)


def _hoisted_ext(ct: Ciphertext, offsets: Sequence[int], ctx: NativeContext) -> list:
    offs = np.asarray([int(o) for o in offsets], dtype=np.int64)
    outs = (ctypes.c_void_p * len(offs))()
    check(lib.ckks_hoisted_rotate_ext(ctx.handle, ct.handle,
                                      offs.ctypes.data_as(_native.I64P), len(offs), outs))
    return [Ciphertext(ctx, outs[i]) for i in range(len(offs))]


def fast_rotate(ct, offsets, context=None, output_ext: bool = False) -> CipherBatch:
    """Hoisted rotations of one ciphertext into a batch; with ``output_ext``
    the outputs stay in the Q u P basis before their ModDown (P rot_k(ct)),
    to be multiplied by extended plaintexts, summed and brought back with one
    ``moddown_from_ext`` (reference operators/attention/input.py:792-826)."""
    ctx = _ctx(ct, context)
    offs = [int(o) for o in offsets]
    if output_ext:
        return CipherBatch(_hoisted_ext(ct, offs, ctx))
    return CipherBatch(_hoisted(ct, offs, ctx))


def moddown_from_ext(ct, context=None):
    """Q-basis copy of ``ct``: ModDown (division by P) of an extended
    ciphertext, a plain copy otherwise."""
    ctx = _ctx(ct, context)
    if not ct.is_ext:
        return ct.deep_copy()
    out = ctypes.c_void_p()
    check(lib.ckks_moddown_ext(ctx.handle, ct.handle, ctypes.byref(out)))
    return _wrap(ctx, out)


def _batch_items(batch) -> list:
    if isinstance(batch, CipherBatch):
        return list(batch.cv)
    if hasattr(batch, "cv") and not isinstance(batch, Ciphertext):
        return list(batch.cv)
    return list(batch)


def grouped_pairwise_mac(batch, plaintexts, groups, context=None):
    """``sum_i batch[i] * plaintexts[i]`` per group, unrescaled (reference
    operators/attention/input.py:814-826, 1274-1286, 1322-1334).  ``groups``
    is either a group count G (the batch split into G consecutive groups of
    equal size; the reference passes 1 and gets one ciphertext back, a list
    for G > 1) or a sequence of index groups (a list back).  One launch per
    group reads each ciphertext and plaintext word once (ckks_grouped_mac);
    extended (Q u P) terms take extended plaintexts and stay extended, for
    ``moddown_from_ext``."""
    cts = _batch_items(batch)
    pts = _batch_items(plaintexts)
    if not cts:
        return []
    ctx = _ctx(cts[0], context)
    if isinstance(groups, (int, np.integer)):
        G = int(groups)
        if G < 1 or len(cts) % G:
            raise ValueError(f"{len(cts)} terms do not split into {G} equal groups.")
        size = len(cts) // G
        index_groups = [list(range(g * size, (g + 1) * size)) for g in range(G)]
        single = G == 1
    else:
        index_groups = [[int(i) for i in grp] for grp in groups]
        single = False
    if not index_groups:
        return []
    order = [i for grp in index_groups for i in grp]
    if any(i < 0 or i >= len(cts) or i >= len(pts) for i in order):
        raise ValueError("grouped_pairwise_mac: term index out of range.")
    sizes = (ctypes.c_int * len(index_groups))(*[len(grp) for grp in index_groups])
    outs = (ctypes.c_void_p * len(index_groups))()
    check(lib.ckks_grouped_mac(ctx.handle, _native.ptr_array([cts[i].handle for i in order]),
                               _native.ptr_array([pts[i].handle for i in order]), sizes,
                               len(index_groups), outs))
    results = [Ciphertext(ctx, outs[g]) for g in range(len(index_groups))]
    return results[0] if single else results


__all__ = [name for name in dir() if not name.startswith("_")]
