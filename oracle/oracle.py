"""ctypes wrapper of the CPU oracle (oracle/ckks_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py as the checker.  The product path never imports
this module.

Arrays are numpy uint64 with canonical residues; ciphertexts are
``[degree, limbs, N]``.
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
_LIB_PATH = _HERE / "build" / "libckks_oracle.so"

_u64p = ctypes.POINTER(ctypes.c_uint64)
_dp = ctypes.POINTER(ctypes.c_double)
_lib = None


def build() -> Path:
    """Compile the oracle with its Makefile (gcc, no GPU needed)."""
    subprocess.run(["make", "-s", "-C", str(_HERE)], check=True)
    return _LIB_PATH


def SIGNATURES(vp, i, u64) -> dict:
    """name -> (restype, argtypes) of the oracle's exported functions."""
    return {
        "orc_mulmod": (u64, [u64, u64, u64]),
        "orc_powmod": (u64, [u64, u64, u64]),
        "orc_is_prime": (i, [u64]),
        "orc_gen_primes": (i, [i, i, i, _u64p, i, _u64p]),
        "orc_min_root": (u64, [u64, i]),
        "orc_chacha20_block": (None, [ctypes.POINTER(ctypes.c_uint32), ctypes.c_uint32,
                                      ctypes.POINTER(ctypes.c_uint32),
                                      ctypes.POINTER(ctypes.c_uint32)]),
        "orc_ctx_create": (vp, [i, i, i, i, i, i, i, u64, i, i]),
        "orc_ctx_free": (None, [vp]),
        "orc_set_threads": (None, [i]),
        "orc_N": (i, [vp]),
        "orc_L": (i, [vp]),
        "orc_alpha": (i, [vp]),
        "orc_digit_size": (i, [vp]),
        "orc_primes": (None, [vp, _u64p]),
        "orc_secret": (None, [vp, ctypes.POINTER(ctypes.c_int8)]),
        "orc_ntt_fwd": (None, [vp, i, _u64p]),
        "orc_ntt_inv": (None, [vp, i, _u64p]),
        "orc_ntt_fwd_limbs": (None, [vp, _u64p, i, i]),
        "orc_ntt_inv_limbs": (None, [vp, _u64p, i, i]),
        "orc_automorphism_coeff": (None, [vp, i, u64, _u64p, _u64p]),
        "orc_automorphism_ntt": (None, [vp, u64, _u64p, _u64p, i]),
        "orc_galois_elt": (u64, [vp, ctypes.c_int64]),
        "orc_encode": (i, [vp, _dp, _dp, i, ctypes.c_double, i, i, _u64p]),
        "orc_encode_coeffs": (None, [vp, _dp, _dp, i, ctypes.c_double, _dp]),
        "orc_decode": (None, [vp, _u64p, i, i, ctypes.c_double, _dp, _dp]),
        "orc_gen_rotation_key": (i, [vp, u64]),
        "orc_gen_relin_key": (i, [vp]),
        "orc_get_key": (i, [vp, u64, _u64p]),
        "orc_encrypt": (i, [vp, _dp, _dp, i, ctypes.c_double, i, ctypes.c_uint32, _u64p]),
        "orc_decrypt_poly": (None, [vp, _u64p, i, i, _u64p]),
        "orc_decrypt": (None, [vp, _u64p, i, i, i, ctypes.c_double, _dp, _dp]),
        "orc_add": (None, [vp, _u64p, _u64p, _u64p, i, i]),
        "orc_sub": (None, [vp, _u64p, _u64p, _u64p, i, i]),
        "orc_mul_pt": (None, [vp, _u64p, _u64p, _u64p, i]),
        "orc_mul_monomial_half": (None, [vp, _u64p, _u64p, i, i, i]),
        "orc_tensor": (None, [vp, _u64p, _u64p, _u64p, i]),
        "orc_modup": (None, [vp, _u64p, i, _u64p]),
        "orc_moddown": (None, [vp, _u64p, i, _u64p]),
        "orc_keyswitch": (i, [vp, u64, _u64p, i, _u64p, _u64p]),
        "orc_relinearize": (i, [vp, _u64p, i, _u64p]),
        "orc_rotate": (i, [vp, _u64p, i, u64, _u64p]),
        "orc_hoisted_rotate": (i, [vp, _u64p, i, _u64p, i, _u64p]),
        "orc_rescale": (None, [vp, _u64p, i, i, _u64p]),
        "orc_drop_limbs": (None, [vp, _u64p, i, i, i, _u64p]),
        "orc_mod_raise": (None, [vp, _u64p, i, i, _u64p]),
        "orc_hoisted_mac_sum_ext": (i, [vp, _u64p, i, _u64p, i, _u64p, u64, i, _u64p]),
        "orc_hoisted_mac_sum_double": (i, [vp, _u64p, i, _u64p, i, _u64p, _u64p, i, _u64p]),
        "orc_hoisted_mac_sum": (i, [vp, _u64p, i, _u64p, i, _u64p, u64, i, _u64p]),
    }


_FAST_PATH = _HERE / "build" / "libckks_oracle_fast.so"
_loaded: dict = {}


def load(path=None):
    """The oracle build at ``path`` (default: the pinned checker), its ctypes
    signatures set; each path is loaded once."""
    path = Path(path) if path is not None else _LIB_PATH
    key = str(path.resolve())
    if key in _loaded:
        return _loaded[key]
    if not path.exists():
        build()
    L = ctypes.CDLL(str(path))
    vp = ctypes.c_void_p
    i = ctypes.c_int
    u64 = ctypes.c_uint64
    sig = SIGNATURES(vp, i, u64)
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _loaded[key] = L
    return L


def lib():
    global _lib
    if _lib is None:
        _lib = load(_LIB_PATH)
    return _lib


def fast_library_path() -> Path:
    """The ORC_FAST build (Shoup reductions) that the CPU baseline times."""
    return _FAST_PATH


def _p(a: np.ndarray):
    assert a.dtype == np.uint64 and a.flags["C_CONTIGUOUS"], (a.dtype, a.flags)
    return a.ctypes.data_as(_u64p)


def _d(a: np.ndarray):
    assert a.dtype == np.float64 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(_dp)


def set_threads(n: int) -> None:
    lib().orc_set_threads(int(n))


def gen_primes(log_n: int, bits: int, count: int, used=()) -> list[int]:
    used_arr = np.asarray(list(used) or [0], dtype=np.uint64)
    out = np.zeros(max(1, count), dtype=np.uint64)
    got = lib().orc_gen_primes(log_n, bits, count, _p(used_arr), len(used), _p(out))
    return [int(v) for v in out[:got]]


def chacha20_block(key_words, counter: int, nonce_words) -> np.ndarray:
    k = (ctypes.c_uint32 * 8)(*key_words)
    n = (ctypes.c_uint32 * 3)(*nonce_words)
    o = (ctypes.c_uint32 * 16)()
    lib().orc_chacha20_block(k, counter, n, o)
    return np.array(list(o), dtype=np.uint32)


class OracleContext:
    """CKKS parameters, tables, secret and key store of the CPU oracle."""

    def __init__(self, *, log_n: int, limbs: int, alpha: int, dnum: int,
                 first_bits: int, dcrt_bits: int, special_bits: int, seed: int,
                 secret_mode: int = 0, hamming_weight: int = 192, library=None):
        self._lib = library if library is not None else lib()
        self._c = self._lib.orc_ctx_create(log_n, limbs, alpha, dnum, first_bits, dcrt_bits,
                                       special_bits, seed, secret_mode, hamming_weight)
        if not self._c:
            raise ValueError("oracle context creation failed (prime search)")
        self.N = 1 << log_n
        self.log_n = log_n
        self.L = limbs
        self.alpha = alpha
        self.ds = self._lib.orc_digit_size(self._c)
        self.primes = np.zeros(limbs + alpha, dtype=np.uint64)
        self._lib.orc_primes(self._c, _p(self.primes))

    def close(self):
        if self._c:
            self._lib.orc_ctx_free(self._c)
            self._c = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # -- tables / ntt ---------------------------------------------------------
    def secret(self) -> np.ndarray:
        out = np.zeros(self.N, dtype=np.int8)
        self._lib.orc_secret(self._c, out.ctypes.data_as(ctypes.POINTER(ctypes.c_int8)))
        return out

    def ntt(self, a: np.ndarray, prime_idx: int) -> np.ndarray:
        a = np.ascontiguousarray(a, dtype=np.uint64).copy()
        self._lib.orc_ntt_fwd(self._c, prime_idx, _p(a))
        return a

    def intt(self, a: np.ndarray, prime_idx: int) -> np.ndarray:
        a = np.ascontiguousarray(a, dtype=np.uint64).copy()
        self._lib.orc_ntt_inv(self._c, prime_idx, _p(a))
        return a

    def ntt_limbs(self, a: np.ndarray, q_limbs: int | None = None) -> np.ndarray:
        a = np.ascontiguousarray(a, dtype=np.uint64).copy()
        limbs = a.shape[-2]
        self._lib.orc_ntt_fwd_limbs(self._c, _p(a), limbs, limbs if q_limbs is None else q_limbs)
        return a

    def intt_limbs(self, a: np.ndarray, q_limbs: int | None = None) -> np.ndarray:
        a = np.ascontiguousarray(a, dtype=np.uint64).copy()
        limbs = a.shape[-2]
        self._lib.orc_ntt_inv_limbs(self._c, _p(a), limbs, limbs if q_limbs is None else q_limbs)
        return a

    def automorphism_coeff(self, a: np.ndarray, prime_idx: int, g: int) -> np.ndarray:
        a = np.ascontiguousarray(a, dtype=np.uint64)
        out = np.zeros_like(a)
        self._lib.orc_automorphism_coeff(self._c, prime_idx, g, _p(a), _p(out))
        return out

    def automorphism_ntt(self, a: np.ndarray, g: int) -> np.ndarray:
        a = np.ascontiguousarray(a, dtype=np.uint64)
        out = np.zeros_like(a)
        limbs = a.size // self.N
        self._lib.orc_automorphism_ntt(self._c, g, _p(a), _p(out), limbs)
        return out

    def galois_elt(self, rotation: int) -> int:
        return int(self._lib.orc_galois_elt(self._c, int(rotation)))

    # -- encoding -------------------------------------------------------------
    def encode(self, values, *, slots: int, scale: float, limbs: int,
               is_ext: bool = False) -> np.ndarray:
        z = np.asarray(values, dtype=np.complex128).reshape(-1)
        re = np.ascontiguousarray(z.real)
        im = np.ascontiguousarray(z.imag)
        total = limbs + (self.alpha if is_ext else 0)
        out = np.zeros((total, self.N), dtype=np.uint64)
        if self._lib.orc_encode(self._c, _d(re), _d(im), slots, scale, limbs, int(is_ext), _p(out)):
            raise ValueError("bad slot count")
        return out

    def encode_coeffs(self, values, *, slots: int, scale: float) -> np.ndarray:
        z = np.asarray(values, dtype=np.complex128).reshape(-1)
        re = np.ascontiguousarray(z.real)
        im = np.ascontiguousarray(z.imag)
        out = np.zeros(self.N, dtype=np.float64)
        self._lib.orc_encode_coeffs(self._c, _d(re), _d(im), slots, scale, _d(out))
        return out

    def decode(self, poly: np.ndarray, *, slots: int, scale: float) -> np.ndarray:
        poly = np.ascontiguousarray(poly, dtype=np.uint64)
        re = np.zeros(slots)
        im = np.zeros(slots)
        self._lib.orc_decode(self._c, _p(poly), poly.shape[0], slots, scale, _d(re), _d(im))
        return re + 1j * im

    # -- keys -------------------------------------------------------------------
    def gen_rotation_key(self, g: int) -> None:
        if self._lib.orc_gen_rotation_key(self._c, g):
            raise RuntimeError("key store full")

    def gen_relin_key(self) -> None:
        if self._lib.orc_gen_relin_key(self._c):
            raise RuntimeError("key store full")

    def get_key(self, g: int) -> np.ndarray:
        digits = self._lib.orc_get_key(self._c, g, None)
        if digits < 0:
            raise KeyError(g)
        out = np.zeros((digits, 2, self.L + self.alpha, self.N), dtype=np.uint64)
        self._lib.orc_get_key(self._c, g, _p(out))
        return out

    # -- encryption -----------------------------------------------------------
    def encrypt(self, values, *, slots: int, scale: float, limbs: int,
                enc_id: int) -> np.ndarray:
        z = np.asarray(values, dtype=np.complex128).reshape(-1)
        re = np.ascontiguousarray(z.real)
        im = np.ascontiguousarray(z.imag)
        ct = np.zeros((2, limbs, self.N), dtype=np.uint64)
        if self._lib.orc_encrypt(self._c, _d(re), _d(im), slots, scale, limbs, enc_id, _p(ct)):
            raise ValueError("bad slot count")
        return ct

    def decrypt_poly(self, ct: np.ndarray) -> np.ndarray:
        ct = np.ascontiguousarray(ct, dtype=np.uint64)
        out = np.zeros(ct.shape[1:], dtype=np.uint64)
        self._lib.orc_decrypt_poly(self._c, _p(ct), ct.shape[0], ct.shape[1], _p(out))
        return out

    def decrypt(self, ct: np.ndarray, *, slots: int, scale: float) -> np.ndarray:
        ct = np.ascontiguousarray(ct, dtype=np.uint64)
        re = np.zeros(slots)
        im = np.zeros(slots)
        self._lib.orc_decrypt(self._c, _p(ct), ct.shape[0], ct.shape[1], slots, scale,
                          _d(re), _d(im))
        return re + 1j * im

    # -- evaluation -------------------------------------------------------------
    def add(self, a, b):
        out = np.zeros_like(a)
        self._lib.orc_add(self._c, _p(a), _p(b), _p(out), a.shape[0], a.shape[1])
        return out

    def sub(self, a, b):
        out = np.zeros_like(a)
        self._lib.orc_sub(self._c, _p(a), _p(b), _p(out), a.shape[0], a.shape[1])
        return out

    def mul_pt(self, ct, pt):
        out = np.zeros_like(ct)
        self._lib.orc_mul_pt(self._c, _p(ct), _p(np.ascontiguousarray(pt)), _p(out), ct.shape[1])
        return out

    def mul_i(self, ct, negative: bool = False):
        out = np.zeros_like(ct)
        self._lib.orc_mul_monomial_half(self._c, _p(ct), _p(out), ct.shape[0], ct.shape[1],
                                    int(negative))
        return out

    def tensor(self, a, b):
        out = np.zeros((3,) + a.shape[1:], dtype=np.uint64)
        self._lib.orc_tensor(self._c, _p(a), _p(b), _p(out), a.shape[1])
        return out

    def modup(self, d: np.ndarray) -> np.ndarray:
        d = np.ascontiguousarray(d, dtype=np.uint64)
        limbs = d.shape[0]
        digits = -(-limbs // self.ds)
        ext = np.zeros((digits, limbs + self.alpha, self.N), dtype=np.uint64)
        self._lib.orc_modup(self._c, _p(d), limbs, _p(ext))
        return ext

    def moddown(self, acc: np.ndarray) -> np.ndarray:
        acc = np.ascontiguousarray(acc, dtype=np.uint64)
        limbs = acc.shape[0] - self.alpha
        out = np.zeros((limbs, self.N), dtype=np.uint64)
        self._lib.orc_moddown(self._c, _p(acc), limbs, _p(out))
        return out

    def keyswitch(self, g: int, d: np.ndarray):
        d = np.ascontiguousarray(d, dtype=np.uint64)
        o0 = np.zeros_like(d)
        o1 = np.zeros_like(d)
        if self._lib.orc_keyswitch(self._c, g, _p(d), d.shape[0], _p(o0), _p(o1)):
            raise KeyError(g)
        return o0, o1

    def relinearize(self, ct3):
        out = np.zeros((2,) + ct3.shape[1:], dtype=np.uint64)
        if self._lib.orc_relinearize(self._c, _p(ct3), ct3.shape[1], _p(out)):
            raise KeyError("relinearization key")
        return out

    def rotate_g(self, ct, g: int):
        out = np.zeros_like(ct)
        if self._lib.orc_rotate(self._c, _p(ct), ct.shape[1], g, _p(out)):
            raise KeyError(g)
        return out

    def hoisted_rotate(self, ct, gs):
        gs_arr = np.asarray(gs, dtype=np.uint64)
        out = np.zeros((len(gs),) + ct.shape, dtype=np.uint64)
        if self._lib.orc_hoisted_rotate(self._c, _p(ct), ct.shape[1], _p(gs_arr), len(gs), _p(out)):
            raise KeyError(gs)
        return out

    def rescale(self, ct):
        polys, limbs = ct.shape[0], ct.shape[1]
        out = np.zeros((polys, limbs - 1, self.N), dtype=np.uint64)
        self._lib.orc_rescale(self._c, _p(ct), polys, limbs, _p(out))
        return out

    def mod_raise(self, ct, target: int):
        ct = np.ascontiguousarray(ct, dtype=np.uint64)
        assert ct.shape[1] == 1
        out = np.zeros((ct.shape[0], target, self.N), dtype=np.uint64)
        self._lib.orc_mod_raise(self._c, _p(ct), ct.shape[0], target, _p(out))
        return out

    def drop_limbs(self, ct, target: int):
        return np.ascontiguousarray(ct[:, :target, :])

    def hoisted_mac_sum(self, ct, baby_gs, pts, giant_g: int, giant_count: int):
        gs = np.asarray(baby_gs, dtype=np.uint64)
        pts = np.ascontiguousarray(pts, dtype=np.uint64)
        out = np.zeros_like(ct)
        if self._lib.orc_hoisted_mac_sum(self._c, _p(ct), ct.shape[1], _p(gs), len(gs), _p(pts),
                                     giant_g, giant_count, _p(out)):
            raise KeyError("missing rotation key")
        return out

    def hoisted_mac_sum_ext(self, ct, baby_gs, pts_ext, giant_g: int, giant_count: int):
        """Extended-basis schedule: pts_ext are [G*B][limbs + alpha][N]."""
        gs = np.asarray(baby_gs, dtype=np.uint64)
        pts = np.ascontiguousarray(pts_ext, dtype=np.uint64)
        assert pts.shape[1] == ct.shape[1] + self.alpha
        out = np.zeros_like(ct)
        if self._lib.orc_hoisted_mac_sum_ext(self._c, _p(ct), ct.shape[1], _p(gs), len(gs), _p(pts),
                                         giant_g, giant_count, _p(out)):
            raise KeyError("missing rotation key")
        return out

    def hoisted_mac_sum_double(self, ct, baby_gs, pts_ext, giant_gs):
        """Double-hoisted schedule: giant group g >= 1 rotated in Q u P by its
        own Galois element giant_gs[g] (giant_gs[0] unused), one ModDown of the
        sum; pts_ext are [G*B][limbs + alpha][N] with G = len(giant_gs)."""
        gs = np.asarray(baby_gs, dtype=np.uint64)
        ggs = np.asarray(giant_gs, dtype=np.uint64)
        pts = np.ascontiguousarray(pts_ext, dtype=np.uint64)
        assert pts.shape[1] == ct.shape[1] + self.alpha
        assert pts.shape[0] >= len(gs) * len(ggs)
        out = np.zeros_like(ct)
        if self._lib.orc_hoisted_mac_sum_double(self._c, _p(ct), ct.shape[1], _p(gs), len(gs),
                                            _p(pts), _p(ggs), len(ggs), _p(out)):
            raise KeyError("missing rotation key")
        return out


__all__ = ["OracleContext", "build", "chacha20_block", "gen_primes", "lib", "set_threads"]
