"""ctypes binding of libckks_mi355x.so (include/ckks_mi355x.h).

The library is the only compute path: if it is missing this module raises at
import, so nothing can silently fall back to host arithmetic.

A process that also runs torch on the GPU imports torch first: torch ships
its own HIP runtime under unversioned file names, so loaded after this
library it comes up as a second runtime that finds no device; loaded before,
this library binds to that runtime by soname and the two share it.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

_LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libckks_mi355x.so"

CKKS_OK = 0
CKKS_EINVAL = 1
CKKS_ERUNTIME = 2
CKKS_ENOKEY = 3


class ckks_params(ctypes.Structure):
    _fields_ = [
        ("log_n", ctypes.c_int),
        ("depth", ctypes.c_int),
        ("dnum", ctypes.c_int),
        ("dcrt_bits", ctypes.c_int),
        ("first_mod", ctypes.c_int),
        ("special_bits", ctypes.c_int),
        ("secret_mode", ctypes.c_int),
        ("hamming_weight", ctypes.c_int),
        ("seed", ctypes.c_uint64),
    ]


class ckks_context_info(ctypes.Structure):
    _fields_ = [
        ("N", ctypes.c_int),
        ("log_n", ctypes.c_int),
        ("L", ctypes.c_int),
        ("alpha", ctypes.c_int),
        ("digit_size", ctypes.c_int),
        ("dnum", ctypes.c_int),
        ("max_slots", ctypes.c_int),
        ("default_scale", ctypes.c_double),
    ]


class ckks_ct_info(ctypes.Structure):
    _fields_ = [
        ("polys", ctypes.c_int),
        ("limbs", ctypes.c_int),
        ("is_ext", ctypes.c_int),
        ("slots", ctypes.c_int),
        ("scale_degree", ctypes.c_int),
        ("scale", ctypes.c_double),
    ]


VP = ctypes.c_void_p
VPP = ctypes.POINTER(ctypes.c_void_p)
I = ctypes.c_int
U64P = ctypes.POINTER(ctypes.c_uint64)
I64P = ctypes.POINTER(ctypes.c_int64)
DP = ctypes.POINTER(ctypes.c_double)

# name -> (restype, argtypes); every function declared in include/ckks_mi355x.h
SIGNATURES = {
    "ckks_last_error": (ctypes.c_char_p, []),
    "ckks_context_create": (I, [ctypes.POINTER(ckks_params), VPP]),
    "ckks_context_destroy": (None, [VP]),
    "ckks_context_info_get": (I, [VP, ctypes.POINTER(ckks_context_info)]),
    "ckks_context_primes": (I, [VP, U64P]),
    "ckks_context_secret": (I, [VP, ctypes.POINTER(ctypes.c_int8)]),
    "ckks_scale_at": (ctypes.c_double, [VP, I]),
    "ckks_rescale_divisor_at": (ctypes.c_double, [VP, I]),
    "ckks_galois_element": (ctypes.c_uint64, [VP, ctypes.c_int64]),
    "ckks_keygen_rotations": (I, [VP, I64P, I]),
    "ckks_keygen_relin": (I, [VP]),
    "ckks_has_rotation_key": (I, [VP, ctypes.c_int64]),
    "ckks_key_download": (I, [VP, ctypes.c_uint64, U64P, ctypes.POINTER(I)]),
    "ckks_clear_rotation_keys": (I, [VP, I64P, I]),
    "ckks_synchronize": (I, [VP]),
    "ckks_memory_info": (I, [VP, ctypes.POINTER(ctypes.c_size_t), ctypes.POINTER(ctypes.c_size_t)]),
    "ckks_memory_stats": (I, [VP, ctypes.POINTER(ctypes.c_size_t), ctypes.POINTER(ctypes.c_size_t),
                              ctypes.POINTER(ctypes.c_uint64)]),
    "ckks_empty_cache": (I, [VP]),
    "ckks_encrypt": (I, [VP, DP, DP, I, I, ctypes.c_double, ctypes.c_uint32, VPP]),
    "ckks_decrypt": (I, [VP, VP, DP, DP]),
    "ckks_encode_rows": (I, [VP, DP, DP, I, I, I, ctypes.c_double, I, VPP]),
    "ckks_encode_scalar": (I, [VP, ctypes.c_double, I, ctypes.c_double, VPP]),
    "ckks_decode": (I, [VP, VP, DP, DP]),
    "ckks_ct_upload": (I, [VP, U64P, I, I, I, I, ctypes.c_double, I, VPP]),
    "ckks_ct_download": (I, [VP, VP, U64P]),
    "ckks_ct_info_get": (I, [VP, ctypes.POINTER(ckks_ct_info)]),
    "ckks_ct_set_scale": (I, [VP, ctypes.c_double, I]),
    "ckks_ct_copy": (I, [VP, VP, VPP]),
    "ckks_ct_free": (None, [VP]),
    "ckks_add": (I, [VP, VP, VP, VPP]),
    "ckks_sub": (I, [VP, VP, VP, VPP]),
    "ckks_add_many": (I, [VP, VPP, VPP, I, I, VPP]),
    "ckks_add_pt": (I, [VP, VP, VP, VPP]),
    "ckks_mul_pt": (I, [VP, VP, VP, VPP]),
    "ckks_grouped_mac": (I, [VP, VPP, VPP, ctypes.POINTER(ctypes.c_int), I, VPP]),
    "ckks_mul_i": (I, [VP, VP, I, VPP]),
    "ckks_add_scalar": (I, [VP, VP, VP, VPP]),
    "ckks_mul_scalar": (I, [VP, VP, VP, VPP]),
    "ckks_mul_no_relin": (I, [VP, VP, VP, VPP]),
    "ckks_relinearize": (I, [VP, VP, VPP]),
    "ckks_mul_relin": (I, [VP, VP, VP, VPP]),
    "ckks_rescale": (I, [VP, VP, VPP]),
    "ckks_drop_limbs": (I, [VP, VP, I, VPP]),
    "ckks_rotate": (I, [VP, VP, ctypes.c_int64, VPP]),
    "ckks_mod_raise": (I, [VP, VP, I, VPP]),
    "ckks_rotate_many": (I, [VP, VPP, I, ctypes.c_int64, VPP]),
    "ckks_rotate_many_noalloc": (I, [VP, VPP, I, ctypes.c_int64, VPP]),
    "ckks_mul_relin_rescale_postop_many": (I, [VP, VPP, VPP, I, I, VPP, VP, VPP]),
    "ckks_profile_enable": (I, [VP, I]),
    "ckks_int_peak": (I, [VP, I, ctypes.POINTER(ctypes.c_double)]),
    "ckks_profile_read": (I, [VP, ctypes.c_char_p, ctypes.c_size_t]),
    "ckks_mul_relin_rescale_many": (I, [VP, VPP, VPP, I, VPP]),
    "ckks_mul_relin_rescale_many_by": (I, [VP, VPP, VPP, I, I, VPP]),
    "ckks_hoisted_rotate": (I, [VP, VP, I64P, I, VPP]),
    "ckks_hoisted_mac_sum": (I, [VP, VPP, I, VPP, ctypes.c_int64, I, VPP]),
    "ckks_hoisted_mac_sum_ext": (I, [VP, VP, I64P, I, VPP, ctypes.c_int64, I, VPP]),
    "ckks_hoisted_mac_sum_many": (I, [VP, VPP, I, I, VPP, ctypes.c_int64, I, VPP]),
    "ckks_hoisted_rotate_many": (I, [VP, VPP, I, I64P, I, VPP]),
    "ckks_hoisted_rotate_ext": (I, [VP, VP, I64P, I, VPP]),
    "ckks_hoisted_mac_sum_ext_many": (I, [VP, VPP, I, I64P, I, VPP, ctypes.c_int64, I, VPP]),
    "ckks_hoisted_mac_sum_double": (I, [VP, VP, I64P, I, VPP, ctypes.c_int64, I, VPP]),
    "ckks_hoisted_mac_sum_double_many": (I, [VP, VPP, I, I64P, I, VPP, ctypes.c_int64, I,
                                             VPP]),
    "ckks_rescale_many": (I, [VP, VPP, I, VPP]),
    "ckks_rescale_many_by": (I, [VP, VPP, I, I, VPP]),
    "ckks_linear_combination": (I, [VP, VPP, I, I, DP, ctypes.c_double, I, ctypes.c_double, I,
                                    VPP]),
    "ckks_moddown_ext": (I, [VP, VP, VPP]),
    "ckks_tensor_upload": (I, [VP, VP, ctypes.c_size_t, VPP]),
    "ckks_tensor_download": (I, [VP, VP, VP, ctypes.c_size_t]),
    "ckks_tensor_free": (None, [VP]),
    "ckks_encode_token_lane": (I, [VP, VP, I, I, I, I, I, I, I, I, ctypes.c_double, I, VPP]),
    "ckks_encode_structured": (I, [VP, VPP, I, I, I64P, I64P, I64P, DP, I, I, I, I, I, I, I,
                                   ctypes.c_double, I, VPP]),
    "ckks_poly_ntt": (I, [VP, U64P, U64P, I, I, I, I]),
    "ckks_poly_modup": (I, [VP, U64P, I, U64P]),
    "ckks_poly_moddown": (I, [VP, U64P, I, U64P]),
    "ckks_ntt_many": (I, [VP, VPP, I, I]),
    "ckks_event_create": (I, [VP, VPP]),
    "ckks_event_record": (I, [VP]),
    "ckks_event_elapsed_ms": (I, [VP, VP, ctypes.POINTER(ctypes.c_float)]),
    "ckks_event_destroy": (None, [VP]),
    "ckks_context_stream": (I, [VP, VPP]),
    "ckks_audit_read": (I, [VP, ctypes.POINTER(ctypes.c_double), I]),
    "ckks_set_split_parts": (I, [VP, I]),
}


def library_path() -> Path:
    return _LIB_PATH


def _load():
    if not _LIB_PATH.exists():
        raise ImportError(
            f"{_LIB_PATH} is missing: build the gfx950 backend first "
            "(python __graft_entry__.py build, or python easyfhe-llama3-8b_amd/build.py)"
        )
    lib = ctypes.CDLL(str(_LIB_PATH))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = _load()


class BackendError(RuntimeError):
    """Runtime failure reported by the backend."""


def check(rc: int) -> None:
    if rc == CKKS_OK:
        return
    msg = (lib.ckks_last_error() or b"").decode()
    if rc == CKKS_EINVAL:
        raise ValueError(msg)
    raise BackendError(msg)


def ptr_array(handles) -> ctypes.Array:
    arr = (ctypes.c_void_p * max(1, len(handles)))()
    for i, h in enumerate(handles):
        arr[i] = h
    return arr
