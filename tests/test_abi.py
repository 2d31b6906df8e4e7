"""The C-ABI library loads and exports every entry point include/ckks_mi355x.h
declares; the Python binding covers exactly that set (no GPU calls)."""

from __future__ import annotations

import ctypes
import re
import subprocess
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "ckks_mi355x.h"


def _declared() -> set[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(ckks_[a-z0-9_]+)\s*\(", text))


def test_header_declares_entry_points():
    names = _declared()
    assert {"ckks_context_create", "ckks_rotate_many", "ckks_hoisted_mac_sum",
            "ckks_poly_ntt", "ckks_last_error"} <= names


def test_library_exports_every_declared_symbol():
    from easyfhe import _native

    lib = ctypes.CDLL(str(_native.library_path()))
    for name in sorted(_declared()):
        assert hasattr(lib, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", str(_native.library_path())],
                         capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r"\bT (ckks_[a-z0-9_]+)\b", out))
    assert _declared() <= exported
    # nothing outside the header is exported with the public prefix
    assert exported <= _declared()


def test_python_binding_matches_header():
    from easyfhe import _native

    assert set(_native.SIGNATURES) == _declared()


def test_error_codes_map_to_exceptions():
    from easyfhe import _native

    # a call that fails validation on the host before touching the GPU
    import pytest

    with pytest.raises(ValueError):
        _native.check(_native.lib.ckks_context_create(None, None))


def test_reference_parameter_set_is_accepted_by_the_prime_rule():
    """assets/feature_major.json of the reference: logN 16, depth 37, dnum 5,
    dcrtBits 59, firstMod 60 (38 limbs, 8 special primes)."""
    import math

    import oracle as O

    L, dnum = 38, 5
    alpha = math.ceil(L / dnum)
    q0 = O.gen_primes(16, 60, 1)
    qs = O.gen_primes(16, 59, L - 1, used=q0)
    ps = O.gen_primes(16, 60, alpha, used=q0 + qs)
    assert len(qs) == L - 1 and len(ps) == alpha
    logP = sum(math.log2(p) for p in ps)
    for j in range(dnum):
        digit = (q0 + qs)[j * alpha:(j + 1) * alpha]
        assert logP > sum(math.log2(q) for q in digit)
