"""Shared test set-up.

`gpu`-marked tests run the gfx950 library through the C ABI and compare with
the CPU oracle (oracle/ckks_oracle.c, test infrastructure only); the others
pin the oracle against closed forms and check the host-side plumbing.
"""

from __future__ import annotations

import math
import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT / "easyfhe-llama3-8b_amd", ROOT / "oracle", ROOT):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP library)")
    config.addinivalue_line("markers", "slow: full-size (N = 2^16) case")
    # A session that may run GPU tests loads torch before any test module
    # loads the backend library: torch bundles its own HIP runtime, and the
    # library binds to a runtime already in the process (the full-size
    # prefill test draws its weights with torch on the device).
    expr = str(config.getoption("markexpr", "") or "")
    if "not gpu" not in expr:
        try:
            import torch  # noqa: F401
        except ImportError:
            pass


# Parameter sets shared by the oracle and the device context.
PARAMS = {
    # small chain with three 2-limb digits
    "small": dict(log_n=12, depth=5, dnum=3, dcrt_bits=40, first_mod=60, special_bits=60),
    # CPU matvec workload: N = 2^13, 4 x 40-bit limbs, one 60-bit special prime
    "matvec": dict(log_n=13, depth=3, dnum=4, dcrt_bits=40, first_mod=40, special_bits=60),
    # the matvec ring with 44-bit special primes (the fp64 arithmetic path on
    # the P limbs, as on the keyswitch chain): 6 x 40-bit limbs, three digits
    # of two, P = two 44-bit primes above each 80-bit digit
    "ext44": dict(log_n=13, depth=5, dnum=3, dcrt_bits=40, first_mod=40, special_bits=44),
    # keyswitch workload: N = 2^16, 60-bit + 35 x 40-bit, dnum 3, 12 44-bit special
    # primes (P = 2^528 above the largest digit, 2^500)
    "keyswitch": dict(log_n=16, depth=35, dnum=3, dcrt_bits=40, first_mod=60, special_bits=44),
}


def oracle_context(name_or_params, seed: int = 0, secret_mode: int = 0, h: int = 192):
    import oracle as O

    p = PARAMS[name_or_params] if isinstance(name_or_params, str) else name_or_params
    L = p["depth"] + 1
    ds = math.ceil(L / p["dnum"])
    return O.OracleContext(log_n=p["log_n"], limbs=L, alpha=ds, dnum=p["dnum"],
                           first_bits=p["first_mod"], dcrt_bits=p["dcrt_bits"],
                           special_bits=p["special_bits"], seed=seed,
                           secret_mode=secret_mode, hamming_weight=h)


def device_context(name_or_params, seed: int = 0, rotations=(), relin: bool = True):
    from easyfhe import fhe

    p = PARAMS[name_or_params] if isinstance(name_or_params, str) else name_or_params
    spec = fhe.CKKSContextSpec(depth=p["depth"], log_n=p["log_n"], dnum=p["dnum"],
                               dcrt_bits=p["dcrt_bits"], first_mod=p["first_mod"],
                               special_bits=p["special_bits"], seed=seed,
                               rotations=tuple(rotations), relin_key=relin)
    return fhe.generate_client_context(spec, device="cuda")


@pytest.fixture(autouse=True)
def _announce(request):
    # name the case before a GPU step so a failing box still says which one ran
    if request.node.get_closest_marker("gpu") is not None:
        print(f"\n[gpu case] {request.node.nodeid}", flush=True)
    yield
