"""Every EasyFHE call the reference makes is accepted by this package.

tests/golden/boundary_calls.json lists each call shape in the reference's
llama3fhe/ tree (module, name, positional count, keyword names; written by
tests/golden/make_boundary_fixture.py from an AST scan).  For each one the
name must exist in the matching ``easyfhe`` module and its signature must
bind that many positional arguments and those keywords.  Attribute names the
reference reads (``easyfhe.float64``, ``easyfhe.cuda.current_device``) must
exist too.  Loading the package needs only the built library, not a GPU.
"""

from __future__ import annotations

import importlib
import inspect
import json
from pathlib import Path

import pytest

FIXTURE = Path(__file__).resolve().parent / "golden" / "boundary_calls.json"


@pytest.fixture(scope="module")
def calls():
    if not FIXTURE.exists():
        pytest.skip("boundary fixture not present (tests/golden/make_boundary_fixture.py)")
    return json.loads(FIXTURE.read_text(encoding="utf-8"))


def _resolve(dotted: str):
    parts = dotted.split(".")
    for cut in range(len(parts), 0, -1):
        try:
            obj = importlib.import_module(".".join(parts[:cut]))
        except ImportError:
            continue
        for p in parts[cut:]:
            obj = getattr(obj, p)
        return obj
    raise ImportError(dotted)


def test_every_call_shape_binds(calls):
    bad = []
    for rec in calls["calls"]:
        where = f"{rec['module']}.{rec['name']} ({rec['sites'][0]})"
        try:
            fn = getattr(_resolve(rec["module"]), rec["name"])
        except (AttributeError, ImportError) as e:
            bad.append(f"{where}: missing ({e})")
            continue
        if rec["star"]:
            continue
        try:
            sig = inspect.signature(fn)
        except (TypeError, ValueError):
            continue  # builtins without a signature: existence is the check
        try:
            sig.bind(*([None] * rec["positional"]), **{k: None for k in rec["keywords"]})
        except TypeError as e:
            bad.append(f"{where}: {rec['positional']} positional + {rec['keywords']}: {e}")
    assert not bad, "\n".join(bad)


def test_every_attribute_exists(calls):
    missing = []
    for dotted, sites in calls["names"].items():
        try:
            _resolve(dotted)
        except (AttributeError, ImportError):
            missing.append(f"{dotted} ({sites[0]})")
    assert not missing, missing


def test_fixture_covers_the_hot_path(calls):
    """The scan found the key-switching entry points the reference drives."""
    names = {(r["module"], r["name"]) for r in calls["calls"]}
    for want in ("homo_rotate", "hoisted_mac_sum", "prepare_hoisted_baby_rotations",
                 "homo_mul_relin_rescale_postop", "fast_rotate", "grouped_pairwise_mac",
                 "moddown_from_ext", "rescale", "align_to"):
        assert ("easyfhe.fhe", want) in names, want
    assert ("easyfhe.bs.openfhe", "bootstrap") in names
