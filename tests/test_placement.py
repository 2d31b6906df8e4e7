"""Refresh placement and limb budgets (easyfhe.bs.placement), on the CPU.

The budgets are pinned by the reference's own statements of them: 13 limbs
before QKV (llama3fhe/graph.py:784-795), PSdepth(SiLU) + 6 - 1 = 11 limbs
before the MLP for the degree-48 SiLU (graph.py:1246-1259), the PS depths
"degree 48 -> depth 6, degree 60 -> depth 7" of approx/chebyshev.py, and the
clamp of operators/norm/refresh.py:70-93.
"""

from __future__ import annotations

import math

import numpy as np
import pytest

from easyfhe.bs import placement as pl


def test_reference_ps_split_is_valid_and_tabulated():
    # k (2^m - 1) > n: the PS split covers the degree, for every tabulated n
    for n in range(1, 2205):
        k, m = pl.reference_ps_degrees(n)
        assert k * ((1 << m) - 1) > n >= (k - 1) * ((1 << m) - 1)
    assert pl.reference_ps_degrees(48) == (7, 3)
    assert pl.reference_ps_depth(np.ones(49)) == 6
    assert pl.reference_ps_depth(np.ones(61)) == 7
    assert pl.reference_ps_depth(np.ones(1)) == 0
    with pytest.raises(ValueError):
        pl.reference_ps_degrees(2205)


def test_build_series_depth_never_exceeds_reference_ps_depth():
    for n in range(1, 600):
        c = np.ones(n + 1)
        assert pl.series_depth(c) == math.ceil(math.log2(n + 1))
        assert pl.series_depth(c) <= pl.reference_ps_depth(c)


def test_layer_budgets():
    assert pl.attention_input_min_limbs() == 13
    assert pl.attention_input_min_limbs(pl.RefreshSchedule(attention_extra_limbs=2)) == 15
    silu48 = np.ones(49)
    assert pl.mlp_input_min_limbs(silu48, depth=pl.reference_ps_depth) == 11
    assert pl.mlp_input_min_limbs(silu48) == 11
    # degree 60: the build's evaluator saves the reference one limb
    silu60 = np.ones(61)
    assert pl.mlp_input_min_limbs(silu60, depth=pl.reference_ps_depth) == 12
    assert pl.mlp_input_min_limbs(silu60) == 11
    unfused = pl.RefreshSchedule(fuse_silu_domain_map=False)
    assert pl.mlp_input_min_limbs(silu48, unfused) == 12
    with pytest.raises(ValueError):
        pl.RefreshSchedule(mlp_suffix_limbs=2)


def test_adaptive_level_drop_clamp():
    f = pl.adaptive_bootstrap_output_level_drop
    assert f(current_limbs=20, requested_level_drop=3, rmsnorm_depth=5, minimum_output_limbs=13) == 2
    assert f(current_limbs=20, requested_level_drop=1, rmsnorm_depth=5, minimum_output_limbs=13) == 1
    assert f(current_limbs=10, requested_level_drop=3, rmsnorm_depth=5, minimum_output_limbs=13) == 0
    assert f(current_limbs=10, requested_level_drop=3, rmsnorm_depth=5, minimum_output_limbs=None) == 3
    for bad in (dict(requested_level_drop=-1, rmsnorm_depth=0, minimum_output_limbs=None),
                dict(requested_level_drop=0, rmsnorm_depth=-1, minimum_output_limbs=None),
                dict(requested_level_drop=0, rmsnorm_depth=0, minimum_output_limbs=1)):
        with pytest.raises(ValueError):
            f(current_limbs=10, **bad)


def test_refresh_counts():
    assert pl.refresh_bootstraps(16) == 8
    assert pl.residual_refresh_bootstraps_per_layer(16) == 16
    assert pl.residual_refresh_bootstraps_per_layer(
        16, pl.RefreshSchedule(pair_residual_bootstrap=False)) == 32
    with pytest.raises(ValueError):
        pl.refresh_bootstraps(15)
