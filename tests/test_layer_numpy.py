"""Pins of the fp64 layer model (oracle/layer_numpy.py) and of the product's
polynomial fits (feature_major/approx.py), on the CPU.

* the direct Chebyshev evaluator against numpy's chebval (a library routine)
  on the affinely mapped points;
* the fitted inverse square root and SiLU series against the functions they
  approximate, over their intervals;
* the polynomial RMSNorm against the exact RMSNorm, within the series error;
* the polynomial SwiGLU MLP against the exact one;
* the feature-major pack of the model against the product's layout.
"""

from __future__ import annotations

import numpy as np
import pytest

import layer_numpy as LN


def test_direct_series_matches_numpy_chebval():
    rng = np.random.default_rng(0)
    c = rng.normal(size=23)
    a, b = -3.0, 5.0
    x = rng.uniform(a, b, 1000)
    y = (2 * x - a - b) / (b - a)
    want = np.polynomial.chebyshev.chebval(y, np.concatenate(([c[0] / 2], c[1:])))
    assert np.allclose(LN.eval_chebyshev_series_direct(x, c, a, b), want, rtol=1e-12, atol=1e-12)
    # a wrong constant-term convention would be caught here
    assert not np.allclose(LN.eval_chebyshev_series_direct(x, c, a, b),
                           np.polynomial.chebyshev.chebval(y, c))


def test_fits_approximate_their_functions():
    from feature_major.approx import rsqrt_entry, silu_entry

    r = rsqrt_entry(0.25, 4.0, 31)
    v = np.linspace(0.25, 4.0, 2001)
    got = LN.eval_chebyshev_series_direct(v, r["coefficients"], 0.25, 4.0)
    assert np.max(np.abs(got - 1 / np.sqrt(v + 1e-5))) < 1e-5
    assert r["max_fit_error"] < 1e-5
    s = silu_entry(-12.0, 12.0, 63)
    g = np.linspace(-12, 12, 2001)
    got = LN.eval_chebyshev_series_direct(g, s["coefficients"], -12.0, 12.0)
    assert np.max(np.abs(got - g / (1 + np.exp(-g)))) < 1e-5


def test_poly_rmsnorm_is_rmsnorm_within_the_fit():
    from feature_major.approx import rsqrt_entry

    rng = np.random.default_rng(1)
    x = rng.normal(size=(64, 512))
    e = rsqrt_entry(0.25, 4.0, 31)
    got = LN.rmsnorm_poly_numpy(x, e["coefficients"], e["fit_interval"])
    exact = x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + 1e-5)
    assert np.max(np.abs(got - exact)) < 1e-4


def test_poly_mlp_is_swiglu_within_the_fit():
    from feature_major.approx import silu_entry

    rng = np.random.default_rng(2)
    x = rng.normal(size=(16, 64))
    G, U = rng.normal(0, 0.1, (96, 64)), rng.normal(0, 0.1, (96, 64))
    Dn = rng.normal(0, 0.1, (64, 96))
    e = silu_entry()
    got = LN.silu_poly_mlp_numpy(x, G, U, Dn, e["coefficients"], e["fit_interval"])
    g = x @ G.T
    exact = ((g / (1 + np.exp(-g))) * (x @ U.T)) @ Dn.T
    assert np.max(np.abs(got - exact)) < 1e-4


@pytest.mark.parametrize("tokens,dim,slots", [(128, 4096, 32768), (60, 512, 4096)])
def test_fm_pack_matches_product_layout(tokens, dim, slots):
    from feature_major import FeatureMajorPrefillLayout

    rng = np.random.default_rng(3)
    x = rng.normal(size=(tokens, dim))
    lay = FeatureMajorPrefillLayout(seq_len=tokens, hidden_dim=dim, slots=slots)
    packed = LN.fm_pack(x, slots)
    assert np.array_equal(packed, lay.pack(x))
    assert np.array_equal(LN.fm_unpack(packed, tokens, dim), x)
    # token t, feature f at slot f * lanes + t % lanes of ciphertext t // lanes
    lanes = slots // dim
    assert packed[5 // lanes, 7 * lanes + 5 % lanes] == x[5, 7]
