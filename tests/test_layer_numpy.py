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


def test_alg2_softmax_model_converges_to_softmax():
    """The Alg2 model with the fitted series equals the exact causal softmax
    (with exact exp and inverse the rounds turn exp(s / 2^k) into
    exp(s) / sum exp(s) for any k); a round too few for its 2^-k scaling
    would give the softmax at twice the temperature instead."""
    from feature_major.attention import SoftmaxConfig

    rng = np.random.default_rng(9)
    T, H = 32, 3
    s = rng.uniform(-3.5, 3.5, (H, T, T))
    cfg = SoftmaxConfig(rounds=2, shift=4.0, bound=4.0)
    got = LN.softmax_alg2_numpy(s, cfg.exp(), cfg.first_inverse(), cfg.inverse(T),
                                rounds=2, shift=4.0)
    valid = np.tril(np.ones((T, T), dtype=bool))[None]
    e = np.where(valid, np.exp(s), 0.0)
    want = e / e.sum(-1, keepdims=True)
    assert np.max(np.abs(got - want)) < 1e-4
    # one round on half the score range (the first inverse's interval is
    # set by exp(2 (s - shift) / 2^k), so it is the same here)
    one = SoftmaxConfig(rounds=1, shift=2.0, bound=2.0)
    half = s / 2
    e1 = np.where(valid, np.exp(half), 0.0)
    assert np.max(np.abs(LN.softmax_alg2_numpy(half, one.exp(), one.first_inverse(),
                                               one.inverse(T), rounds=1, shift=2.0)
                         - e1 / e1.sum(-1, keepdims=True))) < 1e-4
    e2 = np.where(valid, np.exp(s / 2), 0.0)
    assert np.max(np.abs(got - e2 / e2.sum(-1, keepdims=True))) > 1e-2
    q = rng.normal(size=(T, H * 16))
    out = LN.attention_numpy(q, q, q, H)
    assert out.shape == (T, H * 16)
    # token 0 attends to itself only
    assert np.allclose(out[0], q[0])


def test_rope_model_matches_product_plaintexts_and_is_a_rotation():
    """RoPE keeps each (d, d + hd/2) pair's norm and is the identity at
    position 0; the product's per-slot plaintexts (C, S1, S2 with the two
    half-head rotations) reproduce the model on packed rows."""
    from feature_major import FeatureMajorPrefillLayout
    from feature_major.rope import rope_plaintext_rows

    rng = np.random.default_rng(11)
    T, H, hd = 16, 2, 128
    x = rng.normal(size=(T, H * hd))
    y = LN.apply_rope_numpy(x, H, hd)
    assert np.allclose(y[0], x[0])
    xa, xb = x.reshape(T, H, hd)[..., :64], x.reshape(T, H, hd)[..., 64:]
    ya, yb = y.reshape(T, H, hd)[..., :64], y.reshape(T, H, hd)[..., 64:]
    assert np.allclose(xa ** 2 + xb ** 2, ya ** 2 + yb ** 2)
    lay = FeatureMajorPrefillLayout(seq_len=T, hidden_dim=H * hd, slots=4096)
    L = lay.tokens_per_cipher
    packed = lay.pack(x)
    out = np.zeros_like(packed)
    for c in range(lay.cipher_count):
        C, S1, S2 = rope_plaintext_rows(lay, hd, c)
        out[c] = packed[c] * C + np.roll(packed[c], -64 * L) * S1 + np.roll(packed[c], 64 * L) * S2
    assert np.allclose(lay.unpack(out), y)
