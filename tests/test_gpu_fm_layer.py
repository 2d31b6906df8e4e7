"""Feature-major decoder-layer operators on the GPU, decrypted and compared
with the fp64 layer model (oracle/layer_numpy.py):

* complex pairing and the conjugation split (operators/linear/complex.py);
* RMSNorm with the slim-packed single series evaluation
  (operators/norm/rmsnorm.py), with and without gamma, with a doubled input
  (the complex-paired refresh contract), with its slim refresh, and at the
  full Llama shape (128 tokens x 4096 features at N = 2^16).

Tolerances are stated per test: they bound the CKKS error (scale 2^40) and
the drift of the fixed-scale residual bookkeeping, not the series fits,
which the model evaluates identically.
"""

from __future__ import annotations

import numpy as np
import pytest

import layer_numpy as LN
from conftest import PARAMS, device_context

pytestmark = pytest.mark.gpu

FM_SMALL = dict(log_n=13, depth=13, dnum=4, dcrt_bits=40, first_mod=60, special_bits=60)
# deep enough for a bootstrap beside a layer's blocks
FM_REFRESH = dict(log_n=13, depth=57, dnum=4, dcrt_bits=40, first_mod=60, special_bits=60)


def _stream(client, ctx, x, enc0=700):
    from feature_major import FeatureMajorPrefillLayout

    lay = FeatureMajorPrefillLayout(seq_len=x.shape[0], hidden_dim=x.shape[1],
                                    slots=ctx.max_slots)
    packed = lay.pack(x)
    cts = [client.encrypt(packed[i], enc_id=enc0 + i) for i in range(lay.cipher_count)]
    return lay, cts


def _decrypt_stream(client, lay, cts):
    return lay.unpack(np.stack([client.decrypt(c) for c in cts]))


def test_complex_pair_and_split_roundtrip():
    from feature_major.complex import pair_real_ciphers, split_complex_ciphers_twice

    client, ctx = device_context(FM_SMALL, rotations=(2 * 8192 - 1,), relin=False)
    rng = np.random.default_rng(0)
    slots = ctx.max_slots
    xs = [rng.uniform(-1, 1, slots) for _ in range(4)]
    cts = [client.encrypt(x, enc_id=10 + i) for i, x in enumerate(xs)]
    pairs = pair_real_ciphers(cts, crypto_context=ctx)
    assert len(pairs) == 2
    z = client.decrypt_complex(pairs[1])
    assert np.max(np.abs(z - (xs[2] + 1j * xs[3]))) < 1e-7
    split = split_complex_ciphers_twice(pairs, crypto_context=ctx)
    for x, s in zip(xs, split):
        assert np.max(np.abs(client.decrypt(s) - 2 * x)) < 1e-6
    halved = split_complex_ciphers_twice(pairs, crypto_context=ctx, halve=True)
    for x, s in zip(xs, halved):
        assert int(s.state.cur_limbs) == int(cts[0].state.cur_limbs)
        assert np.max(np.abs(client.decrypt(s) - x)) < 1e-6
    with pytest.raises(ValueError):
        pair_real_ciphers(cts[:3], crypto_context=ctx)


@pytest.mark.parametrize("gamma,scale_in,enc_scale", [(False, 1.0, 2.0 ** 40),
                                                     (True, 1.0, 2.0 ** 40),
                                                     (True, 2.0, 2.0 ** 40),
                                                     (False, 1.0, 2.0 ** 41)])
def test_rmsnorm_matches_poly_model(gamma, scale_in, enc_scale):
    """Inputs at the fixed scale, doubled values (input_value_scale 2), and a
    doubled recorded scale (what the complex-paired refresh returns): the
    series' ladder starts at a prime in every case."""
    from feature_major.approx import rsqrt_entry
    from feature_major.rmsnorm import rmsnorm_depth, rmsnorm_fhe, rmsnorm_rotations
    from feature_major import FeatureMajorPrefillLayout

    tokens, dim = 64, 512
    lay0 = FeatureMajorPrefillLayout(seq_len=tokens, hidden_dim=dim, slots=4096)
    client, ctx = device_context(FM_SMALL, rotations=rmsnorm_rotations(lay0))
    rng = np.random.default_rng(1)
    x = rng.normal(size=(tokens, dim))
    w = rng.normal(1.0, 0.1, dim) if gamma else np.zeros(1)
    entry = rsqrt_entry(0.25, 4.0, 31)
    lay = FeatureMajorPrefillLayout(seq_len=tokens, hidden_dim=dim, slots=ctx.max_slots)
    packed = lay.pack(scale_in * x)
    cts = [client.encrypt(packed[i], scaling_factor=enc_scale, enc_id=800 + i)
           for i in range(lay.cipher_count)]
    res = rmsnorm_fhe(cts, w, coeffs=entry, layout=lay, crypto_context=ctx,
                      input_value_scale=scale_in)
    assert res.output_limbs == int(cts[0].state.cur_limbs) - rmsnorm_depth(entry)
    got = _decrypt_stream(client, lay, res.ciphers)
    want = LN.rmsnorm_poly_numpy(x, entry["coefficients"], entry["fit_interval"])
    if gamma:
        want = want * w[None, :]
    err = float(np.max(np.abs(got - want)))
    assert err < 2e-4, err
    assert set(res.stage_seconds) == {"mean_square_and_slim_pack", "rsqrt_polynomial",
                                      "scale_broadcast_and_output"}


def test_rmsnorm_full_llama_shape():
    """128 tokens x 4096 features in 16 ciphertexts at N = 2^16 on the bench
    chain (60-bit + 35 x 40-bit, dnum 3)."""
    from feature_major import FeatureMajorPrefillLayout
    from feature_major.approx import rsqrt_entry
    from feature_major.rmsnorm import rmsnorm_fhe, rmsnorm_rotations

    lay0 = FeatureMajorPrefillLayout(seq_len=128, hidden_dim=4096, slots=32768)
    client, ctx = device_context(PARAMS["keyswitch"], rotations=rmsnorm_rotations(lay0))
    rng = np.random.default_rng(2)
    x = rng.normal(size=(128, 4096))
    entry = rsqrt_entry(0.25, 4.0, 31)
    lay, cts = _stream(client, ctx, x)
    cts = [c.deep_copy() for c in cts]
    res = rmsnorm_fhe(cts, np.zeros(1), coeffs=entry, layout=lay, crypto_context=ctx)
    got = _decrypt_stream(client, lay, res.ciphers)
    want = LN.rmsnorm_poly_numpy(x, entry["coefficients"], entry["fit_interval"])
    err = float(np.max(np.abs(got - want)))
    print(f"rmsnorm 128x4096: max err {err:.3g}, {res.wall_seconds:.3f} s, "
          f"stages {res.stage_seconds}", flush=True)
    assert err < 2e-4, err


@pytest.mark.parametrize("gamma", [False, True])
def test_rmsnorm_slim_refresh_keeps_the_stream_level(gamma):
    """RMSNorm whose slim series is bootstrapped (the reference's adaptive
    slim refresh, operators/norm/rmsnorm.py:517-566): from the fewest limbs
    the slim path allows, the output loses only the product's level (two with
    gamma), against the fp64 model of the same series; without the refresh
    the same input is too shallow.  64 tokens x 512 features at N = 2^13;
    the tolerance covers one bootstrap (~20 bits) of values below 2."""
    from easyfhe.bs import openfhe as bs
    from feature_major import FeatureMajorPrefillLayout
    from feature_major.approx import rsqrt_entry
    from feature_major.rmsnorm import (SlimRefresh, rmsnorm_depth, rmsnorm_fhe,
                                       rmsnorm_rotations, rmsnorm_slim_refresh_depths)

    tokens, dim = 64, 512
    lay0 = FeatureMajorPrefillLayout(seq_len=tokens, hidden_dim=dim, slots=4096)
    client, ctx = device_context(FM_REFRESH, rotations=rmsnorm_rotations(lay0))
    rng = np.random.default_rng(21)
    x = rng.normal(size=(tokens, dim))
    w = rng.normal(1.0, 0.1, dim) if gamma else np.zeros(1)
    entry = rsqrt_entry(0.25, 4.0, 31)
    lost, need = rmsnorm_slim_refresh_depths(entry, bs.input_limbs(ctx))
    assert lost == 1 and need < rmsnorm_depth(entry) + 2
    lay = FeatureMajorPrefillLayout(seq_len=tokens, hidden_dim=dim, slots=ctx.max_slots)
    packed = lay.pack(x)
    cts = [client.encrypt(packed[i], cur_limbs=need, enc_id=900 + i)
           for i in range(lay.cipher_count)]
    # the series' output is refreshed to one limb above the stream the
    # product takes (the input, or one below it with gamma)
    out_levels = need - (1 if gamma else 0)
    prog = bs.generate(ctx, bs.BootstrapSpec(log_slots=12, level_budget=(3, 3),
                                             output_levels=out_levels))
    with pytest.raises(ValueError):
        rmsnorm_fhe(cts, w, coeffs=entry, layout=lay, crypto_context=ctx)
    res = rmsnorm_fhe(cts, w, coeffs=entry, layout=lay, crypto_context=ctx,
                      slim_refresh=SlimRefresh(prog))
    assert res.output_limbs == need - 1 - (1 if gamma else 0)
    assert "rsqrt_slim_bootstrap" in res.stage_seconds
    got = _decrypt_stream(client, lay, res.ciphers)
    want = LN.rmsnorm_poly_numpy(x, entry["coefficients"], entry["fit_interval"])
    if gamma:
        want = want * w[None, :]
    err = float(np.max(np.abs(got - want)))
    print(f"rmsnorm with slim refresh: {need} -> {res.output_limbs} limbs, max err {err:.3g}",
          flush=True)
    res.release()
    prog.release()
    assert err < 2e-4, err


@pytest.mark.parametrize("limbs", [14, 10])
def test_mlp_matches_poly_model(limbs):
    """SwiGLU with the fitted SiLU series: 64 tokens x 512 features, intermediate
    1408 (three pages, the last one partly active), at N = 2^13; entering with
    spare limbs, or with exactly the MLP's depth + 1 (the output on q_0 alone:
    any growth of the exact scales along the series' ladder would overflow)."""
    from feature_major import FeatureMajorPrefillLayout
    from feature_major.approx import silu_entry
    from feature_major.mlp import FeatureMajorMLPLayout, MLPWeights, mlp_depth, mlp_fhe, \
        mlp_rotations

    from easyfhe import fhe

    tokens, dim, inter = 64, 512, 1408
    lay0 = FeatureMajorPrefillLayout(seq_len=tokens, hidden_dim=dim, slots=4096)
    client, ctx = device_context(FM_SMALL, rotations=mlp_rotations(lay0))
    rng = np.random.default_rng(4)
    x = rng.normal(size=(tokens, dim))
    G = rng.normal(0, 0.05, (inter, dim))
    U = rng.normal(0, 0.05, (inter, dim))
    Dn = rng.normal(0, 0.05, (dim, inter))
    silu = silu_entry()
    lay, cts = _stream(client, ctx, x)
    cts = [fhe.align_to(c, c.state.replace(cur_limbs=limbs, scaling_factor=None), ctx)
           for c in cts]
    mlay = FeatureMajorMLPLayout(lay, inter)
    assert mlay.feature_page_count == 3 and mlay.active_width(2) == 384
    with MLPWeights(G, U, Dn, silu=silu, layout=mlay, context=ctx) as w:
        res = mlp_fhe(cts, w, silu=silu, crypto_context=ctx)
    assert res.output_limbs == int(cts[0].state.cur_limbs) - mlp_depth(silu)
    got = _decrypt_stream(client, lay, res.ciphers)
    want = LN.silu_poly_mlp_numpy(x, G, U, Dn, silu["coefficients"], silu["fit_interval"])
    err = float(np.max(np.abs(got - want)))
    print(f"mlp 64x512 (I=1408) from {limbs} limbs: max err {err:.3g}, "
          f"|y| max {np.max(np.abs(want)):.3g}, "
          f"{res.wall_seconds:.3f} s", flush=True)
    assert err < 1e-5, err


def test_residual_add_matches_exact_scales():
    """A stream at a scale away from the fixed one (as a polynomial ladder's
    output is) plus a fixed-scale stream: the higher operand is re-expressed
    at the other's scale on its spare level; at equal levels both drop one."""
    from easyfhe import fhe
    from feature_major.rmsnorm import match_scale, residual_add

    client, ctx = device_context(FM_SMALL)
    rng = np.random.default_rng(5)
    slots = ctx.max_slots
    a, b = rng.uniform(-1, 1, slots), rng.uniform(-1, 1, slots)
    ca = client.encrypt(a, enc_id=900)
    cb = client.encrypt(b, cur_limbs=8, scaling_factor=2.0 ** 40 * 1.003, enc_id=901)
    low = fhe.align_to(ca, ca.state.replace(cur_limbs=8, scaling_factor=None), ctx)
    with pytest.raises(ValueError):
        fhe.homo_add(low, cb, ctx)
    (out,) = residual_add([ca], [cb], crypto_context=ctx)
    assert int(out.state.cur_limbs) == 8
    assert np.max(np.abs(client.decrypt(out) - (a + b))) < 1e-6
    (out2,) = residual_add([cb], [ca], crypto_context=ctx)
    assert np.max(np.abs(client.decrypt(out2) - (a + b))) < 1e-6
    # equal levels, different scales: both operands drop one level
    (out3,) = residual_add([low], [cb], crypto_context=ctx)
    assert int(out3.state.cur_limbs) == 7
    assert np.max(np.abs(client.decrypt(out3) - (a + b))) < 1e-6
    m = match_scale(ca, 8, float(cb.state.scaling_factor), ctx)
    assert np.max(np.abs(client.decrypt(m) - a)) < 1e-7
    with pytest.raises(ValueError):
        match_scale(cb, 8, 2.0 ** 40, ctx)


FM_DEEP = dict(log_n=13, depth=39, dnum=4, dcrt_bits=40, first_mod=60, special_bits=60)


def _attention_setup(seed=6, rotations=None):
    from feature_major import FeatureMajorPrefillLayout
    from feature_major.attention import AttentionGeometry, attention_rotations

    tokens, dim, heads, hd = 64, 512, 4, 128
    lay0 = FeatureMajorPrefillLayout(seq_len=tokens, hidden_dim=dim, slots=4096)
    geo0 = AttentionGeometry(lay0, heads, hd)
    client, ctx = device_context(FM_DEEP, rotations=rotations or attention_rotations(geo0))
    rng = np.random.default_rng(seed)
    q = rng.normal(0, 0.5, (tokens, dim))
    k = rng.normal(0, 0.5, (tokens, dim))
    v = rng.normal(0, 1.0, (tokens, dim))
    return client, ctx, geo0, q, k, v


def test_qk_scores_layout():
    """Score layout of Q K^T / sqrt(hd) for 64 tokens, 4 heads of 128 at
    N = 2^13 (8 ciphertexts of 8 lanes): every head, query and key offset."""
    from feature_major.attention import qk_scores

    client, ctx, geo, q, k, _ = _attention_setup()
    lay, qc = _stream(client, ctx, q, enc0=1000)
    _, kc = _stream(client, ctx, k, enc0=1100)
    res = qk_scores(qc, kc, geo, crypto_context=ctx, output_scale=1 / np.sqrt(128))
    got = geo.unpack_scores(np.stack([client.decrypt(c) for c in res.ciphers]))
    qh = q.reshape(64, 4, 128).transpose(1, 0, 2)
    kh = k.reshape(64, 4, 128).transpose(1, 0, 2)
    want = qh @ kh.transpose(0, 2, 1) / np.sqrt(128)
    err = float(np.max(np.abs(got - want)))
    print(f"qk 64 tokens x 4 heads: max err {err:.3g} (|s| max {np.abs(want).max():.3g}), "
          f"limbs {int(qc[0].state.cur_limbs)} -> {int(res.ciphers[0].state.cur_limbs)}, "
          f"stages {res.stage_seconds}", flush=True)
    assert int(qc[0].state.cur_limbs) - int(res.ciphers[0].state.cur_limbs) == 4
    assert err < 1e-5, err


def test_pv_output_from_probabilities():
    """Feature-major P V from score-layout probabilities (causal, rows summing
    to one) and a value stream: 64 tokens, 4 heads of 128 at N = 2^13."""
    from feature_major.attention import pv_output

    client, ctx, geo, _, _, v = _attention_setup(seed=7)
    rng = np.random.default_rng(8)
    T = 64
    logits = rng.normal(0, 1, (4, T, T))
    causal = np.tril(np.ones((T, T), dtype=bool))
    e = np.where(causal[None], np.exp(logits), 0.0)
    P = e / e.sum(-1, keepdims=True)
    packed = geo.pack_scores(P)
    pc = [client.encrypt(packed[c], enc_id=1200 + c) for c in range(geo.ciphers)]
    lay, vc = _stream(client, ctx, v, enc0=1300)
    res = pv_output(pc, vc, geo, crypto_context=ctx)
    got = _decrypt_stream(client, lay, res.ciphers)
    vh = v.reshape(T, 4, 128).transpose(1, 0, 2)
    want = (P @ vh).transpose(1, 0, 2).reshape(T, 512)
    err = float(np.max(np.abs(got - want)))
    print(f"pv 64 tokens x 4 heads: max err {err:.3g}, limbs -> "
          f"{int(res.ciphers[0].state.cur_limbs)}, stages {res.stage_seconds}", flush=True)
    assert err < 1e-6, err


def test_attention_matches_alg2_model():
    """Causal attention of 64 tokens, 4 heads of 128 at N = 2^13 (QK, the
    Alg2 softmax with two rounds, PV), against the fp64 model of the same
    algorithm (its series included) and, more loosely, exact attention."""
    from feature_major.attention import SoftmaxConfig, attention_fhe, softmax_depth

    client, ctx, geo, q, k, v = _attention_setup(seed=10)
    cfg = SoftmaxConfig(rounds=2, shift=2.0, bound=2.0)
    lay, qc = _stream(client, ctx, q, enc0=1400)
    _, kc = _stream(client, ctx, k, enc0=1500)
    _, vc = _stream(client, ctx, v, enc0=1600)
    res = attention_fhe(qc, kc, vc, geo, cfg, crypto_context=ctx)
    got = _decrypt_stream(client, lay, res.ciphers)
    model = LN.attention_numpy(q, k, v, 4, probs_fn=lambda s: LN.softmax_alg2_numpy(
        s, cfg.exp(), cfg.first_inverse(), cfg.inverse(64), rounds=2, shift=2.0))
    exact = LN.attention_numpy(q, k, v, 4)
    err = float(np.max(np.abs(got - model)))
    used = int(qc[0].state.cur_limbs) - int(res.ciphers[0].state.cur_limbs)
    print(f"attention 64 tokens x 4 heads: max err {err:.3g} vs model, "
          f"{np.max(np.abs(got - exact)):.3g} vs exact, levels {used} "
          f"(softmax depth {softmax_depth(cfg, 64)}), stages "
          f"{ {k: round(t, 3) for k, t in res.stage_seconds.items()} }", flush=True)
    assert err < 1e-4, err
    assert np.max(np.abs(got - exact)) < 1e-3


FM_LAYER = dict(log_n=13, depth=63, dnum=4, dcrt_bits=40, first_mod=60, special_bits=60)


def test_decoder_layer_matches_poly_model():
    """One decoder layer end to end (RMSNorm, Q/K/V with grouped heads, RoPE,
    attention with the Alg2 softmax, W_o, residual, RMSNorm, SwiGLU MLP,
    residual) for 64 tokens x 512 features, 4 query / 2 key-value heads of
    128, intermediate 1408, at N = 2^13 on a 64-limb chain (no refresh);
    against the fp64 model of the same layer."""
    from feature_major import FeatureMajorPrefillLayout
    from feature_major.approx import rsqrt_entry, silu_entry
    from feature_major.attention import SoftmaxConfig
    from feature_major.layer import (DecoderLayerWeights, LayerApproximations,
                                     decoder_layer_depth, decoder_layer_fhe,
                                     decoder_layer_rotations)

    T, D, H, KV, hd, I = 64, 512, 4, 2, 128, 1408
    lay0 = FeatureMajorPrefillLayout(seq_len=T, hidden_dim=D, slots=4096)
    client, ctx = device_context(FM_LAYER, rotations=decoder_layer_rotations(lay0, H, hd))
    rng = np.random.default_rng(12)
    x = rng.normal(0, 1, (T, D))
    sd = 1.0 / np.sqrt(D)
    wq, wo = rng.normal(0, sd, (D, D)), rng.normal(0, sd, (D, D))
    wk, wv = rng.normal(0, sd, (KV * hd, D)), rng.normal(0, sd, (KV * hd, D))
    G, U = rng.normal(0, sd, (I, D)), rng.normal(0, sd, (I, D))
    Dn = rng.normal(0, 1.0 / np.sqrt(I), (D, I))
    ap = LayerApproximations(rsqrt_entry(0.25, 4.0, 31), rsqrt_entry(0.25, 4.0, 31),
                             silu_entry(), SoftmaxConfig(rounds=2, shift=4.0, bound=4.0))
    assert decoder_layer_depth(ap, T) + 1 <= 64
    lay, xc = _stream(client, ctx, x, enc0=1700)
    with DecoderLayerWeights(wq, wk, wv, wo, G, U, Dn, heads=H, kv_heads=KV, head_dim=hd,
                             intermediate=I, approx=ap, layout=lay, context=ctx) as w:
        res = decoder_layer_fhe(xc, w, crypto_context=ctx)
    got = _decrypt_stream(client, lay, res.ciphers)
    sm = ap.softmax
    kw = dict(heads=H, kv_heads=KV, head_dim=hd, input_norm=ap.input_norm,
              post_attention_norm=ap.post_attention_norm, silu=ap.silu)
    model = LN.decoder_layer_numpy(x, wq, wk, wv, wo, G, U, Dn, probs_fn=lambda s: (
        LN.softmax_alg2_numpy(s, sm.exp(), sm.first_inverse(), sm.inverse(T),
                              rounds=sm.rounds, shift=sm.shift)), **kw)
    exact_softmax = LN.decoder_layer_numpy(x, wq, wk, wv, wo, G, U, Dn, **kw)
    err = float(np.max(np.abs(got - model)))
    print(f"layer 64x512: max err {err:.3g} vs model, "
          f"{np.max(np.abs(got - exact_softmax)):.3g} vs exact softmax, "
          f"|out| {np.abs(model).max():.3g}, limbs 64 -> {res.output_limbs}, "
          f"{res.wall_seconds:.2f} s", flush=True)
    assert err < 1e-4, err


def test_refreshed_decoder_layer_matches_poly_model():
    """The layer with its three paired refresh points (bootstraps of the
    residual stream before each RMSNorm and of the softmax's mapped scores),
    two layers in a row from a one-limb input, 64 tokens x 512 features at
    N = 2^13: against the fp64 model of the same two layers.  The tolerance
    covers six bootstraps at ~20 bits on values up to 32."""
    from feature_major import FeatureMajorPrefillLayout
    from feature_major.approx import rsqrt_entry, silu_entry
    from feature_major.attention import SoftmaxConfig
    from feature_major.layer import (DecoderLayerWeights, LayerApproximations,
                                     decoder_layer_refreshed_fhe, decoder_layer_rotations,
                                     refreshed_layer_depths, refreshed_layer_programs)

    T, D, H, KV, hd, I = 64, 512, 4, 2, 128, 1408
    lay0 = FeatureMajorPrefillLayout(seq_len=T, hidden_dim=D, slots=4096)
    client, ctx = device_context(FM_REFRESH, rotations=decoder_layer_rotations(lay0, H, hd))
    # the residual stream's variance grows past 4 by the second layer
    norm = rsqrt_entry(0.5, 16.0, 63)
    ap = LayerApproximations(norm, norm, silu_entry(), SoftmaxConfig(rounds=2, shift=4.0,
                                                                     bound=4.0))
    # a score program at the score block's depth, a shallower one for the
    # residual stream
    prog, res_prog = refreshed_layer_programs(ctx, ap, T, log_slots=12)
    a, b, c = refreshed_layer_depths(ap, T)
    assert prog.output_limbs == b + 1 and res_prog.output_limbs == max(a, c) + 2
    rng = np.random.default_rng(13)
    x = rng.normal(0, 1, (T, D))
    sd = 1.0 / np.sqrt(D)
    wq, wo = rng.normal(0, sd, (D, D)), rng.normal(0, sd, (D, D))
    wk, wv = rng.normal(0, sd, (KV * hd, D)), rng.normal(0, sd, (KV * hd, D))
    G, U = rng.normal(0, sd, (I, D)), rng.normal(0, sd, (I, D))
    Dn = rng.normal(0, 1.0 / np.sqrt(I), (D, I))
    lay = FeatureMajorPrefillLayout(seq_len=T, hidden_dim=D, slots=ctx.max_slots)
    packed = lay.pack(x)
    xc = [client.encrypt(packed[i], cur_limbs=1, enc_id=1800 + i) for i in range(lay.cipher_count)]
    sm = ap.softmax
    kw = dict(heads=H, kv_heads=KV, head_dim=hd, input_norm=ap.input_norm,
              post_attention_norm=ap.post_attention_norm, silu=ap.silu,
              probs_fn=lambda s: LN.softmax_alg2_numpy(s, sm.exp(), sm.first_inverse(),
                                                       sm.inverse(T), rounds=sm.rounds,
                                                       shift=sm.shift))
    with DecoderLayerWeights(wq, wk, wv, wo, G, U, Dn, heads=H, kv_heads=KV, head_dim=hd,
                             intermediate=I, approx=ap, layout=lay, context=ctx) as w:
        r1 = decoder_layer_refreshed_fhe(xc, w, crypto_context=ctx, program=prog,
                                         residual_program=res_prog)
        r2 = decoder_layer_refreshed_fhe(r1.ciphers, w, crypto_context=ctx, program=prog,
                                         residual_program=res_prog)
    want1 = LN.decoder_layer_numpy(x, wq, wk, wv, wo, G, U, Dn, **kw)
    want2 = LN.decoder_layer_numpy(want1, wq, wk, wv, wo, G, U, Dn, **kw)
    got1 = _decrypt_stream(client, lay, r1.ciphers)
    got2 = _decrypt_stream(client, lay, r2.ciphers)
    e1, e2 = float(np.max(np.abs(got1 - want1))), float(np.max(np.abs(got2 - want2)))
    print(f"refreshed layers 64x512: max err {e1:.3g} / {e2:.3g} vs model, |out| "
          f"{np.abs(want2).max():.3g}, limbs out {r1.output_limbs}, {r2.wall_seconds:.2f} s, "
          f"stages {r2.stage_seconds}", flush=True)
    assert e1 < 1e-3 and e2 < 2e-3, (e1, e2)


def test_pv_output_threshold_refresh():
    """The PairFM threshold refresh (reference operators/attention/config.py:
    44-56): with a threshold above the attention output's limbs, the output
    is refreshed before the pairing for W_o (stage ``refresh_pv_output``) and
    the layer still matches the fp64 model; with the default (no threshold)
    the stage does not run.  64 tokens x 512 features at N = 2^13."""
    from feature_major import FeatureMajorPrefillLayout
    from feature_major.approx import rsqrt_entry, silu_entry
    from feature_major.attention import SoftmaxConfig
    from feature_major.layer import (DecoderLayerWeights, LayerApproximations,
                                     decoder_layer_refreshed_fhe, decoder_layer_rotations,
                                     refreshed_layer_programs)

    T, D, H, KV, hd, I = 64, 512, 4, 2, 128, 1408
    lay0 = FeatureMajorPrefillLayout(seq_len=T, hidden_dim=D, slots=4096)
    client, ctx = device_context(FM_REFRESH, rotations=decoder_layer_rotations(lay0, H, hd))
    norm = rsqrt_entry(0.5, 16.0, 63)
    ap = LayerApproximations(norm, norm, silu_entry(), SoftmaxConfig(rounds=2, shift=4.0,
                                                                     bound=4.0))
    prog, res_prog = refreshed_layer_programs(ctx, ap, T, log_slots=12)
    rng = np.random.default_rng(17)
    x = rng.normal(0, 1, (T, D))
    sd = 1.0 / np.sqrt(D)
    wq, wo = rng.normal(0, sd, (D, D)), rng.normal(0, sd, (D, D))
    wk, wv = rng.normal(0, sd, (KV * hd, D)), rng.normal(0, sd, (KV * hd, D))
    G, U = rng.normal(0, sd, (I, D)), rng.normal(0, sd, (I, D))
    Dn = rng.normal(0, 1.0 / np.sqrt(I), (D, I))
    lay = FeatureMajorPrefillLayout(seq_len=T, hidden_dim=D, slots=ctx.max_slots)
    packed = lay.pack(x)
    xc = [client.encrypt(packed[i], cur_limbs=1, enc_id=1900 + i) for i in range(lay.cipher_count)]
    sm = ap.softmax
    kw = dict(heads=H, kv_heads=KV, head_dim=hd, input_norm=ap.input_norm,
              post_attention_norm=ap.post_attention_norm, silu=ap.silu,
              probs_fn=lambda s: LN.softmax_alg2_numpy(s, sm.exp(), sm.first_inverse(),
                                                       sm.inverse(T), rounds=sm.rounds,
                                                       shift=sm.shift))
    want = LN.decoder_layer_numpy(x, wq, wk, wv, wo, G, U, Dn, **kw)
    with DecoderLayerWeights(wq, wk, wv, wo, G, U, Dn, heads=H, kv_heads=KV, head_dim=hd,
                             intermediate=I, approx=ap, layout=lay, context=ctx) as w:
        plain = decoder_layer_refreshed_fhe(xc, w, crypto_context=ctx, program=prog,
                                            residual_program=res_prog)
        forced = decoder_layer_refreshed_fhe(xc, w, crypto_context=ctx, program=prog,
                                             residual_program=res_prog,
                                             pairfm_refresh_min_limbs=64)
    assert "refresh_pv_output" not in plain.stage_seconds
    assert "refresh_pv_output" in forced.stage_seconds
    e0 = float(np.max(np.abs(_decrypt_stream(client, lay, plain.ciphers) - want)))
    e1 = float(np.max(np.abs(_decrypt_stream(client, lay, forced.ciphers) - want)))
    print(f"PV threshold refresh: max err {e0:.3g} without, {e1:.3g} with, "
          f"{forced.stage_seconds['refresh_pv_output']:.3f} s", flush=True)
    assert e0 < 1e-3 and e1 < 1e-3, (e0, e1)


def _exact_layer_and_ranges(x, wq, wk, wv, wo, G, U, Dn, *, heads, kv_heads, head_dim):
    """The layer with exact RMSNorm, SiLU and softmax, and the ranges its
    nonlinearities saw (the calibration pass)."""
    from feature_major.model import layer_ranges

    T = x.shape[0]
    g = heads // kv_heads
    rep = lambda w: np.repeat(w.reshape(kv_heads, head_dim, -1), g, axis=0).reshape(  # noqa: E731
        heads * head_dim, -1)
    norm = lambda a: a / np.sqrt(np.mean(a * a, axis=-1, keepdims=True) + 1e-5)  # noqa: E731
    n1 = norm(x)
    q = LN.apply_rope_numpy(n1 @ wq.T, heads, head_dim)
    k = LN.apply_rope_numpy(n1 @ rep(wk).T, heads, head_dim)
    v = n1 @ rep(wv).T
    qh, kh = (a.reshape(T, heads, head_dim).transpose(1, 0, 2) for a in (q, k))
    scores = qh @ kh.transpose(0, 2, 1) / np.sqrt(head_dim)
    h1 = x + LN.attention_numpy(q, k, v, heads) @ wo.T
    n2 = norm(h1)
    gate = n2 @ G.T
    out = h1 + ((gate / (1.0 + np.exp(-gate))) * (n2 @ U.T)) @ Dn.T
    return out, layer_ranges(x, h1, gate, scores)


def test_prefill_from_token_ids_to_logits():
    """Three encrypted layers from embedded token ids to the final token's
    logits, 64 tokens x 512 features at N = 2^13, each layer's series fitted
    on ranges calibrated with another token sequence; embedding and LM head
    N(0, 0.02), so the first refresh carries a stream far below one.  Against
    the fp64 model of the same layers (fitted series, Algorithm-2 softmax)."""
    from easyfhe.bs import openfhe as bs
    from feature_major import FeatureMajorPrefillLayout
    from feature_major.layer import DecoderLayerWeights, decoder_layer_rotations
    from feature_major.model import (RangeMargins, approximations_for, embed_tokens,
                                     final_logits, prefill_fhe)

    T, D, H, KV, hd, I, V, n_layers = 64, 512, 4, 2, 128, 1408, 1000, 3
    lay = FeatureMajorPrefillLayout(seq_len=T, hidden_dim=D, slots=4096)
    client, ctx = device_context(FM_REFRESH, rotations=decoder_layer_rotations(lay, H, hd))
    probe = bs.generate(ctx, bs.BootstrapSpec(log_slots=12, level_budget=(3, 3), output_levels=0))
    out_levels = ctx.L - probe.depth_limbs - 1
    prog = bs.generate(ctx, bs.BootstrapSpec(log_slots=12, level_budget=(3, 3),
                                             output_levels=out_levels))
    rng = np.random.default_rng(21)
    embed, head = rng.normal(0, 0.02, (V, D)), rng.normal(0, 0.02, (V, D))
    x = embed_tokens(rng.integers(0, V, T), embed)
    x_cal = embed_tokens(rng.integers(0, V, T), embed)
    margins = RangeMargins(softmax_rounds=2, score_span=10.0)
    sd = 1.0 / np.sqrt(D)
    layers, bounds, want = [], [], x
    try:
        for _ in range(n_layers):
            wq, wo = rng.normal(0, sd, (D, D)), rng.normal(0, sd, (D, D))
            wk, wv = rng.normal(0, sd, (KV * hd, D)), rng.normal(0, sd, (KV * hd, D))
            G, U = rng.normal(0, sd, (I, D)), rng.normal(0, sd, (I, D))
            Dn = rng.normal(0, 1.0 / np.sqrt(I), (D, I))
            x_cal, ranges = _exact_layer_and_ranges(x_cal, wq, wk, wv, wo, G, U, Dn, heads=H,
                                                    kv_heads=KV, head_dim=hd)
            ap, bound = approximations_for(ranges, margins)
            sm = ap.softmax
            want = LN.decoder_layer_numpy(
                want, wq, wk, wv, wo, G, U, Dn, heads=H, kv_heads=KV, head_dim=hd,
                input_norm=ap.input_norm, post_attention_norm=ap.post_attention_norm,
                silu=ap.silu,
                probs_fn=lambda s, sm=sm: LN.softmax_alg2_numpy(
                    s, sm.exp(), sm.first_inverse(), sm.inverse(T), rounds=sm.rounds,
                    shift=sm.shift))
            layers.append(DecoderLayerWeights(wq, wk, wv, wo, G, U, Dn, heads=H, kv_heads=KV,
                                              head_dim=hd, intermediate=I, approx=ap,
                                              layout=lay, context=ctx))
            bounds.append(bound)
        packed = lay.pack(x)
        xc = [client.encrypt(packed[i], cur_limbs=1, enc_id=1900 + i)
              for i in range(lay.cipher_count)]
        res = prefill_fhe(xc, layers, crypto_context=ctx, program=prog, residual_bounds=bounds)
        got = _decrypt_stream(client, lay, res.ciphers)
        res.release()
    finally:
        for w in layers:
            w.close()
    ones = np.ones(D)
    lg, lw = (final_logits(h, norm_weight=ones, lm_head=head) for h in (got, want))
    e_h, e_l = float(np.max(np.abs(got - want))), float(np.max(np.abs(lg - lw)))
    print(f"prefill 3 layers 64x512: hidden err {e_h:.3g} (|h| {np.abs(want).max():.3g}), "
          f"logits err {e_l:.3g} (|logit| {np.abs(lw).max():.3g}), bounds {bounds}, "
          f"{res.wall_seconds:.2f} s", flush=True)
    assert int(np.argmax(lg)) == int(np.argmax(lw))
    assert e_h < 2e-3 and e_l < 1e-4, (e_h, e_l)
