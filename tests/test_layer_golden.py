"""Pins of the fp64 layer model (oracle/layer_numpy.py) against golden vectors
of the reference's own numpy mathematics (tests/golden/layer_golden.npz,
written by tests/golden/make_layer_fixtures.py from
llama3fhe/approx/attention.py:23-165 and llama3fhe/approx/layer.py:64-149).

The reference computes in float32 and the model in float64, so each
comparison carries a float32-sized tolerance; every planted mistake below (a
plausible misreading of the reference: a RoPE frequency schedule without the
factor 2, interleaved instead of half-split rotation pairs, no 1/sqrt(hd)
score scale, grouped heads taken round-robin) moves the result by far more.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

import layer_numpy as LN

GOLDEN = Path(__file__).resolve().parent / "golden" / "layer_golden.npz"


@pytest.fixture(scope="module")
def g():
    if not GOLDEN.exists():
        pytest.skip("golden vectors not present (tests/golden/make_layer_fixtures.py writes them)")
    with np.load(GOLDEN, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def _rope_freq_without_two(x, heads, hd, theta=500000.0, start_pos=0):
    T = x.shape[0]
    half = hd // 2
    inv = 1.0 / (theta ** (np.arange(half, dtype=np.float64) / hd))
    ang = np.outer(np.arange(start_pos, start_pos + T, dtype=np.float64), inv)
    h = x.reshape(T, heads, hd).astype(np.float64)
    a, b = h[..., :half], h[..., half:]
    c, s = np.cos(ang)[:, None], np.sin(ang)[:, None]
    return np.concatenate([a * c - b * s, b * c + a * s], -1).reshape(T, -1)


def _rope_interleaved(x, heads, hd, theta=500000.0, start_pos=0):
    T = x.shape[0]
    inv = 1.0 / (theta ** (np.arange(0, hd, 2, dtype=np.float64) / hd))
    ang = np.outer(np.arange(start_pos, start_pos + T, dtype=np.float64), inv)
    h = x.reshape(T, heads, hd).astype(np.float64)
    a, b = h[..., 0::2], h[..., 1::2]
    c, s = np.cos(ang)[:, None], np.sin(ang)[:, None]
    y = np.empty_like(h)
    y[..., 0::2], y[..., 1::2] = a * c - b * s, b * c + a * s
    return y.reshape(T, -1)


@pytest.mark.parametrize("case", [0, 1, 2])
def test_rope_matches_reference(g, case):
    T, hd, H, start = (int(v) for v in g[f"rope{case}_shape"])
    x, want = g[f"rope{case}_x"], g[f"rope{case}_y"]
    got = LN.apply_rope_numpy(x, H, hd, 500000.0, start_pos=start)
    # float32 angles at positions up to ~110 carry ~1e-5 relative error
    tol = 3e-7 * (start + T) * max(1.0, float(np.abs(x).max()))
    assert np.max(np.abs(got - want)) < tol
    for wrong in (_rope_freq_without_two, _rope_interleaved):
        assert np.max(np.abs(wrong(x, H, hd, 500000.0, start) - want)) > 100 * tol
    # the reference's cos/sin tables: the two halves repeat the T x hd/2 angles
    cos = g[f"rope{case}_cos"]
    assert np.array_equal(cos[:, : hd // 2], cos[:, hd // 2:])


def _repeat_heads(k, kv, hd, groups):
    T = k.shape[0]
    return np.repeat(k.reshape(T, kv, hd), groups, axis=1).reshape(T, -1)


@pytest.mark.parametrize("case", [0, 1])
def test_grouped_attention_matches_reference(g, case):
    T, H, KV = (int(v) for v in g[f"attn{case}_shape"])
    hd, groups = T, H // KV
    q, k, v = g[f"attn{case}_q"], g[f"attn{case}_k"], g[f"attn{case}_v"]
    kr, vr = _repeat_heads(k, KV, hd, groups), _repeat_heads(v, KV, hd, groups)
    got_p = {}
    got = LN.attention_numpy(q, kr, vr, H, probs_fn=None)
    want = g[f"attn{case}_out"]
    assert np.max(np.abs(got - want)) < 1e-5 * max(1.0, float(np.abs(want).max()))

    # the scores and probabilities the model's softmax sees
    def capture(s):
        got_p["s"] = s
        valid = np.tril(np.ones(s.shape[-2:], dtype=bool))[None]
        m = np.where(valid, s, -np.inf)
        e = np.where(valid, np.exp(m - m.max(-1, keepdims=True)), 0.0)
        got_p["p"] = e / e.sum(-1, keepdims=True)
        return got_p["p"]

    LN.attention_numpy(q, kr, vr, H, probs_fn=capture)
    valid = np.tril(np.ones((T, T), dtype=bool))[None]
    ws = np.where(valid, g[f"attn{case}_scores"], 0.0)
    assert np.max(np.abs(np.where(valid, got_p["s"], 0.0) - ws)) < 1e-5 * float(np.abs(ws).max())
    assert np.max(np.abs(got_p["p"] - g[f"attn{case}_probs"])) < 1e-6

    # planted mistakes: no score scale; KV heads taken round-robin (h % KV)
    unscaled = LN.attention_numpy(q * np.sqrt(hd), kr, vr, H)
    assert np.max(np.abs(unscaled - want)) > 1e-2
    rr = np.tile(k.reshape(T, KV, hd), (1, groups, 1)).reshape(T, -1)
    rv = np.tile(v.reshape(T, KV, hd), (1, groups, 1)).reshape(T, -1)
    assert np.max(np.abs(LN.attention_numpy(q, rr, rv, H) - want)) > 1e-2


def test_poly_layer_matches_reference(g):
    T, H, KV, hd, F = (int(v) for v in g["layer_shape"])
    w = {n: g[f"layer_{n}"] for n in ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj",
                                       "up_proj", "down_proj")}
    ent = {t: {"coefficients": g[f"layer_{t}_coef"], "fit_interval": g[f"layer_{t}_interval"]}
           for t in ("n1", "n2", "silu")}
    x, want = g["layer_x"], g["layer_hidden"]

    def run(**kw):
        return LN.decoder_layer_numpy(x, w["q_proj"], w["k_proj"], w["v_proj"], w["o_proj"],
                                      w["gate_proj"], w["up_proj"], w["down_proj"], heads=H,
                                      kv_heads=KV, head_dim=hd, input_norm=ent["n1"],
                                      post_attention_norm=ent["n2"], silu=ent["silu"], **kw)

    got = run()
    scale = float(np.abs(want).max())
    err = float(np.max(np.abs(got - want)))
    assert err < 2e-6 * scale, err
    # the layer's sub-blocks must all matter at this tolerance: a RoPE base off
    # by a factor, or the two norms' series exchanged, each move it far more
    assert np.max(np.abs(run(theta=10000.0) - want)) > 100 * 2e-6 * scale
    swapped = LN.decoder_layer_numpy(x, w["q_proj"], w["k_proj"], w["v_proj"], w["o_proj"],
                                     w["gate_proj"], w["up_proj"], w["down_proj"], heads=H,
                                     kv_heads=KV, head_dim=hd, input_norm=ent["n2"],
                                     post_attention_norm=ent["n1"], silu=ent["silu"])
    assert np.max(np.abs(swapped - want)) > 100 * 2e-6 * scale
