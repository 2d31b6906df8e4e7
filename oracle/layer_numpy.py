"""fp64 plaintext model of the encrypted decoder-layer operators.

TEST INFRASTRUCTURE ONLY: imported by tests/ as the checker of decrypted
values.  The product path never imports this module.

Each function restates the mathematics of a reference numpy model that the
reference compares its encrypted layer against:
* ``eval_chebyshev_series_direct``: approx/chebyshev.py:136-163 (the series
  ``c_0/2 + sum_i c_i T_i`` on [a, b], mapped affinely onto [-1, 1]);
* ``rmsnorm_poly_numpy``: approx/rmsnorm.py:24-51 (``x * p(mean(x^2))`` with
  the fitted inverse-square-root series p, no clamping in FHE mode);
* ``silu_poly_mlp_numpy``: the MLP half of approx/layer.py:121-140
  (``down @ (p_silu(gate @ x) * (up @ x))``);
* ``softmax_alg2_numpy``: the "Algorithm 2" softmax of
  operators/attention/softmax.py:648-1262 (exp of the shifted, 2^-k scaled
  scores, then k rounds of squaring and row normalisation), with the given
  series;
* ``attention_numpy``: causal grouped attention, approx/attention.py:134-173;
* ``apply_rope_numpy``: rotary embedding, approx/attention.py:22-70;
* ``decoder_layer_numpy``: the whole layer, approx/layer.py:64-149;
* ``fm_pack`` / ``fm_unpack``: the feature-major token-lane layout of
  layouts/feature_major.py:74-92 (slot = feature * lanes + token % lanes,
  ciphertext = token // lanes).

Pins: ``apply_rope_numpy``, ``attention_numpy`` and ``decoder_layer_numpy``
match golden vectors of the reference's own ``apply_rope_heads``,
``attention_gqa_numpy`` and ``poly_transformer_layer_numpy``
(tests/test_layer_golden.py); the series evaluator, RMSNorm, MLP, Alg2
softmax and packing are pinned by library routines and closed forms
(tests/test_layer_numpy.py).
"""

from __future__ import annotations

import numpy as np


def eval_chebyshev_series_direct(x, coefficients, a: float, b: float) -> np.ndarray:
    """Three-term recurrence T_{n+1} = 2 y T_n - T_{n-1} at y = (2x - a - b)/(b - a)."""
    c = np.asarray(coefficients, dtype=np.float64)
    y = (2.0 * np.asarray(x, dtype=np.float64) - (a + b)) / (b - a)
    if c.size == 0:
        return np.zeros_like(y)
    acc = np.full_like(y, c[0] / 2.0)
    if c.size == 1:
        return acc
    t_prev, t_cur = np.ones_like(y), y
    acc = acc + c[1] * t_cur
    for i in range(2, c.size):
        t_prev, t_cur = t_cur, 2.0 * y * t_cur - t_prev
        acc = acc + c[i] * t_cur
    return acc


def rmsnorm_poly_numpy(x, coefficients, fit_interval) -> np.ndarray:
    """[tokens, hidden] -> x * p(mean(x^2)) per token."""
    x = np.asarray(x, dtype=np.float64)
    lo, hi = (float(v) for v in fit_interval)
    var = np.mean(x * x, axis=-1, keepdims=True)
    return x * eval_chebyshev_series_direct(var, coefficients, lo, hi)


def silu_poly_mlp_numpy(x, gate_weight, up_weight, down_weight, coefficients,
                        fit_interval) -> np.ndarray:
    """[tokens, hidden] -> [tokens, hidden] SwiGLU with the fitted SiLU series."""
    x = np.asarray(x, dtype=np.float64)
    lo, hi = (float(v) for v in fit_interval)
    gate = x @ np.asarray(gate_weight, dtype=np.float64).T
    up = x @ np.asarray(up_weight, dtype=np.float64).T
    act = eval_chebyshev_series_direct(gate, coefficients, lo, hi) * up
    return act @ np.asarray(down_weight, dtype=np.float64).T


def softmax_alg2_numpy(scores, exp_entry, first_inverse, inverse, *, rounds: int,
                       shift: float) -> np.ndarray:
    """Causal softmax of [H, T, T] scores by "Algorithm 2" (the reference's
    encrypted softmax, operators/attention/softmax.py:648-1262): y =
    exp_series((s - shift) / 2^k) on valid keys, then k rounds of
    y <- y^2 * inv(sum_row y^2); the first round's sums are taken as means over
    the valid keys.  With exact series the result is exp(s) / sum exp(s)."""
    s = np.asarray(scores, dtype=np.float64)
    T = s.shape[-1]
    valid = np.tril(np.ones((T, T), dtype=bool))[None]
    count = valid.sum(-1, keepdims=True).astype(np.float64)
    lo, hi = exp_entry["fit_interval"]
    y = np.where(valid, eval_chebyshev_series_direct((s - shift) / 2.0 ** rounds,
                                                     exp_entry["coefficients"], lo, hi), 0.0)
    for r in range(int(rounds)):
        sq = y * y
        tot = sq.sum(-1, keepdims=True)
        e = first_inverse if r == 0 else inverse
        lo, hi = e["fit_interval"]
        if r == 0:
            inv = eval_chebyshev_series_direct(tot / count, e["coefficients"], lo, hi) / count
        else:
            inv = eval_chebyshev_series_direct(tot, e["coefficients"], lo, hi)
        y = sq * inv
    return y


def attention_numpy(q, k, v, heads: int, probs_fn=None) -> np.ndarray:
    """Causal multi-head attention of [T, H hd] streams (heads already
    repeated for grouped queries), scores scaled by 1/sqrt(hd)
    (approx/attention.py:134-173); ``probs_fn`` replaces the exact softmax."""
    q, k, v = (np.asarray(a, dtype=np.float64) for a in (q, k, v))
    T, D = q.shape
    hd = D // int(heads)
    qh, kh, vh = (a.reshape(T, heads, hd).transpose(1, 0, 2) for a in (q, k, v))
    s = qh @ kh.transpose(0, 2, 1) / np.sqrt(hd)
    if probs_fn is None:
        valid = np.tril(np.ones((T, T), dtype=bool))[None]
        m = np.where(valid, s, -np.inf)
        e = np.where(valid, np.exp(m - m.max(-1, keepdims=True)), 0.0)
        p = e / e.sum(-1, keepdims=True)
    else:
        p = probs_fn(s)
    return (p @ vh).transpose(1, 0, 2).reshape(T, D)


def apply_rope_numpy(x, heads: int, head_dim: int, theta: float = 500000.0,
                     start_pos: int = 0) -> np.ndarray:
    """RoPE of [T, heads * hd] rows (approx/attention.py:22-70): pairs (d,
    d + hd/2) rotated by ``p * theta^(-2j / hd)`` at position p."""
    x = np.asarray(x, dtype=np.float64)
    T = x.shape[0]
    hd, half = int(head_dim), int(head_dim) // 2
    inv = 1.0 / (float(theta) ** (np.arange(0, hd, 2, dtype=np.float64) / hd))
    ang = np.outer(np.arange(start_pos, start_pos + T, dtype=np.float64), inv)
    cos, sin = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
    h = x.reshape(T, int(heads), hd)
    a, b = h[..., :half], h[..., half:]
    out = np.concatenate([a * cos - b * sin, b * cos + a * sin], axis=-1)
    return out.reshape(T, -1)


def decoder_layer_numpy(x, wq, wk, wv, wo, gate, up, down, *, heads: int, kv_heads: int,
                        head_dim: int, input_norm, post_attention_norm, silu,
                        probs_fn=None, theta: float = 500000.0) -> np.ndarray:
    """One decoder layer with polynomial RMSNorm and SiLU (approx/layer.py:64-149);
    ``probs_fn`` replaces the exact causal softmax (e.g. the Alg2 model)."""
    x = np.asarray(x, dtype=np.float64)
    g = int(heads) // int(kv_heads)

    def rep(w):
        w = np.asarray(w, dtype=np.float64).reshape(int(kv_heads), int(head_dim), -1)
        return np.repeat(w, g, axis=0).reshape(int(heads) * int(head_dim), -1)

    n1 = rmsnorm_poly_numpy(x, input_norm["coefficients"], input_norm["fit_interval"])
    q = apply_rope_numpy(n1 @ np.asarray(wq).T, heads, head_dim, theta)
    k = apply_rope_numpy(n1 @ rep(wk).T, heads, head_dim, theta)
    v = n1 @ rep(wv).T
    h = x + attention_numpy(q, k, v, heads, probs_fn) @ np.asarray(wo).T
    n2 = rmsnorm_poly_numpy(h, post_attention_norm["coefficients"],
                            post_attention_norm["fit_interval"])
    return h + silu_poly_mlp_numpy(n2, gate, up, down, silu["coefficients"], silu["fit_interval"])


def fm_pack(rows, slots: int) -> np.ndarray:
    """[tokens, dim] -> [ceil(tokens / lanes), slots], lanes = slots // dim."""
    rows = np.asarray(rows)
    tokens, dim = rows.shape
    lanes = slots // dim
    count = -(-tokens // lanes)
    out = np.zeros((count, slots), dtype=rows.dtype)
    for t in range(tokens):
        out[t // lanes, np.arange(dim) * lanes + t % lanes] = rows[t]
    return out


def fm_unpack(packed, tokens: int, dim: int) -> np.ndarray:
    packed = np.asarray(packed)
    slots = packed.shape[1]
    lanes = slots // dim
    out = np.zeros((tokens, dim), dtype=packed.dtype)
    for t in range(tokens):
        out[t] = packed[t // lanes, np.arange(dim) * lanes + t % lanes]
    return out
