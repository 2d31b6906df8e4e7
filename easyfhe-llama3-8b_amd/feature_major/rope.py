"""Rotary position embedding on feature-major streams (the reference applies
it in plaintext form in approx/attention.py:22-70 and inside its attention
input transforms).

Feature ``h hd + d`` of token i pairs with ``h hd + d +- hd/2``:
``x'[d] = x[d] cos(i w_d) - x[d + hd/2] sin(i w_d)`` for ``d < hd/2`` and
``x'[d] = x[d] cos(i w_(d - hd/2)) + x[d - hd/2] sin(i w_(d - hd/2))`` above,
with ``w_j = theta^(-2j / hd)``.  On a feature-major ciphertext that is
``x * C + rot(x, hd/2 * L) * S1 + rot(x, -hd/2 * L) * S2`` with per-slot
plaintexts C, S1, S2 (token ``c L + l``): two rotations (batched over the
stream) and one level.
"""

from __future__ import annotations

import numpy as np

from easyfhe import fhe

from .layout import FeatureMajorPrefillLayout


def _ctx(context):
    return getattr(context, "context", context)


def _release(values) -> None:
    for v in values or ():
        if v is not None:
            v.release()


def rope_angles(positions, head_dim: int, theta: float = 500000.0) -> np.ndarray:
    """[len(positions), head_dim / 2] angles ``p * theta^(-2j / hd)``."""
    inv = 1.0 / (float(theta) ** (np.arange(0, int(head_dim), 2, dtype=np.float64)
                                  / float(head_dim)))
    return np.outer(np.asarray(positions, dtype=np.float64), inv)


def rope_rotations(layout: FeatureMajorPrefillLayout, head_dim: int) -> tuple[int, int]:
    s = (int(head_dim) // 2) * int(layout.tokens_per_cipher)
    return (s, -s)


def rope_plaintext_rows(layout: FeatureMajorPrefillLayout, head_dim: int, c: int,
                        theta: float = 500000.0, start_pos: int = 0) -> np.ndarray:
    """[3, slots]: C, S1, S2 of ciphertext c (zero on padding tokens)."""
    L, D, hd = int(layout.tokens_per_cipher), int(layout.hidden_dim), int(head_dim)
    half = hd // 2
    rows = np.zeros((3, int(layout.slots)))
    f = np.arange(D)
    d = f % hd
    j = d % half
    for l in range(layout.active_tokens(int(c))):
        ang = rope_angles([start_pos + int(c) * L + l], hd, theta)[0][j]
        s = f * L + l
        rows[0, s] = np.cos(ang)
        rows[1, s] = np.where(d < half, -np.sin(ang), 0.0)
        rows[2, s] = np.where(d >= half, np.sin(ang), 0.0)
    return rows


def rope_fhe(stream, layout: FeatureMajorPrefillLayout, *, head_dim: int, crypto_context,
             theta: float = 500000.0, start_pos: int = 0) -> tuple:
    """RoPE of every head of a feature-major stream; inputs are not consumed."""
    ctx = _ctx(crypto_context)
    xs = list(stream)
    if len(xs) != int(layout.cipher_count):
        raise ValueError(f"RoPE expects {layout.cipher_count} ciphertexts.")
    if int(head_dim) % 2 or int(layout.hidden_dim) % int(head_dim):
        raise ValueError("head_dim must be even and divide the hidden width.")
    up, down = rope_rotations(layout, head_dim)
    ra = fhe.homo_rotate_many(xs, up, ctx)
    rb = fhe.homo_rotate_many(xs, down, ctx)
    limbs = int(xs[0].state.cur_limbs)
    out = []
    try:
        for c, (x, a, b) in enumerate(zip(xs, ra, rb)):
            rows = rope_plaintext_rows(layout, head_dim, c, theta, start_pos)
            pts = fhe.encode_rows_cached(ctx, rows, limbs=limbs, scale=ctx.scale_at(limbs),
                                         slots=ctx.max_slots)
            t = [fhe.homo_mul_pt(x, pts[0], ctx), fhe.homo_mul_pt(a, pts[1], ctx),
                 fhe.homo_mul_pt(b, pts[2], ctx)]
            _release(pts)
            s1 = fhe.homo_add(t[0], t[1], ctx)
            s2 = fhe.homo_add(s1, t[2], ctx)
            _release(t + [s1])
            out.append(s2)
        res = fhe.rescale_many(out, ctx)
        return tuple(res)
    finally:
        _release(out)
        _release(ra)
        _release(rb)


__all__ = ["rope_angles", "rope_fhe", "rope_plaintext_rows", "rope_rotations"]
