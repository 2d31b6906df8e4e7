"""One encrypted Llama decoder layer on feature-major ciphertexts (the
reference's per-layer graph, llama3fhe/graph.py:545-1584, whose plaintext
counterpart is approx/layer.py:64-149):

    h   = x + W_o attention(rope(W_q n1), rope(W_k n1), W_v n1),  n1 = rmsnorm(x)
    out = h + mlp(rmsnorm(h))

* RMSNorm: the slim-packed single-series form (``rmsnorm.rmsnorm_fhe``);
* projections: the BSGS linear engine on complex-paired token ciphertexts
  (``x_2r + i x_(2r+1)``: one real projection serves two token groups), each
  weight halved so that the conjugation split after it returns the real
  streams at their own scale; key/value weights with their rows repeated for
  the grouped query heads (``attention.kv_repeat_rows``);
* RoPE on queries and keys (``rope.rope_fhe``);
* causal attention with the Algorithm-2 softmax (``attention.attention_fhe``);
* the SwiGLU MLP (``mlp.mlp_fhe``);
* residual additions with exact-scale matching (``rmsnorm.residual_add``).

The layer runs without refreshes here: it needs a chain that holds its depth
(``decoder_layer_depth``: 72 levels with a 3-round softmax).  Bootstrap placement for a chain that does not is
``easyfhe.bs.placement``'s.
"""

from __future__ import annotations

import time
from dataclasses import dataclass, field

import numpy as np

from easyfhe import fhe

from .attention import (AttentionGeometry, SoftmaxConfig, attention_fhe, attention_rotations,
                        kv_repeat_rows, softmax_depth)
from .complex import pair_real_ciphers, split_complex_ciphers_twice
from .layout import FeatureMajorPrefillLayout
from .linear import LinearOperator, LinearOperatorConfig, LinearWeight, linear_rotations
from .mlp import FeatureMajorMLPLayout, MLPWeights, mlp_depth, mlp_fhe
from .rmsnorm import (SlimRefresh, refresh_slim, residual_add, rmsnorm_depth, rmsnorm_fhe,
                      rmsnorm_rotations, rmsnorm_slim_refresh_depths)
from .rope import rope_fhe, rope_rotations


def _ctx(context):
    return getattr(context, "context", context)


def _release(values) -> None:
    for v in values or ():
        if v is not None:
            v.release()


@dataclass(frozen=True)
class LayerApproximations:
    """The layer's polynomial entries (the reference's per-layer JSON
    artifacts, application/approx_config.py)."""

    input_norm: dict
    post_attention_norm: dict
    silu: dict
    softmax: SoftmaxConfig


def decoder_layer_depth(approx: LayerApproximations, seq_len: int) -> int:
    return (rmsnorm_depth(approx.input_norm) + 1 + 1 + 4 + softmax_depth(approx.softmax, seq_len)
            + 3 + 1 + 1 + rmsnorm_depth(approx.post_attention_norm) + mlp_depth(approx.silu))


def decoder_layer_rotations(layout: FeatureMajorPrefillLayout, heads: int,
                            head_dim: int) -> tuple[int, ...]:
    geo = AttentionGeometry(layout, heads, head_dim)
    keys = set(linear_rotations(dimension=int(layout.hidden_dim),
                                token_lanes=int(layout.tokens_per_cipher),
                                slots=int(layout.slots), include_conjugation=True))
    keys |= set(rmsnorm_rotations(layout)) | set(attention_rotations(geo))
    keys |= set(rope_rotations(layout, head_dim))
    return tuple(sorted(k for k in keys if k))


class DecoderLayerWeights:
    """A layer's projections resident on the device: W_q, W_k, W_v (rows of
    the key/value heads repeated for the query groups), W_o, each halved for
    the complex-paired projection, and the paged MLP."""

    def __init__(self, q, k, v, o, gate, up, down, *, heads: int, kv_heads: int,
                 head_dim: int, intermediate: int, approx: LayerApproximations,
                 layout: FeatureMajorPrefillLayout, context):
        ctx = _ctx(context)
        D = int(layout.hidden_dim)
        q, o = np.asarray(q, dtype=np.float64), np.asarray(o, dtype=np.float64)
        if q.shape != (D, D) or o.shape != (D, D):
            raise ValueError(f"q and o must be {(D, D)}.")
        kr = kv_repeat_rows(k, query_heads=heads, kv_heads=kv_heads, head_dim=head_dim)
        vr = kv_repeat_rows(v, query_heads=heads, kv_heads=kv_heads, head_dim=head_dim)
        self.layout = layout
        self.geometry = AttentionGeometry(layout, heads, head_dim)
        self.approx = approx
        self._w = []
        try:
            self.q = self._keep(LinearWeight(0.5 * q, context=ctx))
            self.k = self._keep(LinearWeight(0.5 * kr, context=ctx))
            self.v = self._keep(LinearWeight(0.5 * vr, context=ctx))
            self.o = self._keep(LinearWeight(0.5 * o, context=ctx))
            self.mlp = MLPWeights(gate, up, down, silu=approx.silu,
                                  layout=FeatureMajorMLPLayout(layout, intermediate), context=ctx)
        except Exception:
            self.close()
            raise

    def _keep(self, w):
        self._w.append(w)
        return w

    def close(self) -> None:
        for w in self._w:
            w.close()
        self._w = []
        if getattr(self, "mlp", None) is not None:
            self.mlp.close()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


@dataclass
class LayerResult:
    ciphers: tuple
    wall_seconds: float
    stage_seconds: dict = field(default_factory=dict)
    output_limbs: int = 0

    def release(self) -> None:
        _release(self.ciphers)
        self.ciphers = ()


def _paired_projection(op: LinearOperator, paired, weight, ctx) -> tuple:
    out, _ = op.apply(paired, weight)
    try:
        return split_complex_ciphers_twice(out, crypto_context=ctx)
    finally:
        _release(out)


def decoder_layer_fhe(input_ciphers, weights: DecoderLayerWeights, *, crypto_context,
                      rope_theta: float = 500000.0) -> LayerResult:
    """One decoder layer of a feature-major residual stream; the input is not
    consumed."""
    ctx = _ctx(crypto_context)
    lay, geo, ap = weights.layout, weights.geometry, weights.approx
    xs = tuple(input_ciphers)
    need = decoder_layer_depth(ap, geo.seq_len) + 1
    if int(xs[0].state.cur_limbs) < need:
        raise ValueError(f"the layer needs {need} limbs, the input has "
                         f"{int(xs[0].state.cur_limbs)}.")
    sync = ctx.synchronize
    stage: dict[str, float] = {}
    t_start = time.perf_counter()
    op = LinearOperator(context=ctx, token_lanes=geo.lanes,
                        config=LinearOperatorConfig(timed_stages=False))
    keep: list = []
    try:
        t0 = time.perf_counter()
        n1 = rmsnorm_fhe(xs, np.zeros(1), coeffs=ap.input_norm, layout=lay, crypto_context=ctx)
        sync()
        stage["input_rmsnorm"] = time.perf_counter() - t0
        t0 = time.perf_counter()
        z = pair_real_ciphers(n1.ciphers, crypto_context=ctx)
        n1.release()
        q = _paired_projection(op, z, weights.q, ctx)
        k = _paired_projection(op, z, weights.k, ctx)
        v = _paired_projection(op, z, weights.v, ctx)
        op.release_babies(z)
        _release(z)
        sync()
        stage["qkv_projection"] = time.perf_counter() - t0
        t0 = time.perf_counter()
        qr = rope_fhe(q, lay, head_dim=geo.head_dim, crypto_context=ctx, theta=rope_theta)
        kr = rope_fhe(k, lay, head_dim=geo.head_dim, crypto_context=ctx, theta=rope_theta)
        _release(q)
        _release(k)
        sync()
        stage["rope"] = time.perf_counter() - t0
        t0 = time.perf_counter()
        att = attention_fhe(qr, kr, v, geo, ap.softmax, crypto_context=ctx)
        _release(qr)
        _release(kr)
        _release(v)
        sync()
        stage["attention"] = time.perf_counter() - t0
        stage.update({f"attention.{k2}": v2 for k2, v2 in att.stage_seconds.items()})
        t0 = time.perf_counter()
        za = pair_real_ciphers(att.ciphers, crypto_context=ctx)
        att.release()
        o = _paired_projection(op, za, weights.o, ctx)
        op.release_babies(za)
        _release(za)
        h = residual_add(xs, o, crypto_context=ctx)
        _release(o)
        keep = list(h)
        sync()
        stage["output_projection_and_residual"] = time.perf_counter() - t0
        t0 = time.perf_counter()
        n2 = rmsnorm_fhe(h, np.zeros(1), coeffs=ap.post_attention_norm, layout=lay,
                         crypto_context=ctx)
        sync()
        stage["post_attention_rmsnorm"] = time.perf_counter() - t0
        t0 = time.perf_counter()
        m = mlp_fhe(n2.ciphers, weights.mlp, silu=ap.silu, crypto_context=ctx, operator=op)
        n2.release()
        out = residual_add(h, m.ciphers, crypto_context=ctx)
        m.release()
        sync()
        stage["mlp_and_residual"] = time.perf_counter() - t0
        return LayerResult(tuple(out), time.perf_counter() - t_start, stage,
                           int(out[0].state.cur_limbs))
    finally:
        _release(keep)
        op.close()


# ---------------------------------------------------------------------------
# the layer with refreshes (bootstraps included)
# ---------------------------------------------------------------------------


def refresh_stream(ciphers, *, crypto_context, program, value_bound: float = 1.0,
                   group: int = 8) -> list:
    """Refresh a real feature-major stream (reference operators/norm/refresh.py:96-150):
    values divided by the power of two S >= value_bound through the recorded
    scale (no level; S < 1 spreads a small stream over the bootstrap's input
    range), adjacent ciphertexts paired as ``a + i b``, the pairs
    bootstrapped in batched groups (keys and diagonals read once per group),
    the conjugation split's factor 2 and S returned to the recorded scale.
    Inputs are not consumed."""
    from easyfhe.bs import openfhe as bs

    ctx = _ctx(crypto_context)
    if not float(value_bound) > 0.0:
        raise ValueError("the value bound must be positive.")
    S = 2.0 ** int(np.ceil(np.log2(float(value_bound))))
    views = []
    for c in ciphers:
        v = c.deep_copy()
        v.set_scale(float(c.state.scaling_factor) * S, 1)
        views.append(v)
    try:
        pairs = pair_real_ciphers(views, crypto_context=ctx)
    finally:
        _release(views)
    try:
        boots = bs.bootstrap_many(list(pairs), ctx, program, group=int(group))
    finally:
        _release(pairs)
    try:
        out = list(split_complex_ciphers_twice(boots, crypto_context=ctx, halve=True))
    finally:
        _release(boots)
    for o in out:
        o.set_scale(float(o.state.scaling_factor) / S, 1)
    return out


def _land_on_ladder(cts, ctx) -> list:
    """One level down, at exactly the scale of the next prime a series drops
    first (the fixed point of its scale ladder)."""
    from .rmsnorm import match_scale

    out = []
    for c in cts:
        limbs = int(c.state.cur_limbs) - 1
        out.append(match_scale(c, limbs, float(int(ctx.primes()[limbs - 1])), ctx))
    return out


def _drop_owned(cts, limbs: int, ctx) -> list:
    """Modulus drop of refreshed ciphertexts to the ``limbs`` the next block
    uses (every later operation then runs on that many limbs); the inputs
    are consumed.  A block's result is bootstrapped next, and the bootstrap
    may spend one limb bringing the input's scale down to its own, so the
    blocks keep one limb above their depth."""
    out = []
    for c in cts:
        d = fhe.align_to(c, c.state.replace(cur_limbs=min(int(limbs), int(c.state.cur_limbs)),
                                            scaling_factor=None), ctx)
        if d is not c:
            c.release()
        out.append(d)
    return out


def refreshed_layer_depths(approx: LayerApproximations, seq_len: int, *,
                           refresh_normalisers: bool = False,
                           input_limbs: int = 1,
                           slim_rmsnorm: bool = False) -> tuple[int, int, int]:
    """Levels of the three blocks between refreshes: RMSNorm + Q/K/V + RoPE +
    QK; the scores' landing + softmax + PV + W_o; RMSNorm + MLP.  With
    ``refresh_normalisers`` every softmax round's slim normaliser is
    bootstrapped (the reference's per-round lambda refresh,
    operators/attention/softmax.py:1044-1095), so the score block needs the
    main stream's levels or the slim normalisers' need, whichever is larger.
    With ``slim_rmsnorm`` the post-attention RMSNorm's slim series is
    refreshed (operators/norm/rmsnorm.py:517-566, schedule.py
    ``adaptive_rmsnorm_slim_refresh``; the input RMSNorm keeps its depth, as
    in the reference), so the last block needs the MLP's levels plus the
    product's, or the slim path's, whichever is larger.  ``input_limbs`` is
    what a bootstrap input needs (``bs.input_limbs``).  A block's input holds
    its levels plus two limbs."""
    from .attention import softmax_depth_refreshed

    a = rmsnorm_depth(approx.input_norm) + 1 + 1 + 4
    if refresh_normalisers:
        # the softmax input (after the landing) holds b limbs
        main, need = softmax_depth_refreshed(approx.softmax, seq_len, input_limbs)
        b = max(1 + main + 3 + 1, need)
    else:
        b = 1 + softmax_depth(approx.softmax, seq_len) + 3 + 1
    if slim_rmsnorm:
        lost, need = rmsnorm_slim_refresh_depths(approx.post_attention_norm, input_limbs)
        c = max(lost + mlp_depth(approx.silu), need - 2)
    else:
        c = rmsnorm_depth(approx.post_attention_norm) + mlp_depth(approx.silu)
    return a, b, c


def normaliser_program(crypto_context, approx: LayerApproximations, seq_len: int, *,
                       log_slots: int, level_budget=(3, 3)):
    """Bootstrap program for the per-round softmax normalisers: it returns
    the softmax input's level (the highest the squares of any round sit
    at), so that the refreshed normaliser never pulls the main stream down."""
    from easyfhe.bs import openfhe as bs
    from easyfhe.chebyshev import chebyshev_depth

    ctx = _ctx(crypto_context)
    lim = bs.input_limbs(ctx)
    _, b, _ = refreshed_layer_depths(approx, seq_len, refresh_normalisers=True, input_limbs=lim)
    exp_d = chebyshev_depth(approx.softmax.exp()["coefficients"])
    # the score block enters with b + lim limbs; the softmax starts after the
    # landing, the series and the mask
    levels = b + lim - 2 - exp_d - 1
    return bs.generate(ctx, bs.BootstrapSpec(log_slots=int(log_slots),
                                             level_budget=tuple(level_budget),
                                             output_levels=int(levels)))


# |1 / x| on the normalisers' intervals stays below 2^8 (the first round's
# inverse starts at 0.006)
_NORMALISER_BOUND = 256.0


def _refresh_normaliser(ct, ctx, program):
    """One slim normaliser refreshed (``rmsnorm.refresh_slim``): the result
    keeps the program's output scale, because dividing the recorded scale
    instead would leave the normaliser 2^8 below it, and every round's
    product with it would carry that loss into the next round's squares."""
    return refresh_slim(ct, ctx, program, _NORMALISER_BOUND)


def rmsnorm_slim_program(crypto_context, approx: LayerApproximations, seq_len: int, *,
                         log_slots: int, level_budget=(3, 3), refresh_normalisers: bool = False):
    """Bootstrap program for the post-attention RMSNorm's slim refresh: its
    output sits one level above the block's input (``refreshed_layer_depths``
    with ``slim_rmsnorm``: c + 2 limbs), where the extraction lands the
    broadcast on the stream's level."""
    from easyfhe.bs import openfhe as bs

    ctx = _ctx(crypto_context)
    lim = bs.input_limbs(ctx)
    _, _, c = refreshed_layer_depths(approx, seq_len, refresh_normalisers=refresh_normalisers,
                                     input_limbs=lim, slim_rmsnorm=True)
    return bs.generate(ctx, bs.BootstrapSpec(log_slots=int(log_slots),
                                             level_budget=tuple(level_budget),
                                             output_levels=int(c + 2)))


def refreshed_layer_programs(crypto_context, approx: LayerApproximations, seq_len: int, *,
                             log_slots: int, level_budget=(3, 3),
                             refresh_normalisers: bool = False, slim_rmsnorm: bool = False):
    """(score program, residual program): bootstrap programs whose outputs
    hold the score block plus one limb, and the deeper of the two residual
    blocks plus two (``refreshed_layer_depths``).  A bootstrap raises its
    input only to its outputs plus its own depth, so the residual program,
    with fewer output levels, runs every stage on fewer limbs."""
    from easyfhe.bs import openfhe as bs

    ctx = _ctx(crypto_context)
    # the score block ends where the next refresh takes its input: one limb,
    # or two on chains whose one-limb scale is near q_0 (bs.input_limbs)
    lim = bs.input_limbs(ctx)
    a, b, c = refreshed_layer_depths(approx, seq_len, refresh_normalisers=refresh_normalisers,
                                     input_limbs=lim, slim_rmsnorm=slim_rmsnorm)
    spec = lambda levels: bs.BootstrapSpec(log_slots=int(log_slots),  # noqa: E731
                                           level_budget=tuple(level_budget),
                                           output_levels=int(levels))
    probe = bs.generate(ctx, spec(0))
    top = ctx.L - probe.depth_limbs - 1
    probe.release()
    if top < b + lim - 1 or top < max(a, c) + 1:
        raise ValueError(f"the chain's bootstraps return at most {top + 1} limbs; the layer "
                         f"needs {max(b + lim, max(a, c) + 2)}.")
    return bs.generate(ctx, spec(b + lim - 1)), bs.generate(ctx, spec(max(a, c) + 1))


def decoder_layer_refreshed_fhe(input_ciphers, weights: DecoderLayerWeights, *, crypto_context,
                                program, residual_program=None, residual_bound: float = 32.0,
                                group: int = 8, rope_theta: float = 500000.0,
                                normaliser_program=None, rmsnorm_program=None,
                                pairfm_refresh_min_limbs: int | None = None,
                                pv_value_bound: float = 8.0) -> LayerResult:
    """One decoder layer with its refreshes (three paired refresh points: the
    residual stream before each RMSNorm, and the softmax's mapped scores;
    the reference refreshes at the same places, graph.py:780-990,
    operators/norm/refresh.py:153-344, the pre-exp checkpoint of
    operators/attention/softmax.py).  ``program`` refreshes the scores and
    must return the score block's depth plus one limb; ``residual_program``
    (default ``program``) refreshes the residual stream and must return the
    deeper residual block plus two (``refreshed_layer_programs`` makes
    both).  With ``normaliser_program`` (``normaliser_program()``) every
    softmax round's slim normaliser is refreshed as well, which shortens
    the score block (``refreshed_layer_programs(refresh_normalisers=True)``
    sizes the programs for it).  With ``rmsnorm_program``
    (``rmsnorm_slim_program()``) the post-attention RMSNorm refreshes its
    slim series instead of spending the stream's levels on it, which
    shortens the last block (``refreshed_layer_programs(slim_rmsnorm=True)``).
    With ``pairfm_refresh_min_limbs`` the attention output is refreshed
    with the residual program (values through ``pv_value_bound``) when it
    reaches the pairing for W_o below that many limbs: the reference's
    PairFM threshold refresh (operators/attention/config.py:44-56,
    ``pairfm_post_refresh_input_limbs`` of schedule.py), which its release
    schedule fires only where the PV output runs short.  The depth plan
    here keeps the output above the W_o block's need, so the refresh fires
    only for thresholds above that (stage ``refresh_pv_output``).
    The input may sit at any level; it is not consumed."""
    from easyfhe.bs import openfhe as bs

    ctx = _ctx(crypto_context)
    lay, geo, ap = weights.layout, weights.geometry, weights.approx
    a_depth, b_depth, c_depth = refreshed_layer_depths(
        ap, geo.seq_len, refresh_normalisers=normaliser_program is not None,
        input_limbs=bs.input_limbs(ctx), slim_rmsnorm=rmsnorm_program is not None)
    slim = None if rmsnorm_program is None else SlimRefresh(rmsnorm_program)
    refresh_lam = (None if normaliser_program is None
                   else (lambda ct: _refresh_normaliser(ct, ctx, normaliser_program)))
    res_prog = program if residual_program is None else residual_program
    sync = ctx.synchronize
    stage: dict[str, float] = {}
    t_start = time.perf_counter()
    op = LinearOperator(context=ctx, token_lanes=geo.lanes,
                        config=LinearOperatorConfig(timed_stages=False))
    keep: list = []
    try:
        t0 = time.perf_counter()
        x = refresh_stream(input_ciphers, crypto_context=ctx, program=res_prog,
                           value_bound=residual_bound, group=group)
        keep = x
        sync()
        stage["refresh_residual_1"] = time.perf_counter() - t0
        if int(x[0].state.cur_limbs) < max(a_depth, c_depth) + 2:
            raise ValueError("the residual bootstrap program's outputs are too shallow for the "
                             "layer.")
        x = keep = _drop_owned(x, a_depth + 2, ctx)
        t0 = time.perf_counter()
        n1 = rmsnorm_fhe(x, np.zeros(1), coeffs=ap.input_norm, layout=lay, crypto_context=ctx)
        z = pair_real_ciphers(n1.ciphers, crypto_context=ctx)
        n1.release()
        q = _paired_projection(op, z, weights.q, ctx)
        k = _paired_projection(op, z, weights.k, ctx)
        v = _paired_projection(op, z, weights.v, ctx)
        op.release_babies(z)
        _release(z)
        qr = rope_fhe(q, lay, head_dim=geo.head_dim, crypto_context=ctx, theta=rope_theta)
        kr = rope_fhe(k, lay, head_dim=geo.head_dim, crypto_context=ctx, theta=rope_theta)
        _release(q)
        _release(k)
        from .attention import pv_output, qk_scores, softmax_alg2

        sa, sb_ = ap.softmax.score_map(1.0 / float(np.sqrt(geo.head_dim)))
        scores = qk_scores(qr, kr, geo, crypto_context=ctx, output_scale=sa, output_offset=sb_)
        _release(qr)
        _release(kr)
        sync()
        stage["rmsnorm_qkv_rope_qk"] = time.perf_counter() - t0
        t0 = time.perf_counter()
        sr = refresh_stream(scores.ciphers, crypto_context=ctx, program=program, value_bound=1.0,
                            group=group)
        scores.release()
        if int(sr[0].state.cur_limbs) < b_depth + bs.input_limbs(ctx):
            _release(sr)
            raise ValueError("the score bootstrap program's outputs are too shallow for the "
                             "layer.")
        sync()
        stage["refresh_scores"] = time.perf_counter() - t0
        t0 = time.perf_counter()
        landed = _land_on_ladder(sr, ctx)
        _release(sr)
        probs = softmax_alg2(landed, geo, ap.softmax, crypto_context=ctx, refresh=refresh_lam)
        _release(landed)
        att = pv_output(probs.ciphers, v, geo, crypto_context=ctx)
        probs.release()
        _release(v)
        att_c = list(att.ciphers)
        if (pairfm_refresh_min_limbs is not None
                and int(att_c[0].state.cur_limbs) < int(pairfm_refresh_min_limbs)):
            sync()
            t1 = time.perf_counter()
            att_c = refresh_stream(att_c, crypto_context=ctx, program=res_prog,
                                   value_bound=pv_value_bound, group=group)
            att.release()
            sync()
            stage["refresh_pv_output"] = time.perf_counter() - t1
        za = pair_real_ciphers(att_c, crypto_context=ctx)
        if att.ciphers:
            att.release()
        else:
            _release(att_c)
        o = _paired_projection(op, za, weights.o, ctx)
        op.release_babies(za)
        _release(za)
        h = residual_add(x, o, crypto_context=ctx)
        _release(o)
        _release(x)
        keep = list(h)
        sync()
        stage["softmax_pv_output_residual"] = time.perf_counter() - t0
        t0 = time.perf_counter()
        hr = refresh_stream(h, crypto_context=ctx, program=res_prog, value_bound=residual_bound,
                            group=group)
        _release(h)
        hr = keep = _drop_owned(hr, c_depth + 2, ctx)
        sync()
        stage["refresh_residual_2"] = time.perf_counter() - t0
        t0 = time.perf_counter()
        n2 = rmsnorm_fhe(hr, np.zeros(1), coeffs=ap.post_attention_norm, layout=lay,
                         crypto_context=ctx, slim_refresh=slim)
        m = mlp_fhe(n2.ciphers, weights.mlp, silu=ap.silu, crypto_context=ctx, operator=op)
        n2.release()
        out = residual_add(hr, m.ciphers, crypto_context=ctx)
        m.release()
        sync()
        stage["rmsnorm_mlp_residual"] = time.perf_counter() - t0
        return LayerResult(tuple(out), time.perf_counter() - t_start, stage,
                           int(out[0].state.cur_limbs))
    finally:
        _release(keep)
        op.close()


__all__ = ["DecoderLayerWeights", "LayerApproximations", "LayerResult", "decoder_layer_depth",
           "decoder_layer_fhe", "decoder_layer_refreshed_fhe", "decoder_layer_rotations",
           "normaliser_program", "refresh_stream", "refreshed_layer_depths",
           "refreshed_layer_programs", "rmsnorm_slim_program"]
