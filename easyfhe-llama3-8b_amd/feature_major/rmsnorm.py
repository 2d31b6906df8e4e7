"""Feature-major RMSNorm and residual additions on ciphertexts (reference
llama3fhe/operators/norm/rmsnorm.py:120-704).

RMSNorm of 128 tokens held as 16 feature-major ciphertexts (slot
``f * lanes + t``) evaluates ``x * p(mean_f x^2)`` with a fitted inverse
square root series p, evaluated once for all tokens:

1. ``x_c^2`` (one batched multiply-relinearise-rescale for the 16 inputs);
2. a rotate-and-add tree over the feature orbit (strides ``lanes * 2^b``,
   b < log2 D): every slot then holds its token's sum of squares;
3. "slim pack": ciphertext c keeps only feature row c (a mask that also
   carries the map onto [-1, 1] and 1/D), and the 16 rows are summed into one
   ciphertext holding all 128 token values;
4. the series on that single ciphertext (plus the map's offset, level-free);
5. each row c is masked out again and broadcast back over the feature orbit
   by the same tree with negative strides;
6. one product with the input (which, if a gamma vector is given, was first
   multiplied by it on its own spare levels).

Depth: square, pack mask, the series, extract mask, product.  An input that
arrives as ``s * x`` (the doubled values of a complex-paired refresh) is
normalised to ``x`` through the masks at no level (``input_value_scale``).

With a ``SlimRefresh`` (the reference's adaptive slim refresh,
operators/norm/rmsnorm.py:517-566) the series' output is bootstrapped when it
sits too low for the product to keep the input's level: one bootstrap of one
ciphertext for all 128 tokens, after which the norm costs the stream only the
product's level, and the slim path needs its own levels (square, pack, series
and a bootstrap input) instead of the stream's.

Every step over the 16 ciphertexts is batched: a tree step is one key switch
call whose key is read once for the batch.
"""

from __future__ import annotations

import math
import time
from dataclasses import dataclass, field

import numpy as np

from easyfhe import fhe
from easyfhe.chebyshev import chebyshev_depth, eval_chebyshev_series_cipher

from .approx import chebyshev_map
from .layout import FeatureMajorPrefillLayout


def _ctx(context):
    return getattr(context, "context", context)


def _release(values) -> None:
    for v in values or ():
        if v is not None:
            v.release()


def is_rmsn_weight(weight, *, atol: float = 0.0) -> bool:
    """True when the gamma vector is absent (QuaRot folds it into the next
    linear and stores zeros or one scalar, approx/rmsnorm.py:85-97)."""
    w = np.asarray(weight, dtype=np.float64).reshape(-1)
    if w.size <= 1:
        return w.size == 0 or abs(float(w[0])) <= atol
    return float(np.max(np.abs(w))) <= atol


def rmsnorm_rotations(layout: FeatureMajorPrefillLayout) -> tuple[int, ...]:
    """Keys of the reduction and broadcast trees (rmsnorm.py:120-131)."""
    stride = int(layout.tokens_per_cipher)
    offs = {stride * (1 << b) for b in range(int(math.log2(int(layout.hidden_dim))))}
    return tuple(sorted(offs | {-o for o in offs}))


def rmsnorm_depth(coeffs: dict, *, apply_gamma: bool = False) -> int:
    """Levels from the input to the output (gamma rides on the input's spare
    levels, so it does not add to this count)."""
    _ = apply_gamma
    return 4 + int(chebyshev_depth(coeffs["coefficients"]))


def rmsnorm_slim_refresh_depths(coeffs: dict, input_limbs: int) -> tuple[int, int]:
    """(levels the stream loses, limbs the input needs) of RMSNorm with its
    slim refresh: the stream loses the product's level only; the slim path
    spends the square, the pack mask and the series below the input and must
    still hold a bootstrap input (``input_limbs``)."""
    return 1, 2 + int(chebyshev_depth(coeffs["coefficients"])) + int(input_limbs)


@dataclass(frozen=True)
class SlimRefresh:
    """Refresh of RMSNorm's slim inverse-square-root ciphertext (reference
    operators/norm/rmsnorm.py:517-566, ``adaptive_rmsnorm_slim_refresh`` of
    schedule.py): when the series leaves it below the level at which the
    extraction lands on the stream's level, ``program`` (a full-slot
    bootstrap program returning at least that level) refreshes it, and the
    result is dropped to exactly that level.  ``value_bound`` bounds the
    series' values on [-1, 1] (the refresh divides by the power of two above
    it)."""

    program: object
    value_bound: float = 2.0


def refresh_slim(ct, crypto_context, program, bound: float):
    """One slim ciphertext refreshed: divided by the power of two S >= bound
    through the recorded scale (no level) so that its values fit the
    bootstrap's input range, bootstrapped, then multiplied by S as an integer
    (no level), so the result keeps the program's output scale.  ``ct`` is
    not consumed."""
    from easyfhe.bs import openfhe as bs

    ctx = _ctx(crypto_context)
    if not float(bound) > 0.0:
        raise ValueError("the value bound must be positive.")
    S = int(2 ** max(0, int(math.ceil(math.log2(float(bound))))))
    v = ct.deep_copy()
    v.set_scale(float(ct.state.scaling_factor) * S, 1)
    try:
        out = bs.bootstrap(v, ctx, program)
    finally:
        v.release()
    if S == 1:
        return out
    k = fhe.encode_scalar(S, int(out.state.cur_limbs), scale_degree=0, mode="integer",
                          context=ctx)
    try:
        return fhe.homo_mul_scalar(out, k, ctx)
    finally:
        out.release()
        k.release()


@dataclass
class RMSNormResult:
    ciphers: tuple
    wall_seconds: float
    stage_seconds: dict = field(default_factory=dict)
    output_limbs: int = 0

    def release(self) -> None:
        _release(self.ciphers)
        self.ciphers = ()


def _fold(cts, stride: int, steps: int, sign: int, ctx) -> list:
    """Rotate-and-add over the feature orbit, all inputs per batched call."""
    cur = list(cts)
    owned = False
    for b in range(steps):
        rot = fhe.homo_rotate_many(cur, sign * stride * (1 << b), ctx)
        nxt = fhe.homo_add_many(cur, rot, ctx)
        _release(rot)
        if owned:
            _release(cur)
        cur, owned = nxt, True
    return cur


def _row_masks(layout: FeatureMajorPrefillLayout, value: float) -> np.ndarray:
    """[cipher_count, slots]: ``value`` on feature row c's active token slots."""
    n, slots, lanes = int(layout.cipher_count), int(layout.slots), int(layout.tokens_per_cipher)
    rows = np.zeros((n, slots), dtype=np.float64)
    for c in range(n):
        act = layout.active_tokens(c)
        rows[c, c * lanes: c * lanes + act] = value
    return rows


def _mul_rows_rescale(cts, rows: np.ndarray, ctx, out_scale: float | None = None) -> list:
    """ct_i * encode(rows[i]) rescaled, every plaintext at the ciphertexts'
    level and the level's scale, or at the scale that lands the products
    exactly on ``out_scale`` (inputs of one scale)."""
    limbs = int(cts[0].state.cur_limbs)
    scale = ctx.scale_at(limbs)
    if out_scale is not None:
        scale = float(out_scale) * float(int(ctx.primes()[limbs - 1])) / float(
            cts[0].state.scaling_factor)
    pts = fhe.encode_rows_cached(ctx, rows, limbs=limbs, scale=scale, slots=ctx.max_slots)
    try:
        prods = [fhe.homo_mul_pt(c, p, ctx) for c, p in zip(cts, pts)]
    finally:
        _release(pts)
    try:
        return fhe.rescale_many(prods, ctx)
    finally:
        _release(prods)


def _align_all(cts, limbs: int, ctx) -> list:
    out = []
    for c in cts:
        if int(c.state.cur_limbs) == limbs:
            out.append(c.deep_copy())
        else:
            out.append(fhe.align_to(c, c.state.replace(cur_limbs=limbs, scaling_factor=None), ctx))
    return out


def rmsnorm_fhe(input_ciphers, weight, *, coeffs: dict, layout: FeatureMajorPrefillLayout,
                crypto_context, input_value_scale: float = 1.0,
                defer_output_scale: bool = False,
                slim_refresh: SlimRefresh | None = None) -> RMSNormResult:
    """``x * p(mean(x^2)) [* gamma]`` per token on feature-major ciphertexts
    (rmsnorm.py:353-704).  With ``slim_refresh`` the series' output is
    refreshed when it would pull the stream down (rmsnorm.py:517-566).
    Inputs are not consumed."""
    ctx = _ctx(crypto_context)
    xs = tuple(input_ciphers)
    if len(xs) != int(layout.cipher_count):
        raise ValueError(f"feature-major RMSNorm expects {layout.cipher_count} input ciphers, "
                         f"got {len(xs)}.")
    if int(layout.cipher_count) > int(layout.hidden_dim):
        raise ValueError("slim feature-major RMSNorm requires cipher_count <= hidden_dim.")
    if int(layout.slots) != int(ctx.max_slots):
        raise ValueError("feature-major RMSNorm requires layout.slots == context.max_slots.")
    if len({int(c.state.cur_limbs) for c in xs}) != 1:
        raise ValueError("RMSNorm inputs must share one level.")
    s_in = float(input_value_scale)
    if not math.isfinite(s_in) or s_in <= 0.0:
        raise ValueError(f"input_value_scale must be finite and positive, got {s_in}.")
    w = np.asarray(weight, dtype=np.float64).reshape(-1)
    apply_gamma = not is_rmsn_weight(w) and not defer_output_scale
    if apply_gamma and w.shape != (int(layout.hidden_dim),):
        raise ValueError(f"RMSNorm gamma must have width {layout.hidden_dim}, got {w.shape}.")
    coefficients = np.asarray(coeffs["coefficients"], dtype=np.float64)
    alpha, beta = chebyshev_map(coeffs["fit_interval"])
    depth = rmsnorm_depth(coeffs)
    limbs_in = int(xs[0].state.cur_limbs)
    if slim_refresh is None:
        if limbs_in < depth + 2:
            raise ValueError(f"RMSNorm needs {depth + 2} limbs, inputs have {limbs_in}.")
    else:
        from easyfhe.bs import openfhe as bs

        _, need = rmsnorm_slim_refresh_depths(coeffs, bs.input_limbs(ctx))
        if limbs_in < need:
            raise ValueError(f"RMSNorm with its slim refresh needs {need} limbs, inputs have "
                             f"{limbs_in}.")
    D = int(layout.hidden_dim)
    lanes = int(layout.tokens_per_cipher)
    steps = int(math.log2(D))
    sync = ctx.synchronize
    stage: dict[str, float] = {}
    t_start = time.perf_counter()
    tmp: list = []
    try:
        t0 = time.perf_counter()
        sq = fhe.homo_mul_relin_rescale_many(xs, xs, ctx)
        red = _fold(sq, lanes, steps, +1, ctx)
        _release(sq)
        # the slim ciphertext lands on the scale of the prime its series drops
        # first, the fixed point of the series' scale ladder
        rl = int(red[0].state.cur_limbs)
        terms = _mul_rows_rescale(red, _row_masks(layout, alpha / (D * s_in * s_in)), ctx,
                                  out_scale=float(int(ctx.primes()[rl - 2])))
        _release(red)
        slim = terms[0]
        for t in terms[1:]:
            nxt = fhe.homo_add(slim, t, ctx)
            slim.release()
            slim = nxt
        _release(terms[1:])
        sync()
        stage["mean_square_and_slim_pack"] = time.perf_counter() - t0

        t0 = time.perf_counter()
        limbs = int(slim.state.cur_limbs)
        if slim_refresh is None:
            off = fhe.encode_scalar(beta, limbs, scaling_factor=float(slim.state.scaling_factor),
                                    context=ctx)
            mapped = fhe.homo_add_scalar(slim, off, ctx)
        else:
            # the map's offset on the token slots only: the others stay at 0,
            # inside the series' interval, so the refresh sees only values in
            # its range (beta alone maps them just outside [-1, 1], where the
            # series grows fast; the reference adds it on the active slots,
            # rmsnorm.py:493-507)
            active = _row_masks(layout, 1.0).sum(axis=0) > 0.0
            off = fhe.encode_rows_cached(ctx, np.where(active, beta, 0.0)[None, :], limbs=limbs,
                                         scale=float(slim.state.scaling_factor),
                                         slots=ctx.max_slots)[0]
            mapped = fhe.homo_add_pt(slim, off, ctx)
        off.release()
        slim.release()
        poly = eval_chebyshev_series_cipher(mapped, coefficients, lower_bound=-1.0,
                                            upper_bound=1.0, crypto_context=ctx,
                                            input_is_chebyshev_mapped=True)
        mapped.release()
        sync()
        stage["rsqrt_polynomial"] = time.perf_counter() - t0
        if slim_refresh is not None:
            # the extraction lands one level below the series' output: that
            # must be the level of the stream the product takes (the input,
            # or one below once gamma is applied)
            want = limbs_in - (1 if apply_gamma else 0) + 1
            if int(poly.state.cur_limbs) < want:
                t0 = time.perf_counter()
                fresh = refresh_slim(poly, ctx, slim_refresh.program, slim_refresh.value_bound)
                poly.release()
                poly = fresh
                if int(poly.state.cur_limbs) < want:
                    raise ValueError(f"the slim refresh program returns "
                                     f"{int(poly.state.cur_limbs)} limbs; RMSNorm needs {want}.")
                if int(poly.state.cur_limbs) > want:
                    dropped = fhe.align_to(poly, poly.state.replace(cur_limbs=want,
                                                                    scaling_factor=None), ctx)
                    if dropped is not poly:
                        poly.release()
                    poly = dropped
                sync()
                stage["rsqrt_slim_bootstrap"] = time.perf_counter() - t0

        t0 = time.perf_counter()
        n = len(xs)
        sel = _mul_rows_rescale([poly] * n, _row_masks(layout, 1.0 / s_in), ctx)
        poly.release()
        bcast = _fold(sel, lanes, steps, -1, ctx)
        _release(sel)
        tmp = bcast
        if apply_gamma:
            gamma_rows = np.repeat(w, lanes)[None, :].repeat(n, axis=0)
            lifted = _mul_rows_rescale(list(xs), gamma_rows, ctx)
            tmp = bcast + lifted
            xa = _align_all(lifted, int(bcast[0].state.cur_limbs), ctx)
        else:
            xa = _align_all(xs, int(bcast[0].state.cur_limbs), ctx)
        tmp = tmp + xa
        out = fhe.homo_mul_relin_rescale_many(xa, bcast, ctx)
        sync()
        stage["scale_broadcast_and_output"] = time.perf_counter() - t0
        return RMSNormResult(tuple(out), time.perf_counter() - t_start, stage,
                             int(out[0].state.cur_limbs))
    finally:
        _release(tmp)


def match_scale(ct, limbs: int, scale: float, crypto_context):
    """``ct`` re-expressed at ``limbs`` limbs with recorded scale ``scale``:
    one integer multiple ``K = rint(scale q / s)`` on its first limbs + 1 limbs
    and a rescale by q (the prime that rescale drops), so the value changes by
    a relative ``K / (scale q / s) - 1`` (below 2^-40 for 40-bit primes).
    Costs one of ``ct``'s levels; ``ct`` is not consumed."""
    ctx = _ctx(crypto_context)
    limbs = int(limbs)
    if int(ct.state.cur_limbs) < limbs + 1:
        raise ValueError(f"matching a scale at {limbs} limbs needs {limbs + 1} limbs, "
                         f"the ciphertext has {ct.state.cur_limbs}.")
    q = float(int(ctx.primes()[limbs]))
    target = float(scale) * q
    acc = fhe.linear_combination([[ct]], [target / float(ct.state.scaling_factor)], 0.0,
                                 limbs + 1, target, 2, ctx)[0]
    try:
        out = fhe.rescale_many([acc], ctx)[0]
    finally:
        acc.release()
    out.set_scale(float(scale), 1)
    return out


def _same_scale(a: float, b: float) -> bool:
    return abs(a / b - 1.0) <= 2.0 ** -30


def residual_add(left, right, *, crypto_context) -> tuple:
    """Limb-wise sums of two feature-major streams (rmsnorm.py:244-351);
    inputs are not consumed.  Operands meet at the lower level; when their
    exact scales differ (the ladders of the polynomial steps move a stream's
    scale away from the fixed one), the higher operand is brought to the
    other's scale by match_scale on its spare level (both drop one level when
    they sit at the same level)."""
    ctx = _ctx(crypto_context)
    a, b = tuple(left), tuple(right)
    if len(a) != len(b):
        raise ValueError("residual streams differ in length.")
    out = []
    for x, y in zip(a, b):
        lx, ly = int(x.state.cur_limbs), int(y.state.cur_limbs)
        sx, sy = float(x.state.scaling_factor), float(y.state.scaling_factor)
        made = []
        if _same_scale(sx, sy):
            limbs = min(lx, ly)
            xa = x if lx == limbs else fhe.align_to(
                x, x.state.replace(cur_limbs=limbs, scaling_factor=None), ctx)
            ya = y if ly == limbs else fhe.align_to(
                y, y.state.replace(cur_limbs=limbs, scaling_factor=None), ctx)
        else:
            if lx < ly:
                x, y, lx, ly, sx, sy = y, x, ly, lx, sy, sx
            limbs = ly if lx > ly else ly - 1
            if limbs < 1:
                raise ValueError("no level left to match the residual scales.")
            ya = y if ly == limbs else fhe.align_to(
                y, y.state.replace(cur_limbs=limbs, scaling_factor=None), ctx)
            xa = match_scale(x, limbs, float(ya.state.scaling_factor), ctx)
        made = [c for c, src in ((xa, x), (ya, y)) if c is not src]
        out.append(fhe.homo_add(xa, ya, ctx))
        _release(made)
    return tuple(out)


__all__ = ["RMSNormResult", "SlimRefresh", "is_rmsn_weight", "match_scale", "refresh_slim",
           "residual_add", "rmsnorm_depth", "rmsnorm_fhe", "rmsnorm_rotations",
           "rmsnorm_slim_refresh_depths"]
