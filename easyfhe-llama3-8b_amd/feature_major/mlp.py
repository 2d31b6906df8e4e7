"""Feature-major SwiGLU MLP on ciphertexts (reference
llama3fhe/operators/linear/mlp.py:32-1126).

``down @ (silu(gate @ x) * (up @ x))`` for 128 tokens in 16 feature-major
ciphertexts.  The intermediate width (14336 for Llama-3-8B) is cut into pages
of the hidden width D; every page is one D x D square of each projection
(zero rows / columns past the intermediate width), so the BSGS linear engine
runs unchanged.  Per page:

1. adjacent token ciphertexts are paired as ``x + i y`` (the 8 complex inputs
   are made once for all pages): a real linear acts on both halves, so each
   projection runs on 8 ciphertexts instead of 16;
2. ``(alpha / 2) G_p z`` and ``(1 / 2) U_p z`` (gate pre-scaled by the SiLU
   series' domain map, whose offset is added as a constant: the series then
   starts at its mapped input without a level of its own); the gate lands
   exactly on the scale of the prime the series drops first, which keeps
   every scale of the series' ladder at the primes;
3. the conjugation split gives the 16 real gate and up streams (its factor 2
   cancels the weights' 1/2);
4. the SiLU series on the 16 gate streams as one batched evaluation, times the
   up streams;
5. re-pairing and ``(1 / 2) Dn_p h``; the pages' down outputs are summed;

and one final split returns the 16 real output streams.  Depth: gate/up
linear, the series, the product, the down linear.
"""

from __future__ import annotations

import time
from dataclasses import dataclass, field

import numpy as np

from easyfhe import fhe
from easyfhe.chebyshev import chebyshev_depth, eval_chebyshev_series_many

from .approx import chebyshev_map
from .complex import pair_real_ciphers, split_complex_ciphers_twice
from .layout import FeatureMajorPrefillLayout
from .linear import LinearOperator, LinearOperatorConfig, LinearWeight, linear_rotations


def _ctx(context):
    return getattr(context, "context", context)


def _release(values) -> None:
    for v in values or ():
        if v is not None:
            v.release()


@dataclass(frozen=True)
class FeatureMajorMLPLayout:
    """Paged intermediate around a canonical feature-major boundary
    (mlp.py:32-133)."""

    canonical: FeatureMajorPrefillLayout
    intermediate_width: int = 14336

    def __post_init__(self) -> None:
        if int(self.intermediate_width) <= 0:
            raise ValueError(f"intermediate_width must be positive, got "
                             f"{self.intermediate_width}.")

    @property
    def page_width(self) -> int:
        return int(self.canonical.hidden_dim)

    @property
    def feature_page_count(self) -> int:
        return -(-int(self.intermediate_width) // self.page_width)

    @property
    def paired_token_cipher_count(self) -> int:
        return -(-int(self.canonical.cipher_count) // 2)

    def active_width(self, page: int) -> int:
        page = int(page)
        if not 0 <= page < self.feature_page_count:
            raise IndexError(f"feature_page={page} is outside [0, {self.feature_page_count}).")
        return min(self.page_width, int(self.intermediate_width) - page * self.page_width)


def mlp_rotations(layout: FeatureMajorPrefillLayout,
                  operator_config: LinearOperatorConfig | None = None) -> tuple[int, ...]:
    """The linear schedule's keys plus the conjugation of the splits."""
    return linear_rotations(dimension=int(layout.hidden_dim),
                            token_lanes=int(layout.tokens_per_cipher),
                            slots=int(layout.slots), include_conjugation=True,
                            operator_config=operator_config)


def mlp_depth(silu: dict) -> int:
    return 3 + int(chebyshev_depth(silu["coefficients"]))


class MLPWeights:
    """Gate, up and down projections resident on the device, one square
    LinearWeight per page and projection, each halved (the conjugation split
    after it doubles) and the gate pre-multiplied by the SiLU domain map's
    alpha."""

    def __init__(self, gate, up, down, *, silu: dict, layout: FeatureMajorMLPLayout,
                 context, dtype=np.float64):
        ctx = _ctx(context)
        gate = np.asarray(gate, dtype=np.float64)
        up = np.asarray(up, dtype=np.float64)
        down = np.asarray(down, dtype=np.float64)
        D, I = int(layout.page_width), int(layout.intermediate_width)
        if gate.shape != (I, D) or up.shape != (I, D):
            raise ValueError(f"gate/up must have shape {(I, D)}, got {gate.shape}, {up.shape}.")
        if down.shape != (D, I):
            raise ValueError(f"down must have shape {(D, I)}, got {down.shape}.")
        alpha, beta = chebyshev_map(silu["fit_interval"])
        self.alpha, self.beta = alpha, beta
        self.layout = layout
        self.gate, self.up, self.down = [], [], []
        try:
            for p in range(layout.feature_page_count):
                act, s = layout.active_width(p), p * D
                g = np.zeros((D, D))
                u = np.zeros((D, D))
                d = np.zeros((D, D))
                g[:act] = (0.5 * alpha) * gate[s: s + act]
                u[:act] = 0.5 * up[s: s + act]
                d[:, :act] = 0.5 * down[:, s: s + act]
                self.gate.append(LinearWeight(g, dtype=dtype, context=ctx))
                self.up.append(LinearWeight(u, dtype=dtype, context=ctx))
                self.down.append(LinearWeight(d, dtype=dtype, context=ctx))
        except Exception:
            self.close()
            raise

    def close(self) -> None:
        for w in self.gate + self.up + self.down:
            w.close()
        self.gate, self.up, self.down = [], [], []

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


@dataclass
class MLPResult:
    ciphers: tuple
    wall_seconds: float
    stage_seconds: dict = field(default_factory=dict)
    output_limbs: int = 0

    def release(self) -> None:
        _release(self.ciphers)
        self.ciphers = ()


def _add_const(cts, value: float, ctx) -> list:
    limbs = int(cts[0].state.cur_limbs)
    out = []
    for c in cts:
        enc = fhe.encode_scalar(float(value), limbs,
                                scaling_factor=float(c.state.scaling_factor), context=ctx)
        out.append(fhe.homo_add_scalar(c, enc, ctx))
        enc.release()
    return out


def mlp_fhe(input_ciphers, weights: MLPWeights, *, silu: dict, crypto_context,
            operator: LinearOperator | None = None) -> MLPResult:
    """SwiGLU MLP of a real feature-major stream (mlp.py:524-1126); inputs
    are not consumed."""
    ctx = _ctx(crypto_context)
    lay = weights.layout
    xs = tuple(input_ciphers)
    n = int(lay.canonical.cipher_count)
    if len(xs) != n:
        raise ValueError(f"MLP expects {n} input ciphers, got {len(xs)}.")
    if n % 2:
        raise ValueError("the paired MLP needs an even number of token ciphertexts.")
    if len({int(c.state.cur_limbs) for c in xs}) != 1:
        raise ValueError("MLP inputs must share one level.")
    depth = mlp_depth(silu)
    if int(xs[0].state.cur_limbs) < depth + 1:
        raise ValueError(f"MLP needs {depth + 1} limbs, inputs have {xs[0].state.cur_limbs}.")
    own_op = operator is None
    op = operator or LinearOperator(context=ctx, token_lanes=int(lay.canonical.tokens_per_cipher),
                                    config=LinearOperatorConfig(timed_stages=False))
    coeffs = np.asarray(silu["coefficients"], dtype=np.float64)
    stage = {"pair": 0.0, "gate_up": 0.0, "split": 0.0, "silu": 0.0, "product": 0.0,
             "down": 0.0, "output_split": 0.0}
    sync = ctx.synchronize
    t_start = time.perf_counter()
    acc: list = []
    z: tuple = ()
    try:
        t0 = time.perf_counter()
        z = pair_real_ciphers(xs, crypto_context=ctx)
        sync()
        stage["pair"] = time.perf_counter() - t0
        for p in range(lay.feature_page_count):
            t0 = time.perf_counter()
            zl = int(z[0].state.cur_limbs)
            g, _ = op.apply(z, weights.gate[p],
                            output_scale=float(int(ctx.primes()[zl - 2])))
            u, _ = op.apply(z, weights.up[p])
            sync()
            stage["gate_up"] += time.perf_counter() - t0
            t0 = time.perf_counter()
            gr = split_complex_ciphers_twice(g, crypto_context=ctx)
            ur = split_complex_ciphers_twice(u, crypto_context=ctx)
            _release(g)
            _release(u)
            gm = _add_const(gr, weights.beta, ctx)
            _release(gr)
            sync()
            stage["split"] += time.perf_counter() - t0
            t0 = time.perf_counter()
            act = eval_chebyshev_series_many(gm, coeffs, lower_bound=-1.0, upper_bound=1.0,
                                             crypto_context=ctx, input_is_chebyshev_mapped=True)
            _release(gm)
            sync()
            stage["silu"] += time.perf_counter() - t0
            t0 = time.perf_counter()
            limbs = int(act[0].state.cur_limbs)
            ua = [fhe.align_to(c, c.state.replace(cur_limbs=limbs, scaling_factor=None), ctx)
                  for c in ur]
            h = fhe.homo_mul_relin_rescale_many(act, ua, ctx)
            _release(act)
            _release([a for a, b in zip(ua, ur) if a is not b])
            _release(ur)
            hz = pair_real_ciphers(h, crypto_context=ctx)
            _release(h)
            sync()
            stage["product"] += time.perf_counter() - t0
            t0 = time.perf_counter()
            y, _ = op.apply(hz, weights.down[p])
            op.release_babies(hz)
            _release(hz)
            if not acc:
                acc = list(y)
            else:
                summed = fhe.homo_add_many(acc, y, ctx)
                _release(acc)
                _release(y)
                acc = summed
            sync()
            stage["down"] += time.perf_counter() - t0
        t0 = time.perf_counter()
        out = split_complex_ciphers_twice(acc, crypto_context=ctx)
        sync()
        stage["output_split"] = time.perf_counter() - t0
        return MLPResult(tuple(out), time.perf_counter() - t_start, stage,
                         int(out[0].state.cur_limbs))
    finally:
        _release(acc)
        _release(z)
        if own_op:
            op.close()


__all__ = ["FeatureMajorMLPLayout", "MLPResult", "MLPWeights", "mlp_depth", "mlp_fhe",
           "mlp_rotations"]
