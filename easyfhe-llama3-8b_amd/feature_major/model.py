"""Encrypted Llama-3 prefill over feature-major ciphertexts: the client's
embedding lookup and exact final RMSNorm + LM head in the clear (reference
application/client.py:39-101), per-layer approximation entries selected from
calibrated ranges (application/approx_config.py:38-60, approx/rmsnorm.py,
approx/softmax.py), and the layer loop with its refreshes between encrypted
layers (model.py:157-220, runner.py:475-640).

Ranges.  Each layer's nonlinearities are series fitted on intervals: the
mean square feeding each RMSNorm, the gate pre-activations, the scores, and
the magnitude of the residual stream the refreshes bring into the bootstrap's
input range.  The reference ships these per layer as fitted artifacts; here
``layer_ranges`` measures them on a calibration sequence in plaintext and
``approximations_for`` widens them by fixed margins.
"""

from __future__ import annotations

import time
from dataclasses import dataclass, field
from typing import Callable, Sequence

import numpy as np

from .approx import rsqrt_entry, silu_entry
from .attention import SoftmaxConfig
from .layer import DecoderLayerWeights, LayerApproximations, decoder_layer_refreshed_fhe

RMS_NORM_EPS = 1e-5


def embed_tokens(token_ids, table) -> np.ndarray:
    """Rows of the embedding table for the token ids (the client's lookup
    before encryption)."""
    ids = np.asarray(token_ids, dtype=np.int64)
    table = np.asarray(table)
    if ids.ndim != 1 or ids.size == 0:
        raise ValueError("token ids must be a non-empty vector.")
    if ids.min() < 0 or ids.max() >= table.shape[0]:
        raise IndexError(f"token id outside [0, {table.shape[0]}).")
    return np.asarray(table[ids], dtype=np.float64)


def final_logits(hidden, *, norm_weight, lm_head, eps: float = RMS_NORM_EPS,
                 token_index: int = -1) -> np.ndarray:
    """Exact final RMSNorm of one token's hidden state and the LM head,
    computed by the client after decryption (reference client.py:60-101; here
    in fp64 throughout)."""
    hidden = np.asarray(hidden, dtype=np.float64)
    if hidden.ndim != 2 or hidden.shape[0] == 0:
        raise ValueError(f"final hidden state must be a non-empty [token, hidden] matrix, "
                         f"got {hidden.shape}.")
    head = np.asarray(lm_head)
    if head.ndim != 2 or head.shape[1] != hidden.shape[1]:
        raise ValueError(f"lm_head must be [vocab, {hidden.shape[1]}], got {head.shape}.")
    t = int(token_index)
    if t < 0:
        t += hidden.shape[0]
    if not 0 <= t < hidden.shape[0]:
        raise IndexError(f"token_index={token_index} is outside [0, {hidden.shape[0]}).")
    last = hidden[t]
    normed = last / np.sqrt(np.mean(last * last) + float(eps)) * np.asarray(norm_weight,
                                                                             dtype=np.float64)
    return head.astype(np.float64, copy=False) @ normed


@dataclass(frozen=True)
class LayerRanges:
    """Plaintext ranges of one layer's nonlinearity inputs on calibration data:
    mean squares of the rows feeding the two RMSNorms, the largest
    magnitudes of the residual stream at the two refresh points and of the
    gate pre-activations, and the extreme valid (causal) scores."""

    input_mean_square: tuple[float, float]
    post_attention_mean_square: tuple[float, float]
    residual_abs_max: float
    gate_abs_max: float
    score_max: float
    score_min: float


def layer_ranges(x, h1, gate, scores) -> LayerRanges:
    """Ranges from a plaintext pass: ``x`` the layer input [T, D], ``h1`` the
    stream after attention's residual add, ``gate`` the gate projection
    [T, I], ``scores`` [H, T, T] scaled scores (the causal part is read)."""
    x, h1 = np.asarray(x, dtype=np.float64), np.asarray(h1, dtype=np.float64)
    ms1, ms2 = np.mean(x * x, axis=-1), np.mean(h1 * h1, axis=-1)
    s = np.asarray(scores, dtype=np.float64)
    valid = np.broadcast_to(np.tril(np.ones(s.shape[-2:], dtype=bool)), s.shape)
    return LayerRanges((float(ms1.min()), float(ms1.max())), (float(ms2.min()), float(ms2.max())),
                       float(max(np.abs(x).max(), np.abs(h1).max())),
                       float(np.abs(np.asarray(gate)).max()), float(s[valid].max()),
                       float(s[valid].min()))


@dataclass(frozen=True)
class RangeMargins:
    """How far the fitted intervals reach beyond the calibrated ranges: the
    RMSNorm intervals by a factor on each side, the residual bound by a
    factor, SiLU and the score interval by fixed amounts."""

    mean_square_factor: float = 4.0
    residual_factor: float = 2.0
    gate_margin: float = 4.0
    score_margin: float = 1.0
    score_span: float = 20.0
    rmsnorm_degree: int = 63
    silu_degree: int = 63
    softmax_rounds: int = 3
    exp_degree: int = 7
    first_inverse_degree: int = 31
    inverse_degree: int = 47


def approximations_for(r: LayerRanges, m: RangeMargins = RangeMargins()
                       ) -> tuple[LayerApproximations, float]:
    """The layer's series entries and residual bound from its ranges.  The
    softmax's shift sits above the largest score, rounded up to an integer
    (the exp series runs on (s - shift) / 2^rounds and the Algorithm-2 rounds
    diverge once a short row's exp exceeds one); the score interval keeps a
    fixed span, since its width sets the first normalising inverse's range
    (exp(-2 span / 2^rounds) to 1), which its series resolves only up to a
    ratio of a few hundred.  Scores below the interval only meet the exp
    series' gentle extrapolation."""
    f = float(m.mean_square_factor)

    def norm(lo_hi):
        lo, hi = lo_hi
        return rsqrt_entry(lo / f, hi * f, int(m.rmsnorm_degree))

    g = float(np.ceil(r.gate_abs_max + m.gate_margin))
    shift = float(np.ceil(max(r.score_max, 0.0) + m.score_margin))
    bound = float(m.score_span) - shift
    if bound < 2.0:
        raise ValueError(f"scores up to {r.score_max:.2f} leave no room in a span of "
                         f"{m.score_span}.")
    sm = SoftmaxConfig(rounds=int(m.softmax_rounds), shift=shift, bound=bound,
                       exp_degree=int(m.exp_degree),
                       first_inverse_degree=int(m.first_inverse_degree),
                       inverse_degree=int(m.inverse_degree))
    ap = LayerApproximations(norm(r.input_mean_square), norm(r.post_attention_mean_square),
                             silu_entry(-g, g, int(m.silu_degree)), sm)
    return ap, float(r.residual_abs_max) * float(m.residual_factor)


@dataclass
class PrefillResult:
    ciphers: tuple
    layer_seconds: list = field(default_factory=list)
    stage_seconds: list = field(default_factory=list)
    wall_seconds: float = 0.0

    def release(self) -> None:
        for c in self.ciphers:
            if c is not None:
                c.release()
        self.ciphers = ()


def prefill_fhe(input_ciphers, layers: Sequence[DecoderLayerWeights], *, crypto_context,
                program, residual_bounds: Sequence[float], residual_program=None,
                normaliser_program=None, rmsnorm_program=None,
                group: int = 8, rope_theta: float = 500000.0,
                on_layer: Callable[[int, float], None] | None = None) -> PrefillResult:
    """The encrypted layers in order, each refreshed as it begins (reference
    model.py:171 Llama3Model.forward).  ``program`` and ``residual_program``
    are the score and residual bootstrap programs of
    ``decoder_layer_refreshed_fhe``, and ``normaliser_program`` /
    ``rmsnorm_program`` its optional softmax-normaliser and slim RMSNorm
    refreshes (the reference's lambda and slim refreshes, which its chain
    needs); ``residual_bounds[i]`` bounds layer i's residual stream; the
    inputs are not consumed.  ``on_layer(i, s)`` is called after each layer
    with its wall time."""
    if len(residual_bounds) != len(layers):
        raise ValueError("one residual bound per layer.")
    if not layers:
        raise ValueError("no layers.")
    out = PrefillResult(())
    cur, owned = list(input_ciphers), False
    t0 = time.perf_counter()
    try:
        for i, w in enumerate(layers):
            res = decoder_layer_refreshed_fhe(cur, w, crypto_context=crypto_context,
                                              program=program, residual_program=residual_program,
                                              residual_bound=float(residual_bounds[i]),
                                              group=group, rope_theta=rope_theta,
                                              normaliser_program=normaliser_program,
                                              rmsnorm_program=rmsnorm_program)
            if owned:
                for c in cur:
                    c.release()
            cur, owned = list(res.ciphers), True
            out.layer_seconds.append(res.wall_seconds)
            out.stage_seconds.append(dict(res.stage_seconds))
            if on_layer is not None:
                on_layer(i, res.wall_seconds)
    except Exception:
        if owned:
            for c in cur:
                c.release()
        raise
    out.ciphers = tuple(cur)
    out.wall_seconds = time.perf_counter() - t0
    return out


__all__ = ["LayerRanges", "PrefillResult", "RangeMargins", "approximations_for", "embed_tokens",
           "final_logits", "layer_ranges", "prefill_fhe"]
