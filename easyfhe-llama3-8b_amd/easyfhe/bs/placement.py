"""Refresh placement and limb budgets of the feature-major layer schedule.

Counterpart of the caller-side rules that decide when a layer bootstraps and
how many limbs each stage receives (reference llama3fhe/schedule.py:34-111,
graph.py:780-990 and 1240-1430, operators/norm/refresh.py:70-150):

* the two residual refresh points of a decoder layer (before the input
  RMSNorm and before the post-attention RMSNorm) bootstrap the 16
  feature-major ciphertexts as 8 complex pairs;
* after a refresh, a cheap modulus drop is clamped so that the consumer still
  receives its minimum limb count (``adaptive_bootstrap_output_level_drop``);
* the minimum limb counts are fixed by the depth of what follows: 13 before
  QKV (graph.py:784-795) and the SiLU series depth plus a 6-limb suffix before
  the MLP (graph.py:1246-1259).

The series depth used for a budget is that of the evaluator which runs it.
This build evaluates Chebyshev series at the minimum depth ceil(log2(n + 1))
(``easyfhe.chebyshev``); the reference's Paterson-Stockmeyer evaluator spends
ceil(log2 k) + m levels with (k, m) from its degree table
(approx/chebyshev.py:51-120), restated in ``reference_ps_depth`` so that the
reference's own budgets can be reproduced.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Callable, Sequence

from .. import chebyshev as cheb
from .. import fhe
from . import openfhe as bs

# Paterson-Stockmeyer m per degree range (first degree, last degree, m): the
# reference's table (approx/chebyshev.py:51-76), kept as data.
_PS_M_RANGES = (
    (1, 2, 1), (3, 11, 2), (12, 13, 3), (14, 17, 2), (18, 55, 3), (56, 59, 4),
    (60, 76, 3), (77, 239, 4), (240, 247, 5), (248, 284, 4), (285, 991, 5),
    (992, 1007, 6), (1008, 1083, 5), (1084, 2015, 6), (2016, 2031, 7), (2032, 2204, 6),
)


def reference_ps_degrees(n: int) -> tuple[int, int]:
    """(k, m) of the reference's Paterson-Stockmeyer split for degree n <= 2204
    (approx/chebyshev.py:79-89): m from the table, k = floor(n / (2^m - 1)) + 1."""
    n = int(n)
    if n <= 0:
        raise ValueError("degree must be positive")
    for lo, hi, m in _PS_M_RANGES:
        if lo <= n <= hi:
            return n // ((1 << m) - 1) + 1, m
    raise ValueError("degree above the tabulated range (2204)")


def reference_ps_depth(coefficients: Sequence[float]) -> int:
    """ceil(log2 k) + m (approx/chebyshev.py:113-124); 0 for a constant."""
    n = cheb.chebyshev_degree(coefficients)
    if n <= 0:
        return 0
    k, m = reference_ps_degrees(n)
    return math.ceil(math.log2(k)) + m


def series_depth(coefficients: Sequence[float]) -> int:
    """Depth of this build's evaluator (ceil(log2(n + 1)))."""
    return cheb.chebyshev_depth(coefficients)


@dataclass(frozen=True)
class RefreshSchedule:
    """The refresh-budget fields of the reference's LayerSchedule
    (schedule.py:34-111) with its production defaults."""

    bootstrap_post_levels: int = 19
    bootstrap_log_slots: int = 15
    bootstrap_level_budget: tuple[int, int] = (4, 4)
    residual_bootstrap_level_drop: int = 0
    residual_bootstrap_iterations: int = 1
    residual_bootstrap_precision: int = 14
    pair_residual_bootstrap: bool = True
    pairfm_post_refresh_input_limbs: int | None = 6
    adaptive_rmsnorm_slim_refresh: bool = True
    fuse_silu_domain_map: bool = True
    mlp_input_level_drop: int = 0
    #: margin above the 13-limb attention budget (LLAMA_FHE_ATTN_EXTRA_LIMBS)
    attention_extra_limbs: int = 0
    #: gate(1) + up-mul(1) + down(1) + residual match + a two-limb floor
    #: (LLAMA_FHE_MLP_SUFFIX_LIMBS)
    mlp_suffix_limbs: int = 6

    def __post_init__(self):
        if int(self.mlp_suffix_limbs) < 3:
            raise ValueError("mlp_suffix_limbs must be at least 3")
        if int(self.residual_bootstrap_level_drop) < 0:
            raise ValueError("residual_bootstrap_level_drop must be non-negative")


#: Score stream before the pre-exp checkpoint: QKV 1 + K adapter 4 + QK 2 +
#: score preprocessing 1 + a 2-limb bootstrap floor (graph.py:784-790).
ATTENTION_SCORE_LIMBS = 10
#: The value stream is never refreshed inside attention and must reach the
#: PairFM pairing at >= 6 limbs: 3 more limbs than the score stream needs
#: (graph.py:786-795).
ATTENTION_VALUE_MARGIN = 3


def attention_input_min_limbs(schedule: RefreshSchedule | None = None) -> int:
    """Limbs the input RMSNorm must leave for QKV -> attention (13 by default)."""
    s = schedule or RefreshSchedule()
    return ATTENTION_SCORE_LIMBS + ATTENTION_VALUE_MARGIN + int(s.attention_extra_limbs)


def mlp_input_min_limbs(silu_coefficients: Sequence[float],
                        schedule: RefreshSchedule | None = None,
                        depth: Callable[[Sequence[float]], int] = series_depth) -> int:
    """Limbs the post-attention RMSNorm must leave for the MLP: the SiLU
    series depth + the suffix, one less when the SiLU domain map is fused
    into the RMSNorm output scale (graph.py:1246-1259)."""
    s = schedule or RefreshSchedule()
    return int(depth(silu_coefficients)) + int(s.mlp_suffix_limbs) - int(bool(s.fuse_silu_domain_map))


def adaptive_bootstrap_output_level_drop(*, current_limbs: int, requested_level_drop: int,
                                         rmsnorm_depth: int,
                                         minimum_output_limbs: int | None) -> int:
    """The post-bootstrap modulus drop, clamped so that an RMSNorm of depth
    ``rmsnorm_depth`` still leaves ``minimum_output_limbs`` (refresh.py:70-93)."""
    current_limbs, requested = int(current_limbs), int(requested_level_drop)
    if requested < 0:
        raise ValueError("requested_level_drop must be non-negative")
    if int(rmsnorm_depth) < 0:
        raise ValueError("rmsnorm_depth must be non-negative")
    if minimum_output_limbs is None:
        return requested
    if int(minimum_output_limbs) <= 1:
        raise ValueError("minimum_output_limbs must exceed one")
    safe = max(0, current_limbs - int(rmsnorm_depth) - int(minimum_output_limbs))
    return min(requested, safe)


def refresh_bootstraps(cipher_count: int, schedule: RefreshSchedule | None = None) -> int:
    """Bootstraps of one residual refresh point: pairs when paired."""
    s = schedule or RefreshSchedule()
    n = int(cipher_count)
    if s.pair_residual_bootstrap:
        if n % 2:
            raise ValueError("complex-paired refresh requires an even stream")
        return n // 2
    return n


def residual_refresh_bootstraps_per_layer(cipher_count: int = 16,
                                          schedule: RefreshSchedule | None = None) -> int:
    """The two residual refresh points of a steady layer (input RMSNorm,
    graph.py:797-826; post-attention RMSNorm, graph.py:1260-1286)."""
    return 2 * refresh_bootstraps(cipher_count, schedule)


def _ctx(context):
    return getattr(context, "context", context)


def _half(ct, ctx):
    """0.5 * ct as one scalar product and a rescale (refresh.py:20-31)."""
    enc = fhe.encode_scalar(0.5, int(ct.state.cur_limbs), scale_degree=1,
                            scaling_factor=float(ct.state.scaling_factor), context=ctx)
    return fhe.homo_mul_scalar_rescale(ct, enc, ctx)


def refresh_ciphers(ciphers, context, program: bs.BootstrapProgram, *, iterations: int = 1,
                    precision_bits: int = 14, halve: bool = False) -> list:
    """Refresh a real feature-major stream by complex-paired bootstraps
    (refresh.py:96-150).  ``bootstrap_pair`` returns 2a and 2b with the factor
    taken into the recorded scale; ``halve`` instead multiplies by 0.5 and
    rescales, as the reference does (one more level)."""
    ctx = _ctx(context)
    cts = list(ciphers)
    if len(cts) % 2:
        raise ValueError("complex-paired refresh requires an even stream")
    out = []
    for i in range(0, len(cts), 2):
        a, b = cts[i], cts[i + 1]
        if int(iterations) == 1:
            ra, rb = bs.bootstrap_pair(a, b, ctx, program)
        else:
            packed = fhe.homo_add(a, fhe.homo_mul_i(b, ctx), ctx)
            value = bs.bootstrap_iterated(packed, ctx, program, iterations=int(iterations),
                                          precision_bits=int(precision_bits))
            conj = fhe.homo_rotate(value, 2 * ctx.N - 1, ctx)
            ra = fhe.homo_add(value, conj, ctx)
            rb = fhe.homo_mul_i(fhe.homo_sub(conj, value, ctx), ctx)
            for t in (ra, rb):
                t.set_scale(2.0 * float(t.state.scaling_factor), 1)
        if halve:
            for t in (ra, rb):
                t.set_scale(0.5 * float(t.state.scaling_factor), 1)
            ra, rb = _half(ra, ctx), _half(rb, ctx)
        out.extend((ra, rb))
    return out


@dataclass
class RefreshResult:
    ciphers: list
    level_drops: list
    output_limbs: tuple


def refresh_and_drop(ciphers, context, program: bs.BootstrapProgram, *,
                     schedule: RefreshSchedule | None = None, rmsnorm_depth: int = 0,
                     minimum_output_limbs: int | None = None) -> RefreshResult:
    """A residual refresh point: paired (or single) bootstraps, then the
    clamped modulus drop of each refreshed ciphertext (refresh.py:207-242)."""
    s = schedule or RefreshSchedule()
    ctx = _ctx(context)
    cts = list(ciphers)
    if s.pair_residual_bootstrap:
        refreshed = refresh_ciphers(cts, ctx, program,
                                    iterations=s.residual_bootstrap_iterations,
                                    precision_bits=s.residual_bootstrap_precision)
    else:
        refreshed = [bs.bootstrap_iterated(c, ctx, program,
                                           iterations=s.residual_bootstrap_iterations,
                                           precision_bits=s.residual_bootstrap_precision)
                     for c in cts]
    out, drops = [], []
    for ct in refreshed:
        limbs = int(ct.state.cur_limbs)
        drop = adaptive_bootstrap_output_level_drop(
            current_limbs=limbs, requested_level_drop=s.residual_bootstrap_level_drop,
            rmsnorm_depth=rmsnorm_depth, minimum_output_limbs=minimum_output_limbs)
        drops.append(drop)
        if drop:
            ct = fhe.align_to(ct, ct.state.replace(cur_limbs=limbs - drop, scaling_factor=None), ctx)
        out.append(ct)
    return RefreshResult(out, drops, tuple(sorted({int(c.state.cur_limbs) for c in out})))


__all__ = [
    "ATTENTION_SCORE_LIMBS", "ATTENTION_VALUE_MARGIN", "RefreshResult", "RefreshSchedule",
    "adaptive_bootstrap_output_level_drop", "attention_input_min_limbs", "mlp_input_min_limbs",
    "reference_ps_degrees", "reference_ps_depth", "refresh_and_drop", "refresh_bootstraps",
    "refresh_ciphers", "residual_refresh_bootstraps_per_layer", "series_depth",
]
