"""Polynomial approximations of the layer's nonlinearities.

The reference ships fitted Chebyshev series per layer in
``assets/polynomials/*.json`` (entries ``{"coefficients": [...],
"fit_interval": [lo, hi]}``, read by approx/rmsnorm.py:54-82 and
approx/silu.py).  This backend fits its own series of the same form:
Chebyshev interpolation at the degree + 1 Chebyshev points of the first kind
on [lo, hi], coefficients in the convention ``c_0/2 + sum_i c_i T_i`` that the
encrypted evaluator and the reference's direct evaluator use.

* inverse square root for RMSNorm, ``1/sqrt(v + eps)`` of the token variance;
* SiLU ``g * sigmoid(g)`` of the gate projection.

The interval and degree are parameters: the reference fits them per layer to
the observed activation ranges; the defaults here cover activations of unit
variance (the synthetic N(0, 1) layer inputs) with margin.
"""

from __future__ import annotations

import numpy as np

from easyfhe.chebyshev import chebyshev_coefficients

RMSNORM_EPS = 1e-5


def fit_entry(func, lo: float, hi: float, degree: int) -> dict:
    """``{"coefficients", "fit_interval", "degree", "max_fit_error"}`` of the
    degree-``degree`` interpolant of ``func`` on [lo, hi]."""
    lo, hi, degree = float(lo), float(hi), int(degree)
    if not hi > lo:
        raise ValueError(f"empty fit interval [{lo}, {hi}].")
    if degree < 1:
        raise ValueError("degree must be >= 1.")
    c = np.asarray(chebyshev_coefficients(func, lo, hi, degree), dtype=np.float64)
    grid = np.linspace(lo, hi, 4097)
    y = (2.0 * grid - (lo + hi)) / (hi - lo)
    approx = np.polynomial.chebyshev.chebval(y, np.concatenate(([c[0] / 2.0], c[1:])))
    err = float(np.max(np.abs(approx - func(grid))))
    return {"coefficients": [float(v) for v in c], "fit_interval": [lo, hi], "degree": degree,
            "max_fit_error": err}


def rsqrt_entry(lo: float = 0.25, hi: float = 4.0, degree: int = 31,
                eps: float = RMSNORM_EPS) -> dict:
    """Series of ``1/sqrt(v + eps)`` on [lo, hi] (the stability epsilon is part
    of the target, as in the reference's fitted entries)."""
    if lo + eps <= 0.0:
        raise ValueError("the rsqrt interval must stay above -eps.")
    return fit_entry(lambda v: 1.0 / np.sqrt(v + eps), lo, hi, degree)


def silu_entry(lo: float = -12.0, hi: float = 12.0, degree: int = 63) -> dict:
    """Series of ``g / (1 + exp(-g))`` on [lo, hi]."""
    return fit_entry(lambda g: g / (1.0 + np.exp(-g)), lo, hi, degree)


def exp_entry(lo: float, hi: float = 0.0, degree: int = 15) -> dict:
    """Series of ``exp(x)`` on [lo, hi] (the shifted, 2^-k scaled scores of
    the softmax)."""
    return fit_entry(np.exp, lo, hi, degree)


def inverse_entry(lo: float, hi: float = 1.0, degree: int = 63) -> dict:
    """Series of ``1/v`` on [lo, hi] (the softmax rounds' normalised row
    sums of squares)."""
    if lo <= 0.0:
        raise ValueError("the inverse needs an interval above zero.")
    return fit_entry(lambda v: 1.0 / v, lo, hi, degree)


def chebyshev_map(fit_interval) -> tuple[float, float]:
    """(alpha, beta) of the affine map v -> alpha v + beta onto [-1, 1]
    (operators/norm/rmsnorm.py:401-402)."""
    lo, hi = (float(v) for v in fit_interval)
    alpha = 2.0 / (hi - lo)
    return alpha, -1.0 - lo * alpha


def entry_depth(entry: dict) -> int:
    """Levels the encrypted evaluator spends on an input already in [-1, 1]."""
    from easyfhe.chebyshev import chebyshev_depth

    return int(chebyshev_depth(entry["coefficients"]))


__all__ = ["RMSNORM_EPS", "chebyshev_map", "entry_depth", "exp_entry", "fit_entry",
           "inverse_entry", "rsqrt_entry", "silu_entry"]
