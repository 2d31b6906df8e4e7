"""Chebyshev series on ciphertexts with exact scale management.

Counterpart of the reference's encrypted polynomial evaluator
``eval_chebyshev_series_cipher`` (reference
llama3fhe/operators/nonlinear/polynomial.py:364-412) and of the coefficient
fit it consumes (reference llama3fhe/approx/chebyshev.py:22-48), designed
for this backend:

* **Scale ladder.**  Every intermediate ciphertext sits on a level j of a
  ladder: limbs ``limbs[j]`` and a scale ``scale[j]`` with
  ``scale[j+1] = scale[j]^2 / (product of the primes dropped between j and
  j+1)``.  Two ciphertexts on one level multiply and rescale onto the next
  level exactly, and every constant is encoded with the scale that lands
  its product on a ladder level.  Additions therefore never combine
  different scales: the usual fixed-scale drift (primes are only within
  about 2^-18 of 2^dcrt_bits) does not enter the result.  A level may drop
  one prime or several (``step``), so a 40-bit chain can run a polynomial at
  a working scale near 2^80 (what bootstrapping's EvalMod needs).
* **Baby-step giant-step recursion.**  ``p = q T_d + r`` with ``d = k 2^j``
  (``T_i = 2 T_d T_(i-d) - T_(2d-i)`` for ``d < i < 2d``), leaves of degree
  below k evaluated as one scaled linear combination of the baby basis
  ``T_1 .. T_(k-1)``.  The same recursion runs symbolically to pick k and to
  report the depth.

Coefficients follow the reference convention ``c_0 / 2 + sum c_i T_i``.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Callable, Sequence

import numpy as np

from . import fhe

# ---------------------------------------------------------------------------
# plaintext coefficient algebra
# ---------------------------------------------------------------------------


def chebyshev_coefficients(func: Callable, a: float, b: float, degree: int) -> np.ndarray:
    """Interpolation coefficients of ``func`` on [a, b] at the degree + 1
    Chebyshev nodes, reference convention (the constant term is c_0 / 2).
    Same quantity as the reference's eval_chebyshev_coefficients
    (approx/chebyshev.py:22-48): a discrete cosine transform of the samples."""
    if degree <= 0:
        raise ValueError("degree must be positive")
    n = degree + 1
    theta = (np.arange(n) + 0.5) * math.pi / n
    x = np.cos(theta) * (0.5 * (b - a)) + 0.5 * (b + a)
    fx = np.array([func(float(v)) for v in x], dtype=np.float64)
    basis = np.cos(np.outer(np.arange(n), theta))
    return (2.0 / n) * basis @ fx


def chebyshev_degree(coefficients: Sequence[float]) -> int:
    c = np.asarray(coefficients, dtype=np.float64)
    nz = np.nonzero(c)[0]
    return int(nz[-1]) if nz.size else 0


def evaluate_direct(x, coefficients: Sequence[float], a: float = -1.0, b: float = 1.0):
    """fp64 value of the series at plaintext points (Clenshaw recurrence)."""
    c = np.asarray(coefficients, dtype=np.float64)
    y = (2.0 * np.asarray(x, dtype=np.float64) - (a + b)) / (b - a)
    b1 = np.zeros_like(y)
    b2 = np.zeros_like(y)
    for ck in c[:0:-1]:
        b1, b2 = 2.0 * y * b1 - b2 + ck, b1
    return y * b1 - b2 + 0.5 * c[0]


def divide_by_t(c: np.ndarray, d: int) -> tuple[np.ndarray, np.ndarray]:
    """Full-convention series ``c`` (p = sum c_i T_i) of degree n with
    d <= n < 2d as ``q T_d + r``; deg r < d."""
    n = len(c) - 1
    q = np.zeros(n - d + 1)
    r = np.array(c[:d], dtype=np.float64)
    q[0] = c[d]
    for i in range(d + 1, n + 1):
        q[i - d] += 2.0 * c[i]
        r[2 * d - i] -= c[i]
    return q, r


def _trim(c: np.ndarray) -> np.ndarray:
    return np.asarray(c[: chebyshev_degree(c) + 1], dtype=np.float64)


# ---------------------------------------------------------------------------
# ladder
# ---------------------------------------------------------------------------


class Ladder:
    """Limb counts and exact scales of consecutive levels (see module doc)."""

    def __init__(self, primes: Sequence[int], top_limbs: int, top_scale: float, step: int,
                 depth: int):
        if step < 1:
            raise ValueError("step must be positive")
        self.primes = [int(q) for q in primes]
        self.step = int(step)
        self.limbs = [int(top_limbs) - j * self.step for j in range(depth + 1)]
        if self.limbs[-1] < 1:
            raise ValueError(
                f"{top_limbs} limbs cannot hold {depth} levels of {step} prime(s)")
        self.scale = [float(top_scale)]
        for j in range(depth):
            self.scale.append(self.scale[j] ** 2 / self.divisor(j + 1))

    @property
    def depth(self) -> int:
        return len(self.limbs) - 1

    def divisor(self, j: int) -> float:
        """Product of the primes dropped when landing on level j."""
        lo = self.limbs[j]
        return math.prod(float(q) for q in self.primes[lo: lo + self.step])

    def entry_limbs(self, j: int) -> int:
        """Limbs an operand needs before the rescale that lands on level j."""
        return self.limbs[j] + self.step


@dataclass
class LCt:
    """A ciphertext on ladder level ``level``."""

    ct: object
    level: int


class LadderOps:
    """Homomorphic operations that keep ciphertexts on a ladder."""

    def __init__(self, context, ladder: Ladder):
        self.ctx = context
        self.lad = ladder
        self.mults = 0  # ciphertext-ciphertext products (one keyswitch each)

    # -- helpers --------------------------------------------------------------
    def _drop(self, ct, limbs: int):
        if int(ct.state.cur_limbs) == limbs:
            return ct
        return fhe.align_to(ct, ct.state.replace(cur_limbs=limbs, scaling_factor=None), self.ctx)

    def _rescale_steps(self, ct):
        # the level's primes in one pass (same words as one rescale per prime)
        return fhe.rescale_many([ct], self.ctx, primes=self.lad.step)[0]

    def _settle(self, ct, level: int):
        ct.set_scale(self.lad.scale[level], 1)
        return LCt(ct, level)

    # -- linear ---------------------------------------------------------------
    def combine(self, terms, const: float, level: int) -> LCt:
        """sum_i w_i x_i + const landing exactly on ``level``.  Each term is
        (LCt or raw ciphertext, weight); operands must hold more limbs than
        the level (one rescale step is taken)."""
        lad = self.lad
        limbs = lad.entry_limbs(level)
        target = lad.scale[level] * lad.divisor(level)
        cts, weights = [], []
        for x, w in terms:
            if w == 0.0:
                continue
            ct = x.ct if isinstance(x, LCt) else x
            src = lad.scale[x.level] if isinstance(x, LCt) else float(ct.state.scaling_factor)
            if int(ct.state.cur_limbs) < limbs:
                raise ValueError("operand is below the requested ladder level")
            cts.append([ct])
            weights.append(float(w) * (target / src))
        if not cts:
            raise ValueError("linear combination without ciphertext terms")
        # one launch: sum_t rint(w_t target / src_t) x_t + rint(const target)
        acc = fhe.linear_combination(cts, weights, float(const) * target, limbs, target, 2,
                                     self.ctx)[0]
        return self._settle(self._rescale_steps(acc), level)

    def lower(self, x: LCt, level: int) -> LCt:
        if x.level == level:
            return x
        if x.level > level:
            raise ValueError("cannot raise a ciphertext on the ladder")
        return self.combine([(x, 1.0)], 0.0, level)

    def add(self, a: LCt, b: LCt, sign: float = 1.0) -> LCt:
        lev = max(a.level, b.level)
        a, b = self.lower(a, lev), self.lower(b, lev)
        fn = fhe.homo_add if sign > 0 else fhe.homo_sub
        return LCt(fn(a.ct, b.ct, self.ctx), lev)

    def add_const(self, a: LCt, c: float) -> LCt:
        if c == 0.0:
            return a
        limbs = int(a.ct.state.cur_limbs)
        enc = fhe.encode_scalar(float(c), limbs, scaling_factor=self.lad.scale[a.level],
                                context=self.ctx)
        return LCt(fhe.homo_add_scalar(a.ct, enc, self.ctx), a.level)

    def double(self, a: LCt) -> LCt:
        return LCt(fhe.homo_add(a.ct, a.ct, self.ctx), a.level)

    # -- products -------------------------------------------------------------
    def mul(self, a: LCt, b: LCt) -> LCt:
        lev = max(a.level, b.level)
        if lev + 1 > self.lad.depth:
            raise ValueError("ladder depth exhausted")
        a, b = self.lower(a, lev), self.lower(b, lev)
        self.mults += 1
        # relinearise and the level's rescales as one ModDown (same words as
        # homo_mul_relin then the rescales)
        prod = fhe.homo_mul_relin_rescale_many([a.ct], [b.ct], self.ctx,
                                               primes=self.lad.step)[0]
        return self._settle(prod, lev + 1)


class BatchLadderOps(LadderOps):
    """LadderOps over a group of ciphertexts that share every level (an LCt's
    ``ct`` is a list): products run as one batched relinearise + rescale, so
    the relinearisation key is read once per group; constants are encoded once
    and shared."""

    def _rescale_steps(self, cts):
        return fhe.rescale_many(cts, self.ctx, primes=self.lad.step)

    def _settle(self, cts, level: int):
        for ct in cts:
            ct.set_scale(self.lad.scale[level], 1)
        return LCt(cts, level)

    def combine(self, terms, const: float, level: int) -> LCt:
        lad = self.lad
        limbs = lad.entry_limbs(level)
        target = lad.scale[level] * lad.divisor(level)
        rows, weights = [], []
        for x, w in terms:
            if w == 0.0:
                continue
            cts = x.ct if isinstance(x, LCt) else list(x)
            src = lad.scale[x.level] if isinstance(x, LCt) else float(cts[0].state.scaling_factor)
            if int(cts[0].state.cur_limbs) < limbs:
                raise ValueError("operand is below the requested ladder level")
            rows.append(cts)
            weights.append(float(w) * (target / src))
        if not rows:
            raise ValueError("linear combination without ciphertext terms")
        acc = fhe.linear_combination(rows, weights, float(const) * target, limbs, target, 2,
                                     self.ctx)
        return self._settle(self._rescale_steps(acc), level)

    def add(self, a: LCt, b: LCt, sign: float = 1.0) -> LCt:
        lev = max(a.level, b.level)
        a, b = self.lower(a, lev), self.lower(b, lev)
        fn = fhe.homo_add_many if sign > 0 else fhe.homo_sub_many
        return LCt(fn(a.ct, b.ct, self.ctx), lev)

    def add_const(self, a: LCt, c: float) -> LCt:
        if c == 0.0:
            return a
        limbs = int(a.ct[0].state.cur_limbs)
        enc = fhe.encode_scalar(float(c), limbs, scaling_factor=self.lad.scale[a.level],
                                context=self.ctx)
        return LCt([fhe.homo_add_scalar(x, enc, self.ctx) for x in a.ct], a.level)

    def double(self, a: LCt) -> LCt:
        return LCt(fhe.homo_add_many(a.ct, a.ct, self.ctx), a.level)

    def mul(self, a: LCt, b: LCt) -> LCt:
        lev = max(a.level, b.level)
        if lev + 1 > self.lad.depth:
            raise ValueError("ladder depth exhausted")
        a, b = self.lower(a, lev), self.lower(b, lev)
        self.mults += len(a.ct)
        prods = fhe.homo_mul_relin_rescale_many(a.ct, b.ct, self.ctx, primes=self.lad.step)
        return self._settle(prods, lev + 1)


class _SymbolicOps:
    """Level bookkeeping only: runs the evaluation schedule without data."""

    def __init__(self):
        self.mults = 0

    def combine(self, terms, const, level):
        return LCt(None, level)

    def lower(self, x, level):
        if x.level > level:
            raise ValueError("cannot raise a ciphertext on the ladder")
        return LCt(None, level)

    def add(self, a, b, sign=1.0):
        return LCt(None, max(a.level, b.level))

    def add_const(self, a, c):
        return a

    def double(self, a):
        return a

    def mul(self, a, b):
        self.mults += 1
        return LCt(None, max(a.level, b.level) + 1)


# ---------------------------------------------------------------------------
# baby-step giant-step evaluation
# ---------------------------------------------------------------------------


class _Series:
    def __init__(self, ops, y: LCt, k: int):
        self.ops = ops
        self.k = k
        self.T = {1: y}

    def t(self, i: int) -> LCt:
        """T_i at level ceil(log2 i): T_2m = 2 T_m^2 - 1 and
        T_(a+b) = 2 T_a T_b - T_(a-b) with a the largest power of two < i."""
        if i in self.T:
            return self.T[i]
        ops = self.ops
        if i & (i - 1) == 0:
            h = self.t(i // 2)
            out = ops.add_const(ops.double(ops.mul(h, h)), -1.0)
        else:
            a = 1 << (i.bit_length() - 1)
            b = i - a
            prod = ops.double(ops.mul(self.t(a), self.t(b)))
            out = ops.add(prod, self.t(a - b), sign=-1.0)
        self.T[i] = out
        return out

    def leaf(self, c: np.ndarray, level: int | None) -> LCt:
        terms = [(self.t(i), float(c[i])) for i in range(1, len(c)) if c[i] != 0.0]
        natural = max(t.level for t, _ in terms) + 1
        return self.ops.combine(terms, float(c[0]), max(natural, level or natural))

    def eval(self, c: np.ndarray, level: int | None = None) -> LCt:
        c = _trim(c)
        n = len(c) - 1
        if n < 1:
            raise ValueError("constant polynomial has no ciphertext value")
        if n < self.k:
            return self.leaf(c, level)
        d = self.k
        while 2 * d <= n:
            d *= 2
        q, r = divide_by_t(c, d)
        q, r = _trim(q), _trim(r)
        giant = self.t(d)
        if len(q) == 1:
            prod = self.ops.combine([(giant, float(q[0]))], 0.0, giant.level + 1)
        else:
            prod = self.ops.mul(self.eval(q), giant)
        if len(r) == 1:
            out = self.ops.add_const(prod, float(r[0]))
        else:
            out = self.ops.add(prod, self.eval(r, prod.level))
        if level is not None and level > out.level:
            out = self.ops.lower(out, level)
        return out


def _full(coefficients) -> np.ndarray:
    c = np.array(coefficients, dtype=np.float64)
    c[0] *= 0.5
    return _trim(c)


def plan_baby(coefficients) -> tuple[int, int, int]:
    """(k, depth, products) minimising depth, then ciphertext products."""
    c = _full(coefficients)
    best = None
    for k in (2, 4, 8, 16, 32, 64):
        if k > 2 * max(2, len(c)):
            break
        ops = _SymbolicOps()
        out = _Series(ops, LCt(None, 0), k).eval(c)
        key = (out.level, ops.mults, k)
        if best is None or key < best:
            best = key
    return best[2], best[0], best[1]


def chebyshev_depth(coefficients) -> int:
    """Levels consumed by evaluate() on an input already in [-1, 1]."""
    return plan_baby(coefficients)[1]


def evaluate(ops: LadderOps, y: LCt, coefficients, level: int | None = None) -> LCt:
    """Series (reference convention) at ``y`` (a ladder ciphertext holding
    values in [-1, 1]); the result lands on ``level`` when given."""
    k = plan_baby(coefficients)[0]
    return _Series(ops, y, k).eval(_full(coefficients), level)


# ---------------------------------------------------------------------------
# drop-in evaluator
# ---------------------------------------------------------------------------


def _native_context(crypto_context):
    return getattr(crypto_context, "context", crypto_context)


def series_depth(coefficients, mapped: bool = False) -> int:
    """Levels eval_chebyshev_series_cipher consumes (one more for the map
    onto [-1, 1] unless the input is already mapped)."""
    return chebyshev_depth(coefficients) + (0 if mapped else 1)


def eval_chebyshev_series_cipher(input_cipher, coefficients, *, lower_bound: float,
                                 upper_bound: float, crypto_context,
                                 input_is_chebyshev_mapped: bool = False):
    """Chebyshev series (reference convention) of one ciphertext on
    [lower_bound, upper_bound] (reference
    operators/nonlinear/polynomial.py:364-412).  One prime per level; the
    input must hold at least series_depth() + 1 limbs."""
    ctx = _native_context(crypto_context)
    coeffs = np.asarray(coefficients, dtype=np.float64)
    if chebyshev_degree(coeffs) < 1:
        raise ValueError("degree must be >= 1")
    primes = [int(q) for q in ctx.primes()[: ctx.L]]
    limbs = int(input_cipher.state.cur_limbs)
    depth = chebyshev_depth(coeffs)
    a, b = float(lower_bound), float(upper_bound)
    if input_is_chebyshev_mapped:
        lad = Ladder(primes, limbs, float(input_cipher.state.scaling_factor), 1, depth)
        ops = LadderOps(ctx, lad)
        y = LCt(input_cipher, 0)
    else:
        if limbs < depth + 2:
            raise ValueError(f"need {depth + 2} limbs, ciphertext has {limbs}")
        top = limbs - 1
        lad = Ladder(primes, top, float(primes[top - 1]), 1, depth)
        ops = LadderOps(ctx, lad)
        y = ops.combine([(input_cipher, 2.0 / (b - a))], -(a + b) / (b - a), 0)
    return evaluate(ops, y, coeffs).ct


def eval_chebyshev_series_many(input_ciphers, coefficients, *, lower_bound: float,
                               upper_bound: float, crypto_context,
                               input_is_chebyshev_mapped: bool = False) -> list:
    """eval_chebyshev_series_cipher over a group of ciphertexts that share
    their limb count and scale: every product of the evaluation is one batched
    relinearise + rescale for the group (BatchLadderOps), so the relinearisation
    key is read once per product level.  Same words as evaluating each
    ciphertext alone."""
    ctx = _native_context(crypto_context)
    cts = list(input_ciphers)
    if not cts:
        return []
    coeffs = np.asarray(coefficients, dtype=np.float64)
    if chebyshev_degree(coeffs) < 1:
        raise ValueError("degree must be >= 1")
    limbs = int(cts[0].state.cur_limbs)
    scale = float(cts[0].state.scaling_factor)
    for ct in cts:
        if int(ct.state.cur_limbs) != limbs:
            raise ValueError("a polynomial group must share its limb count")
        if abs(float(ct.state.scaling_factor) / scale - 1.0) > 2.0 ** -30:
            raise ValueError("a polynomial group must share its scale")
    primes = [int(q) for q in ctx.primes()[: ctx.L]]
    depth = chebyshev_depth(coeffs)
    a, b = float(lower_bound), float(upper_bound)
    if input_is_chebyshev_mapped:
        lad = Ladder(primes, limbs, scale, 1, depth)
        ops = BatchLadderOps(ctx, lad)
        y = LCt(cts, 0)
    else:
        if limbs < depth + 2:
            raise ValueError(f"need {depth + 2} limbs, ciphertexts have {limbs}")
        top = limbs - 1
        lad = Ladder(primes, top, float(primes[top - 1]), 1, depth)
        ops = BatchLadderOps(ctx, lad)
        y = ops.combine([(cts, 2.0 / (b - a))], -(a + b) / (b - a), 0)
    return list(evaluate(ops, y, coeffs).ct)


__all__ = [
    "BatchLadderOps", "Ladder", "LadderOps", "LCt", "chebyshev_coefficients", "chebyshev_degree",
    "chebyshev_depth", "divide_by_t", "eval_chebyshev_series_cipher", "eval_chebyshev_series_many",
    "evaluate",
    "evaluate_direct", "plan_baby", "series_depth",
]
