"""CPU model of the bootstrap program and of the Chebyshev evaluator.

The schedules of ``easyfhe.chebyshev`` and ``easyfhe.bs`` are run on plain
numpy slot vectors (an ``ops`` object with the ladder interface that acts on
values instead of ciphertexts), so that the algebra, the BSGS offsets, the
folded constants and the EvalMod interpolant are checked against the
mathematics without a GPU:

* Chebyshev division and recursion against numpy.polynomial.chebyshev;
* the coefficient fit against numpy's chebinterpolate (same nodes);
* CoeffToSlot -> EvalMod -> SlotToCoeff on t = u 2^-10 + I (I random
  integers, the ModRaise overflow) returns the message.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
from numpy.polynomial import chebyshev as npcheb

from easyfhe import chebyshev as cheb
from easyfhe.bs import lintrans
from easyfhe.bs import openfhe as bs


class ValueOps:
    """Ladder operations on numpy values (optional relative noise)."""

    def __init__(self, noise: float = 0.0, seed: int = 0):
        self.noise = noise
        self.rng = np.random.default_rng(seed)
        self.mults = 0

    def _n(self, v):
        if not self.noise:
            return v
        return v + self.noise * self.rng.standard_normal(np.shape(v))

    def combine(self, terms, const, level):
        acc = const + sum(w * (x.ct if isinstance(x, cheb.LCt) else x) for x, w in terms)
        return cheb.LCt(self._n(acc), level)

    def lower(self, x, level):
        assert level >= x.level
        return cheb.LCt(x.ct, level)

    def add(self, a, b, sign=1.0):
        return cheb.LCt(a.ct + sign * b.ct, max(a.level, b.level))

    def add_const(self, a, c):
        return cheb.LCt(a.ct + c, a.level)

    def double(self, a):
        return cheb.LCt(2.0 * a.ct, a.level)

    def mul(self, a, b):
        self.mults += 1
        return cheb.LCt(self._n(a.ct * b.ct), max(a.level, b.level) + 1)


def test_coefficients_match_numpy_interpolation():
    f = np.exp
    c = cheb.chebyshev_coefficients(lambda v: math.exp(v), -1.0, 1.0, 20)
    ref = npcheb.chebinterpolate(f, 20)
    ref[0] *= 2.0  # reference convention carries 2 c_0
    assert np.allclose(c, ref, atol=1e-14)


def test_division_by_t_d():
    rng = np.random.default_rng(1)
    x = np.linspace(-1, 1, 101)
    for n, d in ((9, 8), (15, 8), (31, 16), (60, 32)):
        c = rng.standard_normal(n + 1)
        q, r = cheb.divide_by_t(c, d)
        td = npcheb.chebval(x, np.eye(d + 1)[d])
        assert len(r) == d
        assert np.allclose(npcheb.chebval(x, q) * td + npcheb.chebval(x, r),
                           npcheb.chebval(x, c), atol=1e-11)


@pytest.mark.parametrize("degree", [1, 2, 3, 7, 8, 15, 27, 48, 59, 60, 77, 120])
def test_series_schedule_values_and_depth(degree):
    rng = np.random.default_rng(degree)
    coeffs = rng.uniform(-1, 1, degree + 1) / np.arange(1, degree + 2)
    y = np.cos(np.linspace(0, math.pi, 257))
    ops = ValueOps()
    out = cheb.evaluate(ops, cheb.LCt(y, 0), coeffs)
    want = cheb.evaluate_direct(y, coeffs)
    assert np.abs(out.ct - want).max() < 1e-12
    depth = cheb.chebyshev_depth(coeffs)
    assert out.level == depth
    # the minimum multiplicative depth of any degree-n evaluation
    assert depth == math.ceil(math.log2(degree + 1))


def test_depth_is_minimal_for_every_degree():
    for n in range(1, 260):
        assert cheb.chebyshev_depth(np.ones(n + 1)) == math.ceil(math.log2(n + 1)), n


def test_clenshaw_matches_numpy_chebval():
    rng = np.random.default_rng(3)
    c = rng.standard_normal(30)
    x = np.linspace(-3, 5, 77)
    ref = c.copy()
    ref[0] *= 0.5
    assert np.allclose(cheb.evaluate_direct(x, c, -3, 5),
                       npcheb.chebval((2 * x - 2) / 8, ref), atol=1e-12)


def _special_fft(u: np.ndarray) -> np.ndarray:
    """z = S_L .. S_1 P u (slots of the coefficient vector u)."""
    n = len(u)
    log_n = n.bit_length() - 1
    idx = np.array([int(format(i, f"0{log_n}b")[::-1], 2) for i in range(n)])
    x = u[idx]
    for s in range(1, log_n + 1):
        x = lintrans.apply_diagonals(lintrans.stage_diagonals(n, s, False), x)
    return x


def _bsgs(x: np.ndarray, plan, rows: np.ndarray) -> np.ndarray:
    """hoisted_mac_sum on values: sum_g rot_(g giant)(sum_b p[gB+b] rot_(off_b) x)."""
    n = len(x)
    offs = bs._baby_offsets(plan, n)
    giant = bs._giant_offset(plan, n)
    acc = np.zeros(n, dtype=np.complex128)
    for g in reversed(range(plan.giant)):
        inner = sum(rows[g * plan.baby + b] * np.roll(x, -offs[b]) for b in range(plan.baby))
        acc = np.roll(acc, -giant) + inner if g < plan.giant - 1 else inner
    return acc


def _horner_check(x, plan, rows):
    """The Horner form used by the device equals the direct BSGS sum."""
    n = len(x)
    offs = bs._baby_offsets(plan, n)
    giant = bs._giant_offset(plan, n)
    direct = sum(np.roll(sum(rows[g * plan.baby + b] * np.roll(x, -offs[b])
                             for b in range(plan.baby)), -g * giant) for g in range(plan.giant))
    return direct


@pytest.mark.parametrize("log_n,budget,strategy",
                         [(6, (2, 2), "normal"), (10, (3, 3), "normal"), (10, (3, 3), "ext_normal"),
                          (10, (4, 4), "ext_normal"), (10, (3, 3), "ext_double_hoist"),
                          (11, (3, 2), "normal")])
def test_bootstrap_model_recovers_message(log_n, budget, strategy):
    n = 1 << log_n
    rng = np.random.default_rng(log_n)
    p = bs.BootstrapParams(strategy=strategy)
    spec = bs.BootstrapSpec(log_slots=log_n, level_budget=budget)
    cts_plans, stc_plans = bs._plans(spec, p)
    if strategy != "normal":
        assert all(plan.giant <= p.giants for plan in (*cts_plans, *stc_plans))
    z = rng.uniform(-1, 1, n) + 1j * rng.uniform(-1, 1, n)
    # coefficient vector of the message at scale Delta' = 2^-10 q_0, plus the
    # integer overflow I of ModRaise (|I| well inside K)
    P = np.array([int(format(i, f"0{log_n}b")[::-1], 2) for i in range(n)])
    u = z.copy()
    for s in reversed(range(1, log_n + 1)):
        u = lintrans.apply_diagonals(lintrans.stage_diagonals(n, s, True), u)
    u_nat = np.empty_like(u)
    u_nat[P] = u
    assert np.abs(_special_fft(u_nat) - z).max() < 1e-9
    I = rng.integers(-12, 13, n) + 1j * rng.integers(-12, 13, n)
    t = u_nat * 2.0 ** -p.ratio_bits + I
    x = _special_fft(t) / (2 * p.K)  # slots of the raised ciphertext at scale 2 K q_0
    for plan in cts_plans:
        rows = plan.plaintext_rows(n)
        y = _bsgs(x, plan, rows)
        assert np.allclose(y, _horner_check(x, plan, rows), atol=1e-9)
        x = y
    assert np.abs(x - t[P] / (2 * p.K)).max() < 1e-9  # bit-reversed t / 2K
    re = x + np.conj(x)
    im = -1j * (x - np.conj(x))
    coeffs = bs._evalmod_coefficients(p)
    outs = []
    for v in (re, im):
        ops = ValueOps()
        c = cheb.evaluate(ops, cheb.LCt(v.real, 0), coeffs)
        for _ in range(p.double_angles):
            c = ops.add_const(ops.double(ops.mul(c, c)), -1.0)
        outs.append(c.ct)
    assert np.abs(outs[0] - np.sin(2 * np.pi * t[P].real)).max() < 1e-9
    u2 = outs[0] + 1j * outs[1]
    ideal = np.sin(2 * np.pi * t[P].real) + 1j * np.sin(2 * np.pi * t[P].imag)
    fold = 1.0 / (2 * math.pi * 2.0 ** -p.ratio_bits)
    for i, plan in enumerate(stc_plans):
        rows = plan.plaintext_rows(n, fold if i == 0 else 1.0)
        u2 = _bsgs(u2, plan, rows)
        ideal = _bsgs(ideal, plan, rows)
    # the schedule equals SlotToCoeff of the exact sine ...
    assert np.abs(u2 - ideal).max() < 1e-8
    # ... whose distance to the message is the sine's curvature on the
    # coefficients (|u_k| ~ |z| / sqrt(n)): (2 pi)^2 |u|^3 2^-20 / 6 per
    # coefficient
    err = np.abs(ideal - z).max()
    assert 1e-12 < err < 2.0 ** -20, err


def test_requirements_and_limb_plan():
    spec = bs.BootstrapSpec(log_slots=15, level_budget=(3, 3), output_levels=0)
    req = bs.requirements([spec], log_n=16)
    assert 2 * 65536 - 1 in req.rotations
    assert all(0 < r < 2 * 65536 for r in req.rotations)
    # extended-basis levels (at most 2 giants): up to 32 babies per level
    assert len(req.rotations) <= 96
    # a sparse program: the sub-sum's rotations n, 2n, .., N/4 plus its
    # n-slot transforms' (all below n; below 2n for the two levels next to
    # the packed EvalMod), and the conjugation
    sparse = bs.requirements([bs.BootstrapSpec(log_slots=7, level_budget=(3, 3))], log_n=16)
    subsum = {128 << k for k in range(8)}
    assert subsum <= set(sparse.rotations)
    assert all(r < 256 for r in set(sparse.rotations) - subsum - {2 * 65536 - 1})
    unpacked = bs.requirements([bs.BootstrapSpec(log_slots=7, level_budget=(3, 3))], log_n=16,
                               params=bs.BootstrapParams(packed_evalmod=False))
    assert all(r < 128 for r in set(unpacked.rotations) - subsum - {2 * 65536 - 1})
    assert len(sparse.rotations) < len(req.rotations)
    with pytest.raises(ValueError):
        bs.requirements([bs.BootstrapSpec(log_slots=16)], log_n=16)


def _slots_of(coeffs: np.ndarray) -> np.ndarray:
    """Full-slot view (N/2 slots) of a real coefficient vector of length N:
    the special FFT of u_k = m_k + i m_(k + N/2)."""
    half = len(coeffs) // 2
    return _special_fft(coeffs[:half] + 1j * coeffs[half:])


@pytest.mark.parametrize("log_n,log_slots,budget", [(10, 4, (2, 2)), (9, 3, (3, 3))])
def test_sparse_bootstrap_model(log_n, log_slots, budget):
    """The sparse program on values: after ModRaise the raised polynomial has
    all N coefficients (the overflow I); the sub-sum (rotations n, 2n, ..)
    is the trace, which keeps gap times the coefficients at multiples of
    gap = N / 2n; the n-slot CoeffToSlot (first level scaled by 1 / gap)
    applied to the full-length, n-periodic vector, EvalMod and SlotToCoeff
    return the message in every copy."""
    N, half = 1 << log_n, 1 << (log_n - 1)
    n = 1 << log_slots
    gap = half // n
    rng = np.random.default_rng(log_n + log_slots)
    p = bs.BootstrapParams()
    spec = bs.BootstrapSpec(log_slots=log_slots, level_budget=budget)
    cts_plans, stc_plans = bs._plans(spec, p, log_n)
    rots = bs._subsum_rotations(spec, log_n)
    assert rots == [n << k for k in range(int(math.log2(gap)))]
    # the message's Y-polynomial (Y = X^gap, 2n real coefficients)
    z = rng.uniform(-1, 1, n) + 1j * rng.uniform(-1, 1, n)
    Pn = np.array([int(format(i, f"0{log_slots}b")[::-1], 2) for i in range(n)])
    u = z.copy()
    for s_ in reversed(range(1, log_slots + 1)):
        u = lintrans.apply_diagonals(lintrans.stage_diagonals(n, s_, True), u)
    u_nat = np.empty_like(u)
    u_nat[Pn] = u
    t = np.concatenate([u_nat.real, u_nat.imag]) * 2.0 ** -p.ratio_bits
    m = np.zeros(N)
    m[::gap] = t
    # its full-slot view repeats z
    assert np.abs(_slots_of(m) - np.tile(z, gap) * 2.0 ** -p.ratio_bits).max() < 1e-9
    # ModRaise: an integer overflow on every coefficient
    I = rng.integers(-12, 13, N).astype(float)
    x = _slots_of(m + I) / (2 * p.K)
    # the sub-sum, as slot rotations
    for r in rots:
        x = x + np.roll(x, -r)
    keep = np.zeros(N)
    keep[::gap] = gap * (m + I)[::gap]
    assert np.abs(x - _slots_of(keep) / (2 * p.K)).max() < 1e-8
    assert np.abs(x - np.tile(x[:n], gap)).max() < 1e-8
    for i, plan in enumerate(cts_plans):
        rows = plan.plaintext_rows(n, 1.0 / gap if i == 0 else 1.0)
        offs = bs._baby_offsets(plan, n)
        giant = bs._giant_offset(plan, n)
        full = np.zeros(half, dtype=np.complex128)
        for g in range(plan.giant):
            inner = sum(np.tile(rows[g * plan.baby + b], gap) * np.roll(x, -offs[b])
                        for b in range(plan.baby))
            full = full + np.roll(inner, -g * giant)
        x_n = _bsgs(x[:n], plan, rows)
        assert np.abs(full - np.tile(x_n, gap)).max() < 1e-8
        x = full
    # bit-reversed t_k + i t_(k+n) (with the kept overflow) / 2K
    tk = (m + I)[::gap]
    want = (tk[:n] + 1j * tk[n:])[Pn] / (2 * p.K)
    assert np.abs(x[:n] - want).max() < 1e-8
    coeffs = bs._evalmod_coefficients(p)
    outs = []
    for v in (x[:n] + np.conj(x[:n]), -1j * (x[:n] - np.conj(x[:n]))):
        ops = ValueOps()
        c = cheb.evaluate(ops, cheb.LCt(v.real, 0), coeffs)
        for _ in range(p.double_angles):
            c = ops.add_const(ops.double(ops.mul(c, c)), -1.0)
        outs.append(c.ct)
    u2 = outs[0] + 1j * outs[1]
    fold = 1.0 / (2 * math.pi * 2.0 ** -p.ratio_bits)
    for i, plan in enumerate(stc_plans):
        u2 = _bsgs(u2, plan, plan.plaintext_rows(n, fold if i == 0 else 1.0))
    err = np.abs(u2 - z).max()
    assert err < 2.0 ** -18, err


def _mac_period(x: np.ndarray, rows: np.ndarray, babies, giant_off: int, giants: int):
    """hoisted_mac_sum on a full-length slot vector with rows of a shorter
    period: sum_g rot_(g giant)(sum_b tile(p[g B + b]) rot_(baby_b) x)."""
    reps, B = len(x) // rows.shape[1], len(babies)
    acc = np.zeros(len(x), dtype=np.complex128)
    for g in range(giants):
        inner = sum(np.tile(rows[g * B + b], reps) * np.roll(x, -babies[b]) for b in range(B))
        acc = acc + np.roll(inner, -g * giant_off)
    return acc


@pytest.mark.parametrize("log_n,log_slots,budget", [(10, 4, (2, 2)), (9, 3, (3, 3)),
                                                     (10, 6, (1, 3))])
def test_sparse_packed_evalmod_model(log_n, log_slots, budget):
    """Sparse program with one EvalMod per ciphertext (n <= N/4): the last
    CoeffToSlot level multiplies its output by the 2n-periodic mask
    a = lo - i hi, so w' + conj(w') holds 2 Re w on the first n slots of
    each 2n and 2 Im w on the next n; the first SlotToCoeff level reads
    d1 s + d2 rot_n(s) through a second baby set.  Checked on values: the
    packed vector, the first SlotToCoeff level against the unpacked level on
    2 w (EvalMod replaced by the identity), and the whole pipeline against
    the message."""
    N, half = 1 << log_n, 1 << (log_n - 1)
    n = 1 << log_slots
    gap = half // n
    rng = np.random.default_rng(3 * log_n + log_slots)
    p = bs.BootstrapParams()
    spec = bs.BootstrapSpec(log_slots=log_slots, level_budget=budget)
    assert bs._packed(spec, log_n, p)
    assert not bs._packed(bs.BootstrapSpec(log_slots=log_n - 1), log_n, p)
    assert not bs._packed(spec, log_n, bs.BootstrapParams(packed_evalmod=False))
    cts_plans, stc_plans = bs._plans(spec, p, log_n)
    a, d1, d2 = bs._packing_masks(n)
    z = rng.uniform(-1, 1, n) + 1j * rng.uniform(-1, 1, n)
    Pn = np.array([int(format(i, f"0{log_slots}b")[::-1], 2) for i in range(n)])
    u = z.copy()
    for s_ in reversed(range(1, log_slots + 1)):
        u = lintrans.apply_diagonals(lintrans.stage_diagonals(n, s_, True), u)
    u_nat = np.empty_like(u)
    u_nat[Pn] = u
    t = np.concatenate([u_nat.real, u_nat.imag]) * 2.0 ** -p.ratio_bits
    m = np.zeros(N)
    m[::gap] = t
    I = rng.integers(-12, 13, N).astype(float)
    x = _slots_of(m + I) / (2 * p.K)
    for r in bs._subsum_rotations(spec, log_n):
        x = x + np.roll(x, -r)
    for i, plan in enumerate(cts_plans):
        factor = 1.0 / gap if i == 0 else 1.0
        if i == len(cts_plans) - 1:
            rows = bs._period_rows(plan, n, 2 * n, out_mask=a, scale_factor=factor)
            x_n = x  # the level's n-periodic input, kept for the unpacked check
            x = _mac_period(x, rows, bs._baby_offsets(plan, 2 * n), bs._giant_offset(plan, 2 * n),
                            plan.giant)
            w = _mac_period(x_n, plan.plaintext_rows(n, factor), bs._baby_offsets(plan, n),
                            bs._giant_offset(plan, n), plan.giant)
        else:
            x = _mac_period(x, plan.plaintext_rows(n, factor), bs._baby_offsets(plan, n),
                            bs._giant_offset(plan, n), plan.giant)
    tk = (m + I)[::gap]
    want = (tk[:n] + 1j * tk[n:])[Pn] / (2 * p.K)
    assert np.abs(w[:n] - want).max() < 1e-8
    assert np.abs(x - np.tile(a, gap // 2) * w).max() < 1e-8
    v = x + np.conj(x)
    packed = np.concatenate([2 * want.real, 2 * want.imag])
    assert np.abs(v - np.tile(packed, gap // 2)).max() < 1e-8
    fold = 1.0 / (2 * math.pi * 2.0 ** -p.ratio_bits)
    plan0 = stc_plans[0]
    rows0 = bs._period_rows(plan0, n, 2 * n, in_masks=(d1, d2), scale_factor=fold)
    babies0 = bs._baby_offsets(plan0, 2 * n, n)
    assert len(babies0) == 2 * plan0.baby and len(set(babies0)) == len(babies0)
    giant0 = bs._giant_offset(plan0, 2 * n)
    # EvalMod as the identity: the first level equals the unpacked one on 2 w
    lin = _mac_period(v, rows0, babies0, giant0, plan0.giant)
    ref = _mac_period(np.tile(2 * want, gap), plan0.plaintext_rows(n, fold),
                      bs._baby_offsets(plan0, n), bs._giant_offset(plan0, n), plan0.giant)
    assert np.abs(lin - ref).max() < 1e-6 * np.abs(ref).max()
    # the pipeline with EvalMod
    coeffs = bs._evalmod_coefficients(p)
    ops = ValueOps()
    c = cheb.evaluate(ops, cheb.LCt(v.real, 0), coeffs)
    for _ in range(p.double_angles):
        c = ops.add_const(ops.double(ops.mul(c, c)), -1.0)
    y = _mac_period(c.ct.astype(np.complex128), rows0, babies0, giant0, plan0.giant)
    for plan in stc_plans[1:]:
        y = _mac_period(y, plan.plaintext_rows(n), bs._baby_offsets(plan, n),
                        bs._giant_offset(plan, n), plan.giant)
    err = np.abs(y - np.tile(z, gap)).max()
    assert err < 2.0 ** -18, err
    # the program's rotation keys cover both masked levels
    rots = set(bs.requirements([spec], log_n=log_n, params=p).rotations)
    assert {r for r in babies0 if r} <= rots
    assert {r for r in bs._baby_offsets(cts_plans[-1], 2 * n) if r} <= rots
