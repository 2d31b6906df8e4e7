"""Full-slot CKKS bootstrapping (reference ``easyfhe.bs.openfhe`` as used by
operators/nonlinear/bootstrap.py:59-189, 352-437).

Pipeline ("modraise_first", reference bootstrap.py:29):

1. **Pre-scale.**  The input (any level, scale Delta_in) is taken to one limb
   with its message scaled to Delta' = q_0 2^-ratio_bits, so that
   t = (m' + q_0 I) / q_0 has a fractional part of at most about 2^-ratio_bits.
2. **ModRaise** (C entry point ``ckks_mod_raise``) to the limbs the program
   needs; the raised ciphertext is read at scale 2 K q_0, so its slots are
   FFT(u) / (2 K) with u_k = t_k + i t_(k+n).
3. **CoeffToSlot**: the inverse special FFT as ``level_budget[0]`` grouped
   sparse stages (``lintrans.plan_levels``), each one hoisted BSGS
   diagonal MAC (``hoisted_mac_sum``) and the rescales that keep the
   diagonals at 2^cts_pt_bits (``_plan_cts_drops``).
4. **EvalMod** on the real and imaginary parts (split with one conjugation):
   a Chebyshev interpolant of cos(2 pi (K y - 1/4) / 2^r) on [-1, 1] and r
   double-angle steps give sin(2 pi t), evaluated on an exact-scale ladder
   (``easyfhe.chebyshev``) at a working scale of at least 2^55 (two primes
   per level on a 40-bit chain).  A sparse program of at most N/4 slots
   packs both parts into one 2n-periodic vector (``_packing_masks``) and
   runs EvalMod once.
5. **SlotToCoeff**: the special FFT, with q_0 / (2 pi Delta') folded into
   its first level; the last level lands on the nominal scale 2^dcrt_bits.

The limb cost is fixed by the chain: the CoeffToSlot drops (at least
budget[0]) + step (depth + r) + step + budget[1] - 1, where step is the primes
per EvalMod level; the program raises to exactly output_levels + 1 + that
many limbs.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np

from .. import chebyshev as cheb
from .. import fhe
from .lintrans import LevelPlan, plan_levels

# Scale of the SlotToCoeff levels before the last one, and the data-scale cap
# of the CoeffToSlot levels (bits).
_STC_SCALE = 2.0**45
_CTS_CAP_BITS = 100
# EvalMod works at a scale of at least this many bits.
_EVALMOD_BITS = 55


@dataclass(frozen=True)
class BootstrapSpec:
    """Program parameters (reference bootstrap.py:59-85)."""

    log_slots: int = 15
    level_budget: tuple = (4, 4)
    output_levels: int = 0
    mode: str = "modraise_first"

    @property
    def slots(self) -> int:
        return 1 << int(self.log_slots)


@dataclass(frozen=True)
class BootstrapParams:
    """K bounds |t| (the integer part I plus the message), r double-angle
    steps, the interpolant error target, the headroom 2^ratio_bits of q_0
    over the pre-scaled message, and the encoding precision of the
    CoeffToSlot diagonals.  The CoeffToSlot output is read modulo 1 after a
    2^ratio_bits magnification, so its relative error bounds the result:
    each bit of cts_pt_bits is a bit of precision until the sine's curvature
    or the input noise dominates; the limbs it costs follow from the chain."""

    K: int = 28
    double_angles: int = 3
    fit_bits: int = 45
    ratio_bits: int = 10
    cts_pt_bits: int = 58
    # linear levels: "ext_normal" keeps the babies in Q u P (one ModDown per
    # giant group, at most `giants` giants); "ext_double_hoist" (the default)
    # also rotates the giant groups in Q u P (one key per giant step, one
    # ModDown per level: 2.5-3.5 % faster bootstraps at 2 giants, the same
    # precision; more giants are slower); "normal" ModDowns every baby
    strategy: str = "ext_double_hoist"
    giants: int = 2
    # sparse programs (n <= N/4 slots): real and imaginary parts share one
    # 2n-periodic vector, so EvalMod runs once per ciphertext, not twice
    packed_evalmod: bool = True



@dataclass
class Requirements:
    rotations: tuple


def _check_spec(spec: BootstrapSpec, log_n: int) -> None:
    if spec.mode != "modraise_first":
        raise ValueError(f"unsupported bootstrap mode {spec.mode!r}")
    if not 1 <= int(spec.log_slots) <= log_n - 1:
        raise ValueError(f"log_slots must be in [1, {log_n - 1}], got {spec.log_slots}")
    budget = tuple(int(v) for v in spec.level_budget)
    if len(budget) != 2 or min(budget) < 1 or max(budget) > log_n - 1:
        raise ValueError(f"level_budget must be two values in [1, {log_n - 1}], got {budget}")


def _transform_log_slots(spec: BootstrapSpec, log_n: int) -> int:
    """The linear transforms act on the program's 2^log_slots slots.  A
    sparse ciphertext's plaintext (log_slots < log_n - 1) is a polynomial in
    Y = X^gap, gap = N / 2^(log_slots + 1), whose full-slot view repeats its
    2^log_slots values; after the sub-sum the raised ciphertext is such a
    polynomial too, and the n-slot special FFT maps its 2n coefficients to
    the n slots (the full-slot view of every rotation and diagonal repeats
    with period n)."""
    return int(spec.log_slots)


def _subsum_rotations(spec: BootstrapSpec, log_n: int) -> list[int]:
    """Rotations of the sub-sum: n, 2n, 4n, .. N/4 for n = 2^log_slots (none
    for a full-slot program).  Adding each rotation sums the N / 2n copies of
    the n-periodic slot vector, i.e. the trace to Z[Y]/(Y^2n + 1): it keeps
    the raised polynomial's coefficients at multiples of gap (times gap) and
    removes the others (reference bootstrap.py:34-45 selects such a program
    for the slim refreshes)."""
    n, half = 1 << int(spec.log_slots), 1 << (int(log_n) - 1)
    out, r = [], n
    while r < half:
        out.append(r)
        r *= 2
    return out


def _plans(spec: BootstrapSpec, params: "BootstrapParams | None" = None, log_n: int = 0):
    b0, b1 = (int(v) for v in spec.level_budget)
    giants = params.giants if params is not None and params.strategy != "normal" else 0
    ls = _transform_log_slots(spec, log_n) if log_n else int(spec.log_slots)
    return (plan_levels(ls, b0, inverse=True, giants=giants),
            plan_levels(ls, b1, inverse=False, giants=giants))


def _baby_offsets(plan: LevelPlan, n: int, shift: int = 0) -> list[int]:
    """Baby rotations of a level whose slot vectors repeat with period n;
    with ``shift`` the list is followed by the same rotations plus shift."""
    offs = [(b * plan.stride - plan.center) % n for b in range(plan.baby)]
    return offs + [(o + shift) % n for o in offs] if shift else offs


def _giant_offset(plan: LevelPlan, n: int) -> int:
    return (plan.baby * plan.stride) % n


def _level_rotations(plan: LevelPlan, n: int, strategy: str = "ext_normal",
                     shift: int = 0) -> set[int]:
    rots = {o for o in _baby_offsets(plan, n, shift) if o}
    if plan.giant > 1 and _giant_offset(plan, n):
        if strategy == "ext_double_hoist":
            # every giant group rotates by its own multiple of the giant step
            rots.update(g * _giant_offset(plan, n) % n for g in range(1, plan.giant))
            rots.discard(0)
        else:
            rots.add(_giant_offset(plan, n))
    return rots


def _packed(spec: BootstrapSpec, log_n: int, p: BootstrapParams) -> bool:
    """Whether the program runs one EvalMod on a 2n-periodic vector that
    holds the real parts in its first n slots and the imaginary parts in the
    next n (possible when 2n slots fit: n <= N/4)."""
    return bool(p.packed_evalmod) and int(spec.log_slots) <= int(log_n) - 2


def _packing_masks(n: int) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """Slot masks of period 2n (lo = the first n slots of each period):
    a = lo - i hi, so that w' + conj(w') for w' = a w is 2 Re w on lo and
    2 Im w on hi (w n-periodic); then u = d1 s + d2 rot_n(s) with
    d1 = lo + i hi, d2 = i lo + hi rebuilds the n-periodic s_lo + i s_hi."""
    lo = np.arange(2 * n) < n
    a = np.where(lo, 1.0 + 0j, -1j)
    d1 = np.where(lo, 1.0 + 0j, 1j)
    d2 = np.where(lo, 1j, 1.0 + 0j)
    return a, d1, d2


def _period_rows(plan: LevelPlan, n: int, m: int, out_mask=None, in_masks=None,
                 scale_factor: float = 1.0) -> np.ndarray:
    """Diagonal rows of a level applied to slot vectors of period m (a
    multiple of n), in the order of hoisted_mac_sum: row g B' + k B + b for
    giant g, input mask k and baby b (B' = B times the number of masks).
    out_mask multiplies the level's output slot-wise; with in_masks
    [d_0, d_1, ..] the level reads u = sum_k d_k rot_(k n)(x), which puts the
    term of offset o on the baby rot_(o + k n)(x) with the diagonal
    d_o(i) d_k(i + o)."""
    masks = list(in_masks) if in_masks is not None else [None]
    B, reps = plan.baby, m // n
    rows = np.zeros((plan.giant * B * len(masks), m), dtype=np.complex128)
    for g in range(plan.giant):
        for k, d_in in enumerate(masks):
            for b in range(B):
                t = g * B + b
                o = t * plan.stride - plan.center
                if t >= plan.width or o % n not in plan.diagonals:
                    continue
                d = np.tile(plan.diagonals[o % n], reps)
                if out_mask is not None:
                    d = d * out_mask
                if d_in is not None:
                    d = d * np.roll(d_in, -o)
                rows[(g * len(masks) + k) * B + b] = np.roll(d, g * B * plan.stride)
    return rows * scale_factor


def requirements(specs, log_n: int, params: "BootstrapParams | None" = None) -> Requirements:
    """Rotation indices every listed program needs, conjugation (2N - 1)
    included (reference bootstrap.py:154-189)."""
    if isinstance(specs, BootstrapSpec):
        specs = (specs,)
    p = params or BootstrapParams()
    rots: set[int] = set()
    for spec in specs:
        _check_spec(spec, int(log_n))
        n = 1 << _transform_log_slots(spec, int(log_n))
        cts, stc = _plans(spec, p, int(log_n))
        packed = _packed(spec, int(log_n), p)
        for i, plan in enumerate(cts):
            m = 2 * n if packed and i == len(cts) - 1 else n
            rots |= _level_rotations(plan, m, p.strategy)
        for i, plan in enumerate(stc):
            if packed and i == 0:
                rots |= _level_rotations(plan, 2 * n, p.strategy, shift=n)
            else:
                rots |= _level_rotations(plan, n, p.strategy)
        rots.update(_subsum_rotations(spec, int(log_n)))
        rots.add(2 * (1 << int(log_n)) - 1)
    return Requirements(rotations=tuple(sorted(rots)))


@dataclass
class _Level:
    name: str
    plan: LevelPlan
    limbs: int          # limbs of the ciphertext entering the level
    primes: int         # primes dropped after the MAC
    pt_scale: float     # encoding scale of the diagonals
    out_scale: float    # exact scale after the rescales
    period: int = 0     # slot period of the diagonals (0: the program's slots)
    shift: int = 0      # second baby set rot_(o + shift) (packed SlotToCoeff input)


@dataclass
class BootstrapProgram:
    """Prepared constants and schedule (reference program object:
    ``.constants.set_cache_mode``, ``.spec.slots``)."""

    spec: BootstrapSpec
    context: object
    evalmod: BootstrapParams
    coefficients: np.ndarray
    cheb_depth: int
    step: int
    raise_limbs: int
    target_ratio: float          # Delta' / q_0
    cts: list = field(default_factory=list)
    stc: list = field(default_factory=list)
    ladder: cheb.Ladder | None = None
    constants: fhe.ConstantBundle | None = None
    output_limbs: int = 0
    subsum: list = field(default_factory=list)  # sub-sum rotations (sparse programs)
    read_scale: float = 0.0                     # scale the CoeffToSlot input is read at
    packed: bool = False                        # one EvalMod on the 2n-periodic vector

    @property
    def depth_limbs(self) -> int:
        return self.raise_limbs - self.output_limbs

    def release(self) -> None:
        if self.constants is not None:
            self.constants.clear_cache()


def _evalmod_coefficients(p: BootstrapParams) -> np.ndarray:
    period = 2.0 ** p.double_angles

    def f(y):
        return math.cos(2.0 * math.pi * (p.K * y - 0.25) / period)

    grid = np.cos(np.linspace(0.0, math.pi, 4001))
    for degree in range(16, 160):
        c = cheb.chebyshev_coefficients(f, -1.0, 1.0, degree)
        err = np.abs(cheb.evaluate_direct(grid, c) - np.cos(
            2.0 * math.pi * (p.K * grid - 0.25) / period)).max()
        if err < 2.0 ** -p.fit_bits:
            return c
    raise ValueError("EvalMod interpolant does not reach the requested precision")


def _plan_cts_drops(n_levels: int, s_bits: float, prime_bits: float, top_bits: float,
                    pt_bits: float) -> list[int]:
    """Primes dropped after each CoeffToSlot level: intermediate levels keep
    their diagonals at 2^pt_bits and the data scale under the cap; the last
    drops as many primes as it takes to land on the EvalMod ladder with its
    own diagonals at 2^pt_bits or finer."""
    drops = []
    for i in range(n_levels):
        if i == n_levels - 1:
            d = 1
            while top_bits + d * prime_bits - s_bits < pt_bits - 0.5:
                d += 1
        else:
            d = 1
            while s_bits + pt_bits - d * prime_bits > _CTS_CAP_BITS:
                d += 1
            s_bits += pt_bits - d * prime_bits
        drops.append(d)
    return drops


def generate(context, spec: BootstrapSpec, evalmod: BootstrapParams | None = None
             ) -> BootstrapProgram:
    """Plan the program for ``context``'s chain, make sure its rotation keys
    exist, and register its diagonals (encoded on first use; cached with
    cache mode "plain") (reference bootstrap.py:113-148)."""
    ctx = getattr(context, "context", context)
    _check_spec(spec, ctx.logN)
    p = evalmod or BootstrapParams()
    primes = [int(q) for q in ctx.primes()[: ctx.L]]
    n = 1 << _transform_log_slots(spec, ctx.logN)
    bits = math.log2(primes[1]) if len(primes) > 1 else math.log2(primes[0])
    step = max(1, math.ceil(_EVALMOD_BITS / bits))
    coeffs = _evalmod_coefficients(p)
    depth = cheb.chebyshev_depth(coeffs)
    if p.strategy not in ("normal", "ext_normal", "ext_double_hoist"):
        raise ValueError(f"unknown linear-level strategy {p.strategy!r}")
    cts_plans, stc_plans = _plans(spec, p, ctx.logN)
    n_cts, n_stc = len(cts_plans), len(stc_plans)
    ladder_levels = depth + p.double_angles
    q0 = float(primes[0])
    s0 = 2.0 * p.K * q0  # scale the raised ciphertext is read at
    # the sub-sum multiplies the kept coefficients by gap = N / 2n: the first
    # CoeffToSlot level's diagonals carry 1 / gap, so the scale plan and the
    # level count are those of the full-slot program
    gap = (ctx.N // 2) // n
    drops = _plan_cts_drops(n_cts, math.log2(s0), bits, step * bits, p.cts_pt_bits)
    cost = sum(drops) + step * ladder_levels + step + (n_stc - 1)
    T = int(spec.output_levels) + 1 + cost
    if T > ctx.L:
        raise ValueError(
            f"output_levels={spec.output_levels} needs {T} limbs (program depth {cost} "
            f"limbs); the chain has {ctx.L}")

    prog = BootstrapProgram(spec=spec, context=ctx, evalmod=p, coefficients=coeffs,
                            cheb_depth=depth, step=step, raise_limbs=T,
                            target_ratio=2.0 ** -p.ratio_bits,
                            subsum=_subsum_rotations(spec, ctx.logN), read_scale=s0,
                            packed=_packed(spec, ctx.logN, p))
    vectors = {}
    mask_a, mask_d1, mask_d2 = _packing_masks(n)

    # CoeffToSlot: the last level lands on the ladder top
    top = T - sum(drops)
    ladder = cheb.Ladder(primes, top, math.prod(float(q) for q in primes[top - step: top]),
                         step, ladder_levels)
    scale = s0
    limbs = T
    for i, (plan, d) in enumerate(zip(cts_plans, drops)):
        div = math.prod(float(q) for q in primes[limbs - d: limbs])
        if i == n_cts - 1:
            want = ladder.scale[0]
            w = want * div / scale
        else:
            w = 2.0 ** p.cts_pt_bits
            want = scale * w / div
        name = f"cts{i}"
        factor = 1.0 / gap if i == 0 else 1.0
        if prog.packed and i == n_cts - 1:
            # the last level also multiplies its output by the packing mask a
            vectors[name] = fhe.PackedRaw(_period_rows(plan, n, 2 * n, out_mask=mask_a,
                                                       scale_factor=factor))
            prog.cts.append(_Level(name, plan, limbs, d, w, want, period=2 * n))
        else:
            vectors[name] = fhe.PackedRaw(plan.plaintext_rows(n, factor))
            prog.cts.append(_Level(name, plan, limbs, d, w, want))
        scale, limbs = want, limbs - d
    prog.ladder = ladder

    # SlotToCoeff: the first level drops `step` primes (back from the
    # EvalMod scale), the last lands on 2^dcrt_bits
    limbs = ladder.limbs[-1]
    scale = ladder.scale[-1]
    fold = 1.0 / (2.0 * math.pi * prog.target_ratio)
    for i, plan in enumerate(stc_plans):
        drop = step if i == 0 else 1
        div = math.prod(float(q) for q in primes[limbs - drop: limbs])
        want = ctx.scale_at(limbs - drop) if i == n_stc - 1 else _STC_SCALE
        w = want * div / scale
        name = f"stc{i}"
        if prog.packed and i == 0:
            # the first level reads u = d1 s + d2 rot_n(s) from EvalMod's
            # 2n-periodic output s: two baby sets, rot_o(s) and rot_(o+n)(s)
            vectors[name] = fhe.PackedRaw(_period_rows(plan, n, 2 * n,
                                                       in_masks=(mask_d1, mask_d2),
                                                       scale_factor=fold))
            prog.stc.append(_Level(name, plan, limbs, drop, w, want, period=2 * n, shift=n))
        else:
            vectors[name] = fhe.PackedRaw(plan.plaintext_rows(n, fold if i == 0 else 1.0))
            prog.stc.append(_Level(name, plan, limbs, drop, w, want))
        scale, limbs = want, limbs - drop
    prog.output_limbs = limbs
    assert limbs == int(spec.output_levels) + 1, (limbs, spec.output_levels)
    prog.constants = fhe.ConstantBundle(vectors, cache_mode="plain")

    need = [r for r in requirements(spec, ctx.logN, p).rotations if not ctx.has_rotation_key(r)]
    if need:
        ctx.generate_rotation_keys(need)
    return prog


# ---------------------------------------------------------------------------
# evaluation
# ---------------------------------------------------------------------------


def _drop(ct, limbs: int, ctx):
    return fhe.align_to(ct, ct.state.replace(cur_limbs=limbs, scaling_factor=None), ctx)


def _prescale(ct, prog: BootstrapProgram, ctx):
    """One-limb ciphertext whose message scale is Delta' (close to
    target_ratio q_0); returns it and Delta' / (target_ratio q_0)."""
    q0 = float(ctx.primes()[0])
    want = prog.target_ratio * q0
    s = float(ct.state.scaling_factor)
    limbs = int(ct.state.cur_limbs)
    c = round(want / s)
    if c >= 1:
        x = _drop(ct, 1, ctx)
        if c > 1:
            enc = fhe.encode_scalar(int(c), 1, scale_degree=0, mode="integer", context=ctx)
            x = fhe.homo_mul_scalar(x, enc, ctx)
        return x, s * c / want
    if limbs < 2:
        raise ValueError("input scale exceeds q_0 2^-ratio_bits and no limb is left to rescale")
    q1 = float(ctx.primes()[1])
    c = round(want * q1 / s)
    x = _drop(ct, 2, ctx)
    enc = fhe.encode_scalar(int(c), 2, scale_degree=0, mode="integer", context=ctx)
    x = fhe.rescale(fhe.homo_mul_scalar(x, enc, ctx), ctx)
    return x, s * c / q1 / want


def _program_slots(prog: BootstrapProgram) -> int:
    return 1 << int(prog.spec.log_slots)


def input_limbs(context, params: "BootstrapParams | None" = None) -> int:
    """Limbs a bootstrap input needs at the chain's one-limb scale: one when
    that scale is at most 2^-ratio_bits q_0 (an integer multiply then brings
    the message to it), two when it is larger (the prescale rescales by q_1:
    chains whose primes are about as wide as q_0)."""
    ctx = getattr(context, "context", context)
    p = params or BootstrapParams()
    want = 2.0 ** -p.ratio_bits * float(ctx.primes()[0])
    return 1 if round(want / float(ctx.scale_at(1))) >= 1 else 2


def _level_layout(lv: _Level, prog: BootstrapProgram) -> tuple[int, list[int], int]:
    """(slot period, baby rotations, giant rotation) of a linear level."""
    m = lv.period or _program_slots(prog)
    return m, _baby_offsets(lv.plan, m, lv.shift), _giant_offset(lv.plan, m)


def _linear_level(x, lv: _Level, prog: BootstrapProgram, ctx):
    m, babies, giant = _level_layout(lv, prog)
    ext = prog.evalmod.strategy != "normal"
    state = fhe.CipherState(cur_limbs=lv.limbs, scale_degree=1, scaling_factor=lv.pt_scale)
    pts = prog.constants.plaintext(lv.name, state=state, slots=m, context=ctx, is_ext=ext)
    acc = fhe.hoisted_mac_sum(x, babies, pts, giant, lv.plan.giant, ctx,
                              strategy=prog.evalmod.strategy)
    if lv.primes:
        acc = fhe.rescale_many([acc], ctx, primes=lv.primes)[0]
    acc.set_scale(lv.out_scale, 1)
    return acc


def _subsum_many(xs: list, prog: BootstrapProgram, ctx) -> list:
    """x <- x + rot(x, r) for the program's sub-sum rotations, on every
    ciphertext of the batch (one batched key switch per rotation)."""
    for r in prog.subsum:
        rot = fhe.homo_rotate_many(xs, int(r), ctx)
        nxt = fhe.homo_add_many(xs, rot, ctx)
        for a, b in zip(xs, rot):
            a.release()
            b.release()
        xs = nxt
    return xs


def _evalmod(ops: cheb.LadderOps, y: cheb.LCt, prog: BootstrapProgram) -> cheb.LCt:
    c = cheb.evaluate(ops, y, prog.coefficients)
    for _ in range(prog.evalmod.double_angles):
        c = ops.add_const(ops.double(ops.mul(c, c)), -1.0)
    return c


def bootstrap(ct, context, program: BootstrapProgram):
    """Refreshed copy of ``ct`` with output_levels + 1 limbs; ``ct`` is not
    consumed (reference bootstrap.py:370)."""
    prog = program
    ctx = getattr(context, "context", context)
    if ct.degree != 1 or ct.is_ext:
        raise ValueError("bootstrap expects a degree-1 Q-basis ciphertext")
    if int(ct.slots) != prog.spec.slots:
        raise ValueError(f"bootstrap input slots={ct.slots} != program slots={prog.spec.slots}")
    x, ratio = _prescale(ct, prog, ctx)
    x = fhe.mod_raise(x, prog.raise_limbs, ctx)
    x = _subsum_many([x], prog, ctx)[0]
    x.set_scale(prog.read_scale, 1)
    for lv in prog.cts:
        x = _linear_level(x, lv, prog, ctx)

    ops = cheb.LadderOps(ctx, prog.ladder)
    y = cheb.LCt(x, 0)
    yc = cheb.LCt(fhe.homo_rotate(x, 2 * ctx.N - 1, ctx), 0)
    re = ops.add(y, yc)
    if prog.packed:
        # 2 Re on the first n slots of each 2n, 2 Im on the next n
        del y, yc, x
        u = _evalmod(ops, re, prog).ct
    else:
        im = cheb.LCt(fhe.homo_mul_i(ops.add(y, yc, sign=-1.0).ct, ctx, negative=True), 0)
        del y, yc, x
        s_re = _evalmod(ops, re, prog)
        s_im = _evalmod(ops, im, prog)
        u = fhe.homo_add(s_re.ct, fhe.homo_mul_i(s_im.ct, ctx), ctx)
        del s_re, s_im
    for lv in prog.stc:
        u = _linear_level(u, lv, prog, ctx)
    u.set_scale(prog.stc[-1].out_scale * ratio, 1)
    return u


def _linear_level_many(xs: list, lv: _Level, prog: BootstrapProgram, ctx) -> list:
    if prog.evalmod.strategy == "normal":
        return [_linear_level(x, lv, prog, ctx) for x in xs]
    m, babies, giant = _level_layout(lv, prog)
    state = fhe.CipherState(cur_limbs=lv.limbs, scale_degree=1, scaling_factor=lv.pt_scale)
    pts = prog.constants.plaintext(lv.name, state=state, slots=m, context=ctx, is_ext=True)
    accs = fhe.hoisted_mac_sum_ext_many(xs, babies, pts, giant, lv.plan.giant, ctx,
                                        strategy=prog.evalmod.strategy)
    if lv.primes:
        accs = fhe.rescale_many(accs, ctx, primes=lv.primes)
    for a in accs:
        a.set_scale(lv.out_scale, 1)
    return accs


def _bootstrap_group(cts: list, ctx, prog: BootstrapProgram) -> list:
    xs, ratios = [], []
    for ct in cts:
        if ct.degree != 1 or ct.is_ext:
            raise ValueError("bootstrap expects degree-1 Q-basis ciphertexts")
        if int(ct.slots) != prog.spec.slots:
            raise ValueError(f"bootstrap input slots={ct.slots} != program slots={prog.spec.slots}")
        x, ratio = _prescale(ct, prog, ctx)
        xs.append(fhe.mod_raise(x, prog.raise_limbs, ctx))
        ratios.append(ratio)
    xs = _subsum_many(xs, prog, ctx)
    for x in xs:
        x.set_scale(prog.read_scale, 1)
    for lv in prog.cts:
        xs = _linear_level_many(xs, lv, prog, ctx)
    ops = cheb.BatchLadderOps(ctx, prog.ladder)
    conj = fhe.homo_rotate_many(xs, 2 * ctx.N - 1, ctx)
    y, yc = cheb.LCt(xs, 0), cheb.LCt(conj, 0)
    re = ops.add(y, yc)
    if prog.packed:
        # real and imaginary parts share each ciphertext's 2n-periodic vector
        del xs, conj, y, yc
        u = _evalmod(ops, re, prog).ct
    else:
        im = [fhe.homo_mul_i(d, ctx, negative=True) for d in ops.add(y, yc, sign=-1.0).ct]
        del xs, conj, y, yc
        k = len(cts)
        # real and imaginary parts of the whole group run through EvalMod together
        s = _evalmod(ops, cheb.LCt(re.ct + im, 0), prog).ct
        mi = [fhe.homo_mul_i(s[k + i], ctx) for i in range(k)]
        u = fhe.homo_add_many(s[:k], mi, ctx)
        for x in mi:
            x.release()
        del s, mi
    for lv in prog.stc:
        u = _linear_level_many(u, lv, prog, ctx)
    for x, r in zip(u, ratios):
        x.set_scale(prog.stc[-1].out_scale * r, 1)
    return u


def bootstrap_many(cts, context, program: BootstrapProgram, group: int = 16) -> list:
    """Refreshed copies of several ciphertexts, ``group`` at a time: every
    key switch of a group runs as one batched launch that reads its key once,
    and EvalMod evaluates the group's real and imaginary parts as one batch.
    Identical results to ``bootstrap`` per ciphertext."""
    ctx = getattr(context, "context", context)
    cts = list(cts)
    out: list = []
    for i0 in range(0, len(cts), max(1, int(group))):
        out.extend(_bootstrap_group(cts[i0: i0 + max(1, int(group))], ctx, program))
    return out


def bootstrap_pair(real_a, real_b, context, program: BootstrapProgram):
    """Two real-valued ciphertexts refreshed by one bootstrap: a + i b is
    bootstrapped and split by one conjugation (reference
    operators/norm/refresh.py:33-67).  The split yields 2a and 2b; the
    factor 2 is taken out of the recorded scale, so no level is spent."""
    ctx = getattr(context, "context", context)
    packed = fhe.homo_add(real_a, fhe.homo_mul_i(real_b, ctx), ctx)
    value = bootstrap(packed, ctx, program)
    conj = fhe.homo_rotate(value, 2 * ctx.N - 1, ctx)
    twice_a = fhe.homo_add(value, conj, ctx)
    twice_b = fhe.homo_mul_i(fhe.homo_sub(conj, value, ctx), ctx)
    for t in (twice_a, twice_b):
        t.set_scale(2.0 * float(t.state.scaling_factor), 1)
    return twice_a, twice_b


def _to_scale(ct, limbs: int, scale: float, value: float, ctx):
    """value * ct on ``limbs`` limbs at exactly ``scale`` (one rescale; ct
    needs more than ``limbs`` limbs)."""
    x = _drop(ct, limbs + 1, ctx)
    q = float(ctx.primes()[limbs])
    w = scale * q / float(x.state.scaling_factor)
    enc = fhe.encode_scalar(float(value), limbs + 1, scaling_factor=w, context=ctx)
    out = fhe.rescale(fhe.homo_mul_scalar(x, enc, ctx), ctx)
    out.set_scale(scale, 1)
    return out


def bootstrap_iterated(ct, context, program: BootstrapProgram, iterations: int = 2,
                       precision_bits: int = 8):
    """Two-pass (Meta-BTS) refresh: B(ct) - 2^-p B(2^p (B(ct) - ct)), which
    removes the first pass's error up to p more bits; one more level is
    consumed (reference operators/nonlinear/bootstrap.py:352-437).  Scales are
    aligned exactly (not within the fixed-scale tolerance), so the gain is not
    capped by prime drift."""
    ctx = getattr(context, "context", context)
    if int(iterations) not in (1, 2):
        raise ValueError("bootstrap iterations must be one or two")
    first = bootstrap(ct, ctx, program)
    if int(iterations) == 1:
        return first
    limbs = int(ct.state.cur_limbs)
    out_limbs = int(first.state.cur_limbs)
    if out_limbs <= max(limbs, 1):
        raise ValueError("the first pass left no level for the correction")
    s_in = float(ct.state.scaling_factor)
    down = _to_scale(first, limbs, s_in, 1.0, ctx)
    diff = fhe.homo_sub(down, ct, ctx)
    p = int(precision_bits)
    if p > 0:
        enc = fhe.encode_scalar(1 << p, limbs, scale_degree=0, mode="integer", context=ctx)
        diff = fhe.homo_mul_scalar(diff, enc, ctx)
    err = bootstrap(diff, ctx, program)
    s1 = float(first.state.scaling_factor)
    corr = _to_scale(err, out_limbs - 1, s1, 2.0 ** -p, ctx)
    base = _drop(first, out_limbs - 1, ctx)
    base.set_scale(s1, 1)
    return fhe.homo_sub(base, corr, ctx)


__all__ = ["BootstrapParams", "BootstrapProgram", "BootstrapSpec", "Requirements", "bootstrap",
           "bootstrap_iterated", "bootstrap_many", "bootstrap_pair", "generate", "requirements"]
