"""Homomorphic CoeffToSlot / SlotToCoeff as grouped sparse FFT stages.

The slots of a full-packed ciphertext are z_j = m(rho^(g_j)) / scale with
rho = exp(2 pi i / 4n), g_j = 5^j mod 4n and n = N/2, and the complex vector
u_k = m_k + i m_(k+n) is mapped to z by the special FFT

    z = S_L ... S_1 P u,

where P is the bit-reversal permutation and stage S_s (block length
2^s) is the butterfly x_j, x_(j+h) <- x_j + tau x_(j+h), x_j - tau x_(j+h)
with h = 2^(s-1) and tau = rho_s^(5^j mod 2^(s+2)), rho_s = exp(2 pi i / 2^(s+2))
(split k by parity; 5^(n/2) = 1 + 2n mod 4n gives the sign of the odd half).
CoeffToSlot applies S_1^-1 ... S_L^-1 (slots end in bit-reversed order) and
SlotToCoeff applies S_L ... S_1 to that order, so P never has to be
evaluated: EvalMod between them works slot by slot.

Each stage has three diagonals (offsets 0, +h, -h); consecutive stages are
multiplied into one matrix per level (level budget), whose diagonals sit at
multiples of the smallest stage offset.  A level is evaluated as
rot_(-c)(ct) followed by a BSGS diagonal MAC over the shifted offsets, which
is exactly fhe.hoisted_mac_sum's schedule.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np


def stage_diagonals(n: int, s: int, inverse: bool) -> dict[int, np.ndarray]:
    """Diagonals {offset: vector} of S_s (or S_s^-1) on n slots:
    out[i] = sum_off d_off[i] * x[(i + off) mod n]."""
    length = 1 << s
    h = length >> 1
    i = np.arange(n)
    j = i % length
    low = j < h
    jj = np.where(low, j, j - h)
    e = np.array([pow(5, int(t), 4 * length) for t in range(h)], dtype=np.int64)
    tau = np.exp(2j * np.pi * e[jj] / (4 * length))
    d0 = np.zeros(n, dtype=np.complex128)
    dp = np.zeros(n, dtype=np.complex128)
    dm = np.zeros(n, dtype=np.complex128)
    if not inverse:
        # low: x_j + tau x_(j+h); high: x_(j-h) - tau x_j
        d0[low] = 1.0
        dp[low] = tau[low]
        dm[~low] = 1.0
        d0[~low] = -tau[~low]
    else:
        # X = x_j + tau y, Y = x_j - tau y  =>  x = (X + Y)/2, y = (X - Y)/(2 tau)
        d0[low] = 0.5
        dp[low] = 0.5
        dm[~low] = 0.5 / tau[~low]
        d0[~low] = -0.5 / tau[~low]
    out = {0: d0}
    out[h % n] = out.get(h % n, 0) + dp
    out[(-h) % n] = out.get((-h) % n, 0) + dm
    return out


def compose(a: dict[int, np.ndarray], b: dict[int, np.ndarray], n: int) -> dict[int, np.ndarray]:
    """Diagonals of A B: (A B)[i, i + ka + kb] += a_ka[i] b_kb[i + ka]."""
    out: dict[int, np.ndarray] = {}
    for ka, va in a.items():
        for kb, vb in b.items():
            k = (ka + kb) % n
            term = va * np.roll(vb, -ka)
            out[k] = out[k] + term if k in out else term
    return {k: v for k, v in out.items() if np.any(v != 0)}


def apply_diagonals(d: dict[int, np.ndarray], x: np.ndarray) -> np.ndarray:
    return sum(v * np.roll(x, -k) for k, v in d.items())


def level_groups(log_n: int, budget: int) -> list[list[int]]:
    """Stages 1..log_n split into `budget` consecutive groups (sizes differ by
    at most one, larger groups first)."""
    budget = max(1, min(budget, log_n))
    base, extra = divmod(log_n, budget)
    groups, s = [], 1
    for g in range(budget):
        size = base + (1 if g < extra else 0)
        groups.append(list(range(s, s + size)))
        s += size
    return groups


@dataclass
class LevelPlan:
    """One level: diagonals at offsets c + stride * t for t in [0, width),
    evaluated as BSGS with `baby` babies after a pre-rotation by -c."""

    stride: int
    center: int  # pre-rotation amount c (slots), offsets start at -c
    width: int
    baby: int
    giant: int
    diagonals: dict[int, np.ndarray]  # offset (mod n) -> vector

    def rotations(self, n: int) -> set[int]:
        rots = {(-self.center) % n}
        rots.update(self.stride * b for b in range(1, self.baby))
        if self.giant > 1:
            rots.add(self.stride * self.baby)
        return {r % n for r in rots if r % n}

    def plaintext_rows(self, n: int, scale_factor: float = 1.0) -> np.ndarray:
        """Rows p[g B + b] = rot_(-g B stride)(d_(c' + (g B + b) stride)) as
        required by hoisted_mac_sum, times scale_factor."""
        rows = np.zeros((self.giant * self.baby, n), dtype=np.complex128)
        for g in range(self.giant):
            for b in range(self.baby):
                t = g * self.baby + b
                if t >= self.width:
                    continue
                off = (t * self.stride - self.center) % n
                if off in self.diagonals:
                    rows[t] = np.roll(self.diagonals[off], g * self.baby * self.stride)
        return rows * scale_factor


def plan_levels(log_n: int, budget: int, inverse: bool, giants: int = 0) -> list[LevelPlan]:
    """Level plans in evaluation order.  inverse=True is CoeffToSlot
    (S_L^-1 first), inverse=False is SlotToCoeff (S_1 first).  The baby count
    is about sqrt(width); with ``giants`` > 0 it is the smallest power of two
    that needs at most that many giant steps (the extended-basis schedule
    pays one ModDown per giant group, so it wants few giants)."""
    n = 1 << log_n
    groups = level_groups(log_n, budget)
    order = list(reversed(groups)) if inverse else groups
    plans = []
    for grp in order:
        stages = list(reversed(grp)) if inverse else grp
        # matrix of the group: the later-applied stage multiplies on the left
        mat = None
        for s in stages:
            d = stage_diagonals(n, s, inverse)
            mat = d if mat is None else compose(d, mat, n)
        stride = 1 << (min(grp) - 1)
        span = (1 << max(grp)) - stride  # largest |offset|
        if 2 * span + stride > n:
            # offsets cover every multiple of stride modulo n
            span, width = 0, n // stride
        else:
            width = 2 * span // stride + 1
        baby = 1 << max(0, math.ceil(math.log2(width)) // 2 + (math.ceil(math.log2(width)) % 2))
        if giants > 0:
            baby = 1
            while -(-width // baby) > giants:
                baby *= 2
        baby = min(baby, 64)
        giant = -(-width // baby)
        plans.append(LevelPlan(stride=stride, center=span, width=width, baby=baby, giant=giant,
                               diagonals=mat))
    return plans


__all__ = ["LevelPlan", "apply_diagonals", "compose", "level_groups", "plan_levels",
           "stage_diagonals"]
