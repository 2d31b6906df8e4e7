"""Causal multi-head attention on feature-major ciphertexts (the role of the
reference's C/Delta attention, llama3fhe/operators/attention/qk.py,
softmax.py, pv.py; its plaintext references approx/attention.py:134-203).

Layouts.  T tokens in n = T / L ciphertexts of L token lanes (feature-major:
slot ``f L + l`` of ciphertext c holds feature f of token ``c L + l``); H
heads of hd features (feature ``h hd + d``), T <= hd.  Scores and
probabilities use the *score layout*: ciphertext c (the query tokens of
ciphertext c) holds ``S[h, i, (i + delta) mod T]`` at slot
``(h hd + delta) L + l`` for ``i = c L + l`` -- the key offset delta takes the
place of the feature inside each head block.

QK.  The key stream shifted by delta tokens, ``K^(delta)_c[f L + l] =
K[(c L + l + delta) mod T, f]``, is ``K^(r)`` of ciphertext ``(c + a) mod n``
for ``delta = a L + r``; ``K^(r)`` is a lane shift with carry into the next
ciphertext (two rotations and two masks).  For each query ciphertext and
delta, ``Q_c * K^(delta)_c`` holds the per-feature products; their sums over
each head's hd features come from a rotate-and-add tree, run in groups of L
offsets: for offset r of a group, the sum of L consecutive features of its
product lands on the features ``= r mod L`` (one extended-basis hoisted MAC
over the L rotations ``(e - r) L``, the mask in its plaintexts, batched over
the groups), the remaining log2(hd / L) tree steps, and a final mask-and-shift
that places group a at feature offsets ``a L .. a L + L - 1``.  Depth:
lane-shift mask, product, MAC mask, merge mask.

Softmax ("Algorithm 2", softmax.py:648-1262).  ``y = exp((s - U) / 2^k)`` by a
Chebyshev series (its domain map folded into the last QK mask), causal mask,
then k rounds of ``y <- y^2 / sum_row y^2``: after k rounds
``y = exp(s) / sum exp(s)``.  Each round's row sums are packed into one slim
ciphertext (the RMSNorm packing: row c at feature offset c), normalised by
the public count of valid keys, inverted by one series evaluation for all
rows (``1/x`` on a narrow interval), optionally refreshed by a bootstrap, and
broadcast back over the head blocks.  The main stream loses two levels per
round.

PV.  ``O_c = sum_delta B_delta(P_c) * V^(delta)_c`` where ``B_delta`` spreads
the probabilities of offset delta over the head's hd features;
``V^(delta)`` is the shifted value stream built like ``K^(delta)``.  The
spread runs in groups of L offsets (one hoisted rotation per group, a tree
over strides of L features, and extended-basis MACs whose masks fill the
rest; see pv_output).  The products are summed as degree-2 ciphertexts and
relinearised once per query ciphertext.  Depth: mask, MAC, product.

Grouped-query attention uses key/value projections whose rows are repeated
for the query heads of each group (``kv_repeat_rows``): the streams then
carry H heads like the queries.
"""

from __future__ import annotations

import time
from dataclasses import dataclass, field

import numpy as np

from easyfhe import fhe

from .layout import FeatureMajorPrefillLayout


def _ctx(context):
    return getattr(context, "context", context)


def _release(values) -> None:
    for v in values or ():
        if v is not None:
            v.release()


def _log2(v: int, name: str) -> int:
    v = int(v)
    if v <= 0 or v & (v - 1):
        raise ValueError(f"{name}={v} must be a power of two.")
    return v.bit_length() - 1


@dataclass(frozen=True)
class AttentionGeometry:
    """Token/head geometry of one attention over a feature-major stream."""

    layout: FeatureMajorPrefillLayout
    heads: int
    head_dim: int

    def __post_init__(self) -> None:
        L, T = self.lanes, int(self.layout.seq_len)
        _log2(self.head_dim, "head_dim")
        _log2(L, "token lanes")
        if int(self.heads) * int(self.head_dim) != int(self.layout.hidden_dim):
            raise ValueError("heads * head_dim must equal the hidden width.")
        if T % L:
            raise ValueError("seq_len must fill whole ciphertexts.")
        if T > int(self.head_dim):
            raise ValueError("the score layout needs seq_len <= head_dim.")
        if L > int(self.head_dim):
            raise ValueError("token lanes must not exceed head_dim.")

    @property
    def lanes(self) -> int:
        return int(self.layout.tokens_per_cipher)

    @property
    def ciphers(self) -> int:
        return int(self.layout.cipher_count)

    @property
    def seq_len(self) -> int:
        return int(self.layout.seq_len)

    @property
    def slots(self) -> int:
        return int(self.layout.slots)

    # -- masks ---------------------------------------------------------------
    def lane_mask(self, r: int) -> np.ndarray:
        """1 on lanes l < L - r (the lanes a shift by r keeps in place)."""
        lanes = np.arange(self.slots) % self.lanes
        return (lanes < self.lanes - int(r)).astype(np.float64)

    def feature_mask(self, modulus: int, below: int, value: float = 1.0) -> np.ndarray:
        """``value`` on features f with ``f mod modulus < below``."""
        f = np.arange(self.slots) // self.lanes
        return np.where((f % int(modulus)) < int(below), float(value), 0.0)

    def residue_mask(self, modulus: int, residue: int) -> np.ndarray:
        """1 on features f with ``f mod modulus == residue``."""
        f = np.arange(self.slots) // self.lanes
        return ((f % int(modulus)) == int(residue)).astype(np.float64)

    def causal_mask(self, c: int) -> np.ndarray:
        """Score-layout validity of query ciphertext c: key (i + delta) mod T
        is at most i (delta = 0, or the offset wraps past T)."""
        L, T, hd = self.lanes, self.seq_len, int(self.head_dim)
        s = np.arange(self.slots)
        f, l = s // L, s % L
        delta = f % hd
        i = int(c) * L + l
        return ((delta < T) & ((delta == 0) | (i + delta >= T))).astype(np.float64)

    def valid_counts(self, c: int) -> np.ndarray:
        """Valid keys of each lane's query token: i + 1."""
        return int(c) * self.lanes + np.arange(self.lanes) + 1.0

    # -- score layout (host side, for callers and tests) ------------------------
    def pack_scores(self, scores: np.ndarray) -> np.ndarray:
        """[H, T, T] -> [n, slots] in the score layout."""
        L, T, hd = self.lanes, self.seq_len, int(self.head_dim)
        out = np.zeros((self.ciphers, self.slots))
        for c in range(self.ciphers):
            for l in range(L):
                i = c * L + l
                for h in range(int(self.heads)):
                    d = np.arange(T)
                    out[c, (h * hd + d) * L + l] = scores[h, i, (i + d) % T]
        return out

    def unpack_scores(self, packed: np.ndarray) -> np.ndarray:
        L, T, hd = self.lanes, self.seq_len, int(self.head_dim)
        out = np.zeros((int(self.heads), T, T))
        for c in range(self.ciphers):
            for l in range(L):
                i = c * L + l
                for h in range(int(self.heads)):
                    d = np.arange(T)
                    out[h, i, (i + d) % T] = packed[c, (h * hd + d) * L + l]
        return out


def kv_repeat_rows(weight: np.ndarray, *, query_heads: int, kv_heads: int,
                   head_dim: int) -> np.ndarray:
    """``[kv_heads * hd, D] -> [query_heads * hd, D]``: query head h reads
    key/value head ``h // (query_heads / kv_heads)`` (approx/attention.py:134-150)."""
    w = np.asarray(weight)
    if w.shape[0] != int(kv_heads) * int(head_dim):
        raise ValueError("key/value weight rows must be kv_heads * head_dim.")
    if int(query_heads) % int(kv_heads):
        raise ValueError("query heads must be a multiple of key/value heads.")
    g = int(query_heads) // int(kv_heads)
    heads = w.reshape(int(kv_heads), int(head_dim), -1)
    return np.repeat(heads, g, axis=0).reshape(int(query_heads) * int(head_dim), -1)


# ---------------------------------------------------------------------------
# rotation keys
# ---------------------------------------------------------------------------


def qk_rotations(geo: AttentionGeometry) -> set[int]:
    L, hd = geo.lanes, int(geo.head_dim)
    keys = set()
    for r in range(1, L):
        keys.update((r, r - L, r * L, -r * L))
    keys.update(L << b for b in range(_log2(hd, "head_dim")))
    keys.update(-a * L * L for a in range(1, geo.ciphers))
    return {k for k in keys if k}


def softmax_rotations(geo: AttentionGeometry) -> set[int]:
    L, hd = geo.lanes, int(geo.head_dim)
    keys = {L << b for b in range(_log2(hd, "head_dim"))}
    keys.update(-(L << b) for b in range(_log2(hd, "head_dim")))
    keys.update(s * c * L for c in range(1, geo.ciphers) for s in (1, -1))
    return keys


def pv_rotations(geo: AttentionGeometry) -> set[int]:
    L, hd = geo.lanes, int(geo.head_dim)
    keys = {a * L * L for a in range(1, -(-geo.seq_len // L))}
    keys.update(-(L * L << b) for b in range(_log2(hd // L, "head_dim / lanes")))
    for r in range(1, L):
        keys.update((r, r - L, -r * L))
    return keys


def attention_rotations(geo: AttentionGeometry) -> tuple[int, ...]:
    return tuple(sorted(qk_rotations(geo) | softmax_rotations(geo) | pv_rotations(geo)))


# ---------------------------------------------------------------------------
# building blocks
# ---------------------------------------------------------------------------


def _encode(ctx, rows, limbs: int, scale: float | None = None) -> list:
    rows = np.atleast_2d(np.asarray(rows, dtype=np.float64))
    return fhe.encode_rows_cached(ctx, rows, limbs=int(limbs),
                                  scale=float(scale) if scale else ctx.scale_at(int(limbs)),
                                  slots=ctx.max_slots)


def _encode_ext(ctx, rows, limbs: int) -> list:
    rows = np.atleast_2d(np.asarray(rows, dtype=np.float64))
    return fhe.encode_rows_cached(ctx, rows, limbs=int(limbs), scale=ctx.scale_at(int(limbs)),
                                  slots=ctx.max_slots, is_ext=True)


def _mul_pt_rescale(cts, pts, ctx) -> list:
    """ct_i * pt_i (or one shared pt), then one batched rescale."""
    pts = list(pts)
    prods = [fhe.homo_mul_pt(c, pts[i] if len(pts) > 1 else pts[0], ctx)
             for i, c in enumerate(cts)]
    try:
        return fhe.rescale_many(prods, ctx)
    finally:
        _release(prods)


def _rotate_add_tree(cts, strides, ctx) -> list:
    """x <- x + rot(x, s) for each stride, all ciphertexts per batched call."""
    cur, owned = list(cts), False
    for s in strides:
        rot = []
        for i in range(0, len(cur), 64):
            rot.extend(fhe.homo_rotate_many(cur[i: i + 64], int(s), ctx))
        nxt = fhe.homo_add_many(cur, rot, ctx)
        _release(rot)
        if owned:
            _release(cur)
        cur, owned = nxt, True
    return cur if owned else [c.deep_copy() for c in cur]


def _rotate_many(cts, rotation: int, ctx) -> list:
    if int(rotation) == 0:
        return [c.deep_copy() for c in cts]
    out = []
    for i in range(0, len(cts), 64):
        out.extend(fhe.homo_rotate_many(cts[i: i + 64], int(rotation), ctx))
    return out


def _mul_relin_rescale(left, right, ctx) -> list:
    out = []
    for i in range(0, len(left), 64):
        out.extend(fhe.homo_mul_relin_rescale_many(left[i: i + 64], right[i: i + 64], ctx))
    return out


def lane_shifts(stream, geo: AttentionGeometry, *, crypto_context) -> list:
    """``shifted[r][c][f L + l] = X[(c L + l + r) mod T, f]`` for r < L: the
    token shift by r of every ciphertext, lanes past the end carried over
    from the next ciphertext (one mask level).  ``shifted[0]`` are copies at
    the same level as the others."""
    ctx = _ctx(crypto_context)
    xs = list(stream)
    n, L = geo.ciphers, geo.lanes
    limbs = int(xs[0].state.cur_limbs)
    out = []
    for r in range(L):
        if r == 0:
            one = _encode(ctx, np.ones(geo.slots), limbs)
            out.append(_mul_pt_rescale(xs, one, ctx))
            _release(one)
            continue
        keep = _rotate_many(xs, r, ctx)
        carry = _rotate_many([xs[(c + 1) % n] for c in range(n)], r - L, ctx)
        pk = _encode(ctx, geo.lane_mask(r), limbs)
        pc = _encode(ctx, 1.0 - geo.lane_mask(r), limbs)
        a = _mul_pt_rescale(keep, pk, ctx)
        b = _mul_pt_rescale(carry, pc, ctx)
        _release(keep + carry + pk + pc)
        out.append(fhe.homo_add_many(a, b, ctx))
        _release(a + b)
    return out


def _shifted(shifts, geo: AttentionGeometry, c: int, delta: int):
    a, r = divmod(int(delta), geo.lanes)
    return shifts[r][(int(c) + a) % geo.ciphers]


@dataclass
class StageResult:
    ciphers: tuple
    stage_seconds: dict = field(default_factory=dict)

    def release(self) -> None:
        _release(self.ciphers)
        self.ciphers = ()


def qk_scores(query, key, geo: AttentionGeometry, *, crypto_context,
              output_scale: float = 1.0, output_offset: float = 0.0) -> StageResult:
    """Score layout of ``output_scale * Q K^T + output_offset`` (per head,
    every key offset; the causal mask is applied by the softmax).  Query and
    key streams are not consumed and must share one level.  The outputs land
    exactly on the scale of the prime below their last one, where a series
    evaluated on them starts its ladder."""
    ctx = _ctx(crypto_context)
    qs, ks = list(query), list(key)
    n, L, hd, T = geo.ciphers, geo.lanes, int(geo.head_dim), geo.seq_len
    if len(qs) != n or len(ks) != n:
        raise ValueError(f"QK expects {n} query and key ciphertexts.")
    sb, hb = _log2(L, "lanes"), _log2(hd, "head_dim")
    stage = {}
    sync = ctx.synchronize
    t0 = time.perf_counter()
    shifts = lane_shifts(ks, geo, crypto_context=ctx)
    # the queries meet the shifted keys at the shifts' level
    lk = int(shifts[0][0].state.cur_limbs)
    qa = [fhe.align_to(q, q.state.replace(cur_limbs=lk, scaling_factor=None), ctx) for q in qs]
    sync()
    stage["key_shifts"] = time.perf_counter() - t0
    groups = -(-T // L)
    zs = []  # per query ciphertext, per group a: head sums at offsets r < L
    t0 = time.perf_counter()
    try:
        for c in range(n):
            prods = _mul_relin_rescale([qa[c]] * (groups * L),
                                       [_shifted(shifts, geo, c, d) for d in range(groups * L)],
                                       ctx)
            lp = int(prods[0].state.cur_limbs)
            # group a interleaves its L offsets r at features = r mod L, each
            # holding the sum of L consecutive features of its product:
            #   Y_a = sum_r mask_r * sum_e rot(P_(a L + r), (e - r) L)
            # one extended-basis hoisted MAC per r over all groups (one ModUp,
            # L key inner products and one ModDown per product; the mask rides
            # in the MAC's plaintexts)
            acc = None
            for r in range(L):
                pt = _encode_ext(ctx, geo.residue_mask(L, r), lp)
                try:
                    m = fhe.hoisted_mac_sum_ext_many(
                        [prods[a * L + r] for a in range(groups)],
                        [(e - r) * L for e in range(L)], pt * L, 0, 1, ctx)
                finally:
                    _release(pt)
                if acc is None:
                    acc = m
                else:
                    nxt = fhe.homo_add_many(acc, m, ctx)
                    _release(acc + m)
                    acc = nxt
            _release(prods)
            packed = fhe.rescale_many(acc, ctx)
            _release(acc)
            zs.append(_rotate_add_tree(packed, [L << b for b in range(sb, hb)], ctx))
            _release(packed)
        sync()
        stage["products_and_head_sums"] = time.perf_counter() - t0
        t0 = time.perf_counter()
        lz = int(zs[0][0].state.cur_limbs)
        target = float(int(ctx.primes()[lz - 2]))
        mscale = target * float(int(ctx.primes()[lz - 1])) / float(zs[0][0].state.scaling_factor)
        mr = _encode(ctx, geo.feature_mask(hd, L, output_scale), lz, mscale)
        out = []
        for c in range(n):
            sel = _mul_pt_rescale(zs[c], mr, ctx)
            acc = sel[0]
            for a in range(1, groups):
                y = fhe.homo_rotate(sel[a], -a * L * L, ctx)
                nxt = fhe.homo_add(acc, y, ctx)
                acc.release()
                y.release()
                acc = nxt
            _release(sel[1:])
            if output_offset:
                enc = fhe.encode_scalar(float(output_offset), int(acc.state.cur_limbs),
                                        scaling_factor=float(acc.state.scaling_factor),
                                        context=ctx)
                nxt = fhe.homo_add_scalar(acc, enc, ctx)
                acc.release()
                enc.release()
                acc = nxt
            out.append(acc)
        _release(mr)
        sync()
        stage["merge"] = time.perf_counter() - t0
        return StageResult(tuple(out), stage)
    finally:
        for z in zs:
            _release(z)
        for s in shifts:
            _release(s)
        _release([a for a, q in zip(qa, qs) if a is not q])


@dataclass(frozen=True)
class SoftmaxConfig:
    """Algorithm-2 softmax constants (the role of the reference's per-layer
    ``U_hat``, ``k`` and polynomial entries, approx/softmax.py:20-99): scores
    are assumed in [-bound, shift]; exp runs on ``(s - shift) / 2^rounds``."""

    rounds: int = 2
    shift: float = 4.0
    bound: float = 4.0
    exp_degree: int = 15
    first_inverse_degree: int = 47
    inverse_degree: int = 63

    def __post_init__(self) -> None:
        if int(self.rounds) < 1:
            raise ValueError("softmax needs at least one round.")
        if not float(self.shift) + float(self.bound) > 0.0:
            raise ValueError("empty score interval.")

    @property
    def exp_low(self) -> float:
        return -(float(self.bound) + float(self.shift)) / float(2 ** int(self.rounds))

    def exp(self) -> dict:
        from .approx import exp_entry

        return exp_entry(1.02 * self.exp_low, 0.0, int(self.exp_degree))

    def first_inverse(self) -> dict:
        """Round 1 normalises the row sum of y0^2 by the valid-key count: the
        mean of y0^2 lies in [exp(2 exp_low), 1]."""
        from .approx import inverse_entry

        return inverse_entry(0.9 * float(np.exp(2.0 * self.exp_low)), 1.05,
                             int(self.first_inverse_degree))

    def inverse(self, seq_len: int) -> dict:
        """Later rounds: y sums to one on its row, so sum y^2 is in [1/T, 1]."""
        from .approx import inverse_entry

        return inverse_entry(0.9 / float(seq_len), 1.05, int(self.inverse_degree))

    def score_map(self, score_scale: float) -> tuple[float, float]:
        """(scale, offset) of the QK output so that it is the exp series'
        mapped input ``alpha (score_scale q.k - shift) / 2^k + beta``."""
        from .approx import chebyshev_map

        a, b = chebyshev_map(self.exp()["fit_interval"])
        k2 = float(2 ** int(self.rounds))
        return float(score_scale) * a / k2, b - a * float(self.shift) / k2


def softmax_depth(cfg: SoftmaxConfig, seq_len: int) -> int:
    from easyfhe.chebyshev import chebyshev_depth

    first = chebyshev_depth(cfg.first_inverse()["coefficients"])
    later = chebyshev_depth(cfg.inverse(seq_len)["coefficients"])
    exp_d = chebyshev_depth(cfg.exp()["coefficients"])
    return exp_d + 1 + (first + 4) + (int(cfg.rounds) - 1) * (later + 4)


def softmax_depth_refreshed(cfg: SoftmaxConfig, seq_len: int,
                            input_limbs: int = 1) -> tuple[int, int]:
    """With every round's normaliser refreshed: (levels the main stream
    consumes, limbs the softmax input needs so that round r's slim
    normaliser keeps ``input_limbs`` limbs after its series, what its
    bootstrap takes).  The main stream
    then loses two levels per round (square, product with the normaliser):
    the inverse series runs on the slim ciphertext, which the refresh lifts
    back above the squares."""
    from easyfhe.chebyshev import chebyshev_depth

    exp_d = chebyshev_depth(cfg.exp()["coefficients"])
    first = chebyshev_depth(cfg.first_inverse()["coefficients"])
    later = chebyshev_depth(cfg.inverse(seq_len)["coefficients"])
    rounds = int(cfg.rounds)
    main = exp_d + 1 + 2 * rounds
    # round r starts exp_d + 1 + 2 r levels down; its slim normaliser is two
    # levels below that and needs the series' depth plus one limb
    need = max(exp_d + 1 + 2 * r + 2 + (first if r == 0 else later) + int(input_limbs)
               for r in range(rounds))
    return main, need


def _slim_active(geo: AttentionGeometry) -> np.ndarray:
    """Slots of the slim normaliser that hold a row sum: ciphertext c's lanes
    at feature offset c of every head block, i.e. slot mod (hd L) < n L."""
    s = np.arange(geo.slots)
    return (s % (int(geo.head_dim) * geo.lanes)) < geo.ciphers * geo.lanes


def _lane_rows(geo: AttentionGeometry, c: int, lane_values, *, modulus: int, below: int):
    """Values per lane on features f with f mod modulus < below."""
    s = np.arange(geo.slots)
    f, l = s // geo.lanes, s % geo.lanes
    vals = np.asarray(lane_values, dtype=np.float64)[l]
    return np.where((f % int(modulus)) < int(below), vals, 0.0)


def softmax_alg2(mapped_scores, geo: AttentionGeometry, cfg: SoftmaxConfig, *, crypto_context,
                 refresh=None) -> StageResult:
    """Causal softmax over each head's keys of score-layout ciphertexts that
    hold the exp series' mapped input (``qk_scores`` with ``cfg.score_map``).
    ``refresh`` (optional) bootstraps the slim normaliser of every round.
    Inputs are not consumed; invalid offsets come out zero."""
    from easyfhe.chebyshev import eval_chebyshev_series_cipher, eval_chebyshev_series_many

    from .approx import chebyshev_map

    ctx = _ctx(crypto_context)
    xs = list(mapped_scores)
    n, L, hd, T = geo.ciphers, geo.lanes, int(geo.head_dim), geo.seq_len
    hb = _log2(hd, "head_dim")
    stage = {}
    sync = ctx.synchronize
    t0 = time.perf_counter()
    y = eval_chebyshev_series_many(xs, cfg.exp()["coefficients"], lower_bound=-1.0,
                                   upper_bound=1.0, crypto_context=ctx,
                                   input_is_chebyshev_mapped=True)
    ly = int(y[0].state.cur_limbs)
    causal = _encode(ctx, np.stack([geo.causal_mask(c) for c in range(n)]), ly)
    masked = _mul_pt_rescale(y, causal, ctx)
    _release(y + causal)
    y = masked
    sync()
    stage["exp"] = time.perf_counter() - t0
    try:
        for r in range(int(cfg.rounds)):
            t0 = time.perf_counter()
            entry = cfg.first_inverse() if r == 0 else cfg.inverse(T)
            alpha, beta = chebyshev_map(entry["fit_interval"])
            weights = [1.0 / geo.valid_counts(c) if r == 0 else np.ones(L) for c in range(n)]
            sq = _mul_relin_rescale(y, y, ctx)
            _release(y)
            y = []
            sums = _rotate_add_tree(sq, [L << b for b in range(hb)], ctx)
            rl = int(sums[0].state.cur_limbs)
            target = float(int(ctx.primes()[rl - 2]))
            pscale = target * float(int(ctx.primes()[rl - 1])) / float(sums[0].state.scaling_factor)
            pack = _encode(ctx, np.stack([_lane_rows(geo, c, alpha * weights[c], modulus=hd,
                                                     below=1) for c in range(n)]), rl, pscale)
            terms = _mul_pt_rescale(sums, pack, ctx)
            _release(sums + pack)
            slim = terms[0]
            for c in range(1, n):
                t = fhe.homo_rotate(terms[c], -c * L, ctx)
                nxt = fhe.homo_add(slim, t, ctx)
                slim.release()
                t.release()
                slim = nxt
            _release(terms[1:])
            # the map's offset on the slots that hold a row sum only: the
            # others stay at 0, the middle of the series' interval, so the
            # series stays bounded there (beta alone maps them just outside
            # [-1, 1], where a degree-47 series reaches hundreds) and a
            # refresh sees only values in its range (the reference fills
            # them too, softmax.py:1020-1031)
            off = _encode(ctx, np.where(_slim_active(geo), beta, 0.0),
                          int(slim.state.cur_limbs), float(slim.state.scaling_factor))
            mapped = fhe.homo_add_pt(slim, off[0], ctx)
            _release([slim] + off)
            inv = eval_chebyshev_series_cipher(mapped, entry["coefficients"], lower_bound=-1.0,
                                               upper_bound=1.0, crypto_context=ctx,
                                               input_is_chebyshev_mapped=True)
            mapped.release()
            if refresh is not None:
                fresh = refresh(inv)
                inv.release()
                inv = fresh
            li = int(inv.state.cur_limbs)
            parts = [inv.deep_copy()] + [fhe.homo_rotate(inv, c * L, ctx) for c in range(1, n)]
            inv.release()
            ext = _encode(ctx, np.stack([_lane_rows(geo, c, weights[c], modulus=hd, below=1)
                                         for c in range(n)]), li)
            sel = _mul_pt_rescale(parts, ext, ctx)
            _release(parts + ext)
            lam = _rotate_add_tree(sel, [-(L << b) for b in range(hb)], ctx)
            _release(sel)
            # a refreshed normaliser may sit above the squares: both go to the
            # lower of the two levels
            tl = min(int(lam[0].state.cur_limbs), int(sq[0].state.cur_limbs))
            sqa = _to_limbs(sq, tl, ctx)
            lama = _to_limbs(lam, tl, ctx)
            y = _mul_relin_rescale(sqa, lama, ctx)
            _release([a for a, b in zip(sqa, sq) if a is not b])
            _release([a for a, b in zip(lama, lam) if a is not b])
            _release(sq + lam)
            sync()
            stage[f"round_{r + 1}"] = time.perf_counter() - t0
        return StageResult(tuple(y), stage)
    except Exception:
        _release(y)
        raise


def _to_limbs(cts, limbs: int, ctx) -> list:
    return [fhe.align_to(c, c.state.replace(cur_limbs=int(limbs), scaling_factor=None), ctx)
            for c in cts]


def pv_output(probs, value, geo: AttentionGeometry, *, crypto_context) -> StageResult:
    """Feature-major ``O[i, h hd + d] = sum_j P[h, i, j] V[j, h hd + d]`` from
    score-layout probabilities (zero at invalid offsets) and a feature-major
    value stream; inputs are not consumed.

    The probabilities of offset ``delta = a L + m`` are spread over their
    head in groups of L offsets: ``G_a = rot(P_c, a L)`` (in features, one
    hoisted rotation per group) masked to each head's first L features, spread
    by the tree over strides ``L 2^b`` (copies at every feature ``= m mod L``),
    then one extended-basis hoisted MAC per m over all groups,
    ``B_(a L + m) = sum_k mask_k * rot(W_a, m - k)`` (features ``= k mod L``
    read the copy at residue m of their own L-block), which fills the
    remaining L - 1 features of each block.  Depth: mask, MAC, product."""
    ctx = _ctx(crypto_context)
    ps, vs = list(probs), list(value)
    n, L, hd, T = geo.ciphers, geo.lanes, int(geo.head_dim), geo.seq_len
    if len(ps) != n or len(vs) != n:
        raise ValueError(f"PV expects {n} probability and value ciphertexts.")
    sb, hb = _log2(L, "lanes"), _log2(hd, "head_dim")
    groups = -(-T // L)
    stage = {}
    sync = ctx.synchronize
    t0 = time.perf_counter()
    shifts = lane_shifts(vs, geo, crypto_context=ctx)
    sync()
    stage["value_shifts"] = time.perf_counter() - t0
    out = []
    t_spread = t_prod = 0.0
    try:
        lp = int(ps[0].state.cur_limbs)
        first = _encode(ctx, geo.feature_mask(hd, L), lp)
        lw = lp - 1
        fill = [_encode_ext(ctx, geo.residue_mask(L, r), lw) for r in range(L)]
        for c in range(n):
            t0 = time.perf_counter()
            rots = fhe.prepare_hoisted_baby_rotations(ps[c], [a * L * L for a in range(groups)],
                                                      ctx)
            masked = _mul_pt_rescale(list(rots), first, ctx)
            _release(rots)
            ws = _rotate_add_tree(masked, [-(L * L << b) for b in range(hb - sb)], ctx)
            _release(masked)
            spread = [None] * (groups * L)
            for m in range(L):
                # features = k mod L take the copy at residue m of their own
                # block, (m - k) features away (up or down, inside the head)
                pts = [fill[k][0] for k in range(L)]
                acc = fhe.hoisted_mac_sum_ext_many(ws, [(m - k) * L for k in range(L)], pts, 0, 1,
                                                   ctx)
                res = fhe.rescale_many(acc, ctx)
                _release(acc)
                for a in range(groups):
                    spread[a * L + m] = res[a]
            _release(ws)
            spread = spread[:T]
            sync()
            t_spread += time.perf_counter() - t0
            t0 = time.perf_counter()
            vsh = [_shifted(shifts, geo, c, d) for d in range(T)]
            limbs = min(int(spread[0].state.cur_limbs), int(vsh[0].state.cur_limbs))
            sa = _to_limbs(spread, limbs, ctx)
            va = _to_limbs(vsh, limbs, ctx)
            acc = None
            for x, y in zip(sa, va):
                t = fhe.homo_mul_no_relin(x, y, ctx)
                if acc is None:
                    acc = t
                else:
                    nxt = fhe.homo_add(acc, t, ctx)
                    acc.release()
                    t.release()
                    acc = nxt
            _release([a for a, b in zip(sa, spread) if a is not b])
            _release([a for a, b in zip(va, vsh) if a is not b])
            _release(spread)
            rl = fhe.homo_relinearize(acc, ctx)
            acc.release()
            out.append(fhe.rescale_many([rl], ctx)[0])
            rl.release()
            sync()
            t_prod += time.perf_counter() - t0
        _release(first)
        for f in fill:
            _release(f)
        stage["probability_spread"] = t_spread
        stage["products"] = t_prod
        return StageResult(tuple(out), stage)
    finally:
        for s_ in shifts:
            _release(s_)


def attention_fhe(query, key, value, geo: AttentionGeometry, cfg: SoftmaxConfig, *,
                  crypto_context, score_scale: float | None = None,
                  refresh=None) -> StageResult:
    """Causal attention ``softmax(s Q K^T) V`` per head of feature-major
    query/key/value streams (one level each; s = 1/sqrt(hd) by default) into
    a feature-major output stream."""
    ctx = _ctx(crypto_context)
    s = 1.0 / float(np.sqrt(int(geo.head_dim))) if score_scale is None else float(score_scale)
    a, b = cfg.score_map(s)
    stage = {}
    scores = qk_scores(query, key, geo, crypto_context=ctx, output_scale=a, output_offset=b)
    stage.update({f"qk.{k}": v for k, v in scores.stage_seconds.items()})
    try:
        probs = softmax_alg2(scores.ciphers, geo, cfg, crypto_context=ctx, refresh=refresh)
    finally:
        scores.release()
    stage.update({f"softmax.{k}": v for k, v in probs.stage_seconds.items()})
    try:
        out = pv_output(probs.ciphers, value, geo, crypto_context=ctx)
    finally:
        probs.release()
    stage.update({f"pv.{k}": v for k, v in out.stage_seconds.items()})
    return StageResult(out.ciphers, stage)


__all__ = ["AttentionGeometry", "SoftmaxConfig", "StageResult", "attention_fhe",
           "softmax_alg2", "softmax_depth", "attention_rotations", "kv_repeat_rows",
           "lane_shifts", "pv_output", "pv_rotations", "qk_rotations", "qk_scores",
           "softmax_rotations"]
