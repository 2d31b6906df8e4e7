"""Pins of the CPU oracle against published vectors and mathematics.

The reference has no tests and its arithmetic lives in EasyFHE, which is
absent (reference docs/SETUP.md:15-34), so each oracle function is pinned
here by something that does not restate its own formula: RFC 8439 vectors,
sympy primality, brute force on small moduli, O(N^2) transforms and
schoolbook products with Python integers, exact CRT reconstructions.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import sympy

import oracle as O
from conftest import oracle_context


def _small_ctx(log_n=8, limbs=4, dnum=2, first=60, dcrt=40, special=60, seed=0):
    alpha = math.ceil(limbs / dnum)
    return O.OracleContext(log_n=log_n, limbs=limbs, alpha=alpha, dnum=dnum, first_bits=first,
                           dcrt_bits=dcrt, special_bits=special, seed=seed)


def _centered(v: int, q: int) -> int:
    v %= q
    return v - q if v > (q - 1) // 2 else v


def _crt(residues, primes) -> int:
    Q = math.prod(int(p) for p in primes)
    x = 0
    for r, p in zip(residues, primes):
        p = int(p)
        Qi = Q // p
        x += int(r) * Qi * pow(Qi, -1, p)
    return x % Q


# ---------------------------------------------------------------------------
# PRNG, primes, roots
# ---------------------------------------------------------------------------


def test_chacha20_rfc8439_block_vector():
    """RFC 8439 sec. 2.3.2: key 00..1f, nonce 000000090000004a00000000, counter 1."""
    key = [int.from_bytes(bytes(range(4 * i, 4 * i + 4)), "little") for i in range(8)]
    nonce = [0x09000000, 0x4A000000, 0x00000000]
    out = O.chacha20_block(key, 1, nonce).astype("<u4").tobytes().hex()
    assert out == (
        "10f1e7e4d13b5915500fdd1fa32071c4c7d1f4c733c068030422aa9ac3d46c4e"
        "d2826446079faa0914c2d705d98b02a2b5129cd1de164eb9cbd083e8a2503c4e"
    )


def test_chacha20_rfc8439_zero_key_vector():
    """RFC 8439 appendix A.1, test vector 1 (all-zero key, nonce, counter)."""
    out = O.chacha20_block([0] * 8, 0, [0, 0, 0]).astype("<u4").tobytes().hex()
    assert out == (
        "76b8e0ada0f13d90405d6ae55386bd28bdd219b8a08ded1aa836efcc8b770dc7"
        "da41597c5157488d7724e03fb8d84a376a43b8f41518a11cc387b669b2ee6586"
    )


def test_miller_rabin_matches_sympy():
    lib = O.lib()
    rng = np.random.default_rng(7)
    cands = [int(v) for v in rng.integers(2**40, 2**60, 400, dtype=np.uint64)]
    # Carmichael numbers and strong pseudoprimes to small bases
    cands += [561, 41041, 825265, 321197185, 2047, 1373653, 25326001, 3215031751,
              2152302898747, 3474749660383, 341550071728321, 3825123056546413051,
              2**61 - 1, 2**59 - 55, 2**31 - 1]
    for c in cands:
        assert bool(lib.orc_is_prime(c)) == sympy.isprime(c), c


@pytest.mark.parametrize("log_n,bits", [(12, 40), (13, 40), (16, 40), (16, 60), (16, 59)])
def test_prime_rule_is_nearest_first(log_n, bits):
    """The selected primes are exactly the count nearest NTT-friendly primes
    to 2^bits below 2^60 (checked against sympy over every candidate)."""
    M = 2 << log_n
    count = 6
    got = O.gen_primes(log_n, bits, count)
    assert len(got) == count
    for q in got:
        assert q % M == 1 and sympy.isprime(q) and q < 2**60
    far = max(abs(q - (1 << bits)) for q in got)
    # every prime candidate strictly closer than the farthest chosen is chosen
    k = 0
    while k * M <= far:
        for c in {(1 << bits) - k * M + 1, (1 << bits) + k * M + 1}:
            if 0 < c < 2**60 and abs(c - (1 << bits)) < far and sympy.isprime(c):
                assert c in got
        k += 1
    # distinctness against a used list
    more = O.gen_primes(log_n, bits, 3, used=got[:2])
    assert not set(more) & set(got[:2])


@pytest.mark.parametrize("q,log_n", [(97, 4), (193, 5), (257, 6), (7681, 8), (12289, 9)])
def test_min_root_brute_force(q, log_n):
    N = 1 << log_n
    roots = [r for r in range(1, q) if pow(r, N, q) == q - 1]
    assert int(O.lib().orc_min_root(q, log_n)) == min(roots)


# ---------------------------------------------------------------------------
# NTT
# ---------------------------------------------------------------------------


def _bitrev(i, bits):
    return int(format(i, f"0{bits}b")[::-1], 2)


def test_ntt_matches_naive_dft():
    """a_hat[i] = sum_k a_k psi^((2 br(i) + 1) k), psi the minimal primitive
    2N-th root, by direct O(N^2) evaluation."""
    ctx = _small_ctx(log_n=8)
    N = ctx.N
    rng = np.random.default_rng(0)
    for p in range(ctx.L + ctx.alpha):
        q = int(ctx.primes[p])
        psi = int(O.lib().orc_min_root(q, 8))
        a = rng.integers(0, q, N, dtype=np.uint64)
        A = ctx.ntt(a, p)
        ai = [int(v) for v in a]
        for i in range(N):
            w = pow(psi, 2 * _bitrev(i, 8) + 1, q)
            acc, wk = 0, 1
            for k in range(N):
                acc += ai[k] * wk
                wk = wk * w % q
            assert acc % q == int(A[i])
        assert np.array_equal(ctx.intt(A, p), a)


def test_ntt_roundtrip_full_size():
    ctx = oracle_context("keyswitch")
    rng = np.random.default_rng(1)
    a = np.stack([rng.integers(0, int(ctx.primes[l]), ctx.N, dtype=np.uint64)
                  for l in range(ctx.L)])
    assert np.array_equal(ctx.intt_limbs(ctx.ntt_limbs(a)), a)


def test_negacyclic_convolution_theorem():
    """NTT^-1(NTT(a) NTT(b)) equals the schoolbook product mod X^N + 1."""
    ctx = _small_ctx(log_n=8)
    N = ctx.N
    q = int(ctx.primes[1])
    rng = np.random.default_rng(2)
    a = rng.integers(0, q, N, dtype=np.uint64)
    b = rng.integers(0, q, N, dtype=np.uint64)
    A, B = ctx.ntt(a, 1), ctx.ntt(b, 1)
    C = np.array([int(x) * int(y) % q for x, y in zip(A, B)], dtype=np.uint64)
    c = ctx.intt(C, 1)
    ref = [0] * N
    for i in range(N):
        for j in range(N):
            k = i + j
            if k < N:
                ref[k] += int(a[i]) * int(b[j])
            else:
                ref[k - N] -= int(a[i]) * int(b[j])
    assert [v % q for v in ref] == [int(v) for v in c]


@pytest.mark.parametrize("g", [5, 25, 5**7 % 512, 511, 3])
def test_automorphism_ntt_vs_coefficients(g):
    ctx = _small_ctx(log_n=8)
    rng = np.random.default_rng(3)
    q = int(ctx.primes[0])
    a = rng.integers(0, q, ctx.N, dtype=np.uint64)
    lhs = ctx.ntt(ctx.automorphism_coeff(a, 0, g), 0)
    rhs = ctx.automorphism_ntt(ctx.ntt(a, 0), g)
    assert np.array_equal(lhs, rhs)
    # coefficient map by definition: X^k -> X^(k g) with X^N = -1
    N = ctx.N
    ref = [0] * N
    for k in range(N):
        e = k * g % (2 * N)
        if e < N:
            ref[e] = int(a[k])
        else:
            ref[e - N] = (-int(a[k])) % q
    assert [int(v) for v in ctx.automorphism_coeff(a, 0, g)] == ref


# ---------------------------------------------------------------------------
# encoder
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("slots", [128, 16])
def test_encoder_matches_canonical_embedding(slots):
    """m(zeta^(5^j)) = scale z_j for zeta = exp(i pi / N), m real, slot
    values repeated with period `slots` in the sparse case: the coefficients
    are the inverse of that evaluation (direct O(N n) formula)."""
    ctx = _small_ctx(log_n=8)
    N = ctx.N
    rng = np.random.default_rng(4)
    z = rng.uniform(-1, 1, slots) + 1j * rng.uniform(-1, 1, slots)
    scale = 2.0**30
    got = ctx.encode_coeffs(z, slots=slots, scale=scale)
    gap = N // (2 * slots)
    n2 = 2 * slots  # degree of m'(Y), Y = X^gap, evaluation at rho = exp(2 pi i / 4n)
    k = np.arange(n2)
    expo = np.array([pow(5, j, 4 * slots) for j in range(slots)])
    rho = np.exp(2j * np.pi / (4 * slots))
    # m'_k = (1/n) Re sum_j scale z_j rho^(-k 5^j)  (n points and their conjugates)
    mp = np.real((scale * z[None, :] * rho ** (-np.outer(k, expo))).sum(axis=1)) / slots
    ref = np.zeros(N)
    ref[::gap] = mp
    assert np.max(np.abs(got - np.rint(ref))) <= 1.0
    assert np.mean(got == np.rint(ref)) > 0.99
    # evaluation of the encoded polynomial reproduces the slots
    zeta = np.exp(1j * np.pi / N)
    pts = np.array([pow(5, j, 2 * N) for j in range(slots)])
    vals = (got[None, :] * zeta ** np.outer(pts, np.arange(N))).sum(axis=1) / scale
    assert np.abs(vals - z).max() < 1e-6


def test_decode_inverts_encode_and_monomial_closed_form():
    ctx = _small_ctx(log_n=10, limbs=3)
    slots = ctx.N // 2
    rng = np.random.default_rng(5)
    z = rng.uniform(-1, 1, slots) + 1j * rng.uniform(-1, 1, slots)
    pt = ctx.encode(z, slots=slots, scale=2.0**40, limbs=3)
    assert np.abs(ctx.decode(pt, slots=slots, scale=2.0**40) - z).max() < 1e-9
    # m = X: slot j decodes to zeta^(5^j)
    N = ctx.N
    x = np.zeros((3, N), dtype=np.uint64)
    x[:, 1] = 1
    xn = ctx.ntt_limbs(x)
    dec = ctx.decode(xn, slots=slots, scale=1.0)
    want = np.exp(1j * np.pi / N * np.array([pow(5, j, 2 * N) for j in range(slots)]))
    assert np.abs(dec - want).max() < 1e-9


# ---------------------------------------------------------------------------
# RNS base conversion, ModDown, rescale (exact big-integer checks)
# ---------------------------------------------------------------------------


def _coeff(ctx, poly, limbs):
    return ctx.intt_limbs(poly, q_limbs=limbs)


def test_modup_is_crt_lift_plus_small_multiple():
    """ext_j limb t = x + u Q_j (mod t) with x the CRT value of digit j's
    residues in [0, Q_j) and 0 <= u < |digit| (fast base conversion)."""
    ctx = _small_ctx(log_n=8, limbs=5, dnum=2)  # digits of 3 and 2 limbs, alpha 3
    rng = np.random.default_rng(6)
    limbs = 5
    d = np.stack([rng.integers(0, int(ctx.primes[l]), ctx.N, dtype=np.uint64) for l in range(limbs)])
    ext = ctx.modup(d)
    dcoef = _coeff(ctx, d, limbs)
    E = limbs + ctx.alpha
    order = [int(ctx.primes[l]) for l in range(limbs)] + [int(ctx.primes[ctx.L + j]) for j in range(ctx.alpha)]
    for j in range(ext.shape[0]):
        lo, hi = j * ctx.ds, min((j + 1) * ctx.ds, limbs)
        Qj = math.prod(order[lo:hi])
        ecoef = ctx.intt_limbs(ext[j], q_limbs=limbs)
        for k in range(0, ctx.N, 17):
            x = _crt([dcoef[l, k] for l in range(lo, hi)], order[lo:hi])
            for t in range(E):
                if lo <= t < hi:
                    assert ecoef[t, k] == dcoef[t, k]
                    continue
                diff = (int(ecoef[t, k]) - x) % order[t]
                assert any(diff == (u * Qj) % order[t] for u in range(hi - lo)), (j, t, k)


def test_moddown_is_division_by_p_within_alpha():
    """ModDown(acc) = floor(X / P) - u (mod Q) with |u| <= alpha, X the CRT
    value of acc over Q u P (centered conversion: u in [-alpha/2, alpha/2 + 1])."""
    ctx = _small_ctx(log_n=8, limbs=4, dnum=2)
    rng = np.random.default_rng(8)
    limbs = 4
    order = [int(ctx.primes[l]) for l in range(limbs)] + [int(ctx.primes[ctx.L + j]) for j in range(ctx.alpha)]
    acc = np.stack([rng.integers(0, q, ctx.N, dtype=np.uint64) for q in order])
    out = ctx.moddown(acc)
    acoef = ctx.intt_limbs(acc, q_limbs=limbs)
    ocoef = ctx.intt_limbs(out)
    Q = math.prod(order[:limbs])
    P = math.prod(order[limbs:])
    us = []
    for k in range(0, ctx.N, 7):
        X = _crt([acoef[t, k] for t in range(limbs + ctx.alpha)], order)
        V = _crt([ocoef[t, k] for t in range(limbs)], order[:limbs])
        u = _centered(X // P - V, Q)
        assert abs(u) <= ctx.alpha
        us.append(u)
    assert abs(np.mean(us)) < 1.0  # centered: no systematic bias


def test_rescale_is_rounded_division():
    ctx = _small_ctx(log_n=8, limbs=4, dnum=2)
    rng = np.random.default_rng(9)
    limbs = 4
    primes = [int(ctx.primes[l]) for l in range(limbs)]
    ct = np.stack([np.stack([rng.integers(0, q, ctx.N, dtype=np.uint64) for q in primes])
                   for _ in range(2)])
    out = ctx.rescale(ct)
    Q = math.prod(primes)
    ql = primes[-1]
    for d in range(2):
        c = ctx.intt_limbs(ct[d])
        o = ctx.intt_limbs(out[d])
        for k in range(0, ctx.N, 5):
            X = _centered(_crt([c[t, k] for t in range(limbs)], primes), Q)
            want = (X + ql // 2) // ql  # round(X / ql), ties impossible (ql odd)
            V = _crt([o[t, k] for t in range(limbs - 1)], primes[:-1])
            assert (V - want) % math.prod(primes[:-1]) == 0


def test_mod_raise_is_centered_lift():
    """Every raised coefficient's CRT value over the target limbs, centered,
    equals the one-limb coefficient centered mod q_0."""
    ctx = _small_ctx(log_n=8, limbs=4, dnum=2)
    rng = np.random.default_rng(10)
    q0 = int(ctx.primes[0])
    ct = rng.integers(0, q0, (2, 1, ctx.N), dtype=np.uint64)
    ct[0, 0, :3] = [0, (q0 - 1) // 2, (q0 + 1) // 2]  # both sides of the centre
    out = ctx.mod_raise(ct, 4)
    primes = [int(ctx.primes[l]) for l in range(4)]
    Q = math.prod(primes)
    for d in range(2):
        c = ctx.intt_limbs(ct[d])
        o = ctx.intt_limbs(out[d])
        for k in range(0, ctx.N, 3):
            X = _centered(_crt([o[t, k] for t in range(4)], primes), Q)
            assert X == _centered(int(c[0, k]), q0), (d, k)


def test_mod_raise_plaintext_is_m_plus_q0_multiple():
    """decrypt(ModRaise(ct)) = m + q_0 I with I small (|I| <= (h + 1) / 2 for
    a sparse secret of weight h); its q_0 residue is the original plaintext."""
    ctx = oracle_context("small")
    slots = ctx.N // 2
    rng = np.random.default_rng(13)
    z = rng.uniform(-1, 1, slots)
    ct = ctx.encrypt(z, slots=slots, scale=2.0**40, limbs=1, enc_id=3)
    raised = ctx.mod_raise(ct, ctx.L)
    m0 = ctx.intt_limbs(ctx.decrypt_poly(ct))
    mr = ctx.intt_limbs(ctx.decrypt_poly(raised))
    q0 = int(ctx.primes[0])
    primes = [int(p) for p in ctx.primes[: ctx.L]]
    Q = math.prod(primes)
    worst = 0
    for k in range(0, ctx.N, 11):
        X = _centered(_crt([mr[t, k] for t in range(ctx.L)], primes), Q)
        m = _centered(int(m0[0, k]), q0)
        assert (X - m) % q0 == 0
        worst = max(worst, abs((X - m) // q0))
    assert 0 < worst <= (192 + 1) // 2


# ---------------------------------------------------------------------------
# keys, encryption and homomorphic identities (decrypted values)
# ---------------------------------------------------------------------------


def test_secret_is_sparse_ternary():
    ctx = oracle_context("small")
    s = ctx.secret()
    assert set(np.unique(s)) <= {-1, 0, 1}
    assert int((s != 0).sum()) == 192
    u = O.OracleContext(log_n=12, limbs=2, alpha=1, dnum=2, first_bits=60, dcrt_bits=40,
                        special_bits=60, seed=3, secret_mode=1)
    su = u.secret()
    assert set(np.unique(su)) == {-1, 0, 1} and abs((su == 0).mean() - 1 / 3) < 0.05


def test_switching_key_structure():
    """b_j + a_j s = e_j + [P]_q s' on digit j's primes and e_j elsewhere,
    with |e_j| <= 21 (centered binomial, eta 21)."""
    ctx = _small_ctx(log_n=8, limbs=4, dnum=2)
    g = ctx.galois_elt(1)
    ctx.gen_rotation_key(g)
    key = ctx.get_key(g)
    K = ctx.L + ctx.alpha
    s = ctx.secret().astype(np.int64)
    N = ctx.N
    # s' = s(X^g) as integers
    sp = np.zeros(N, dtype=np.int64)
    for k in range(N):
        e = k * g % (2 * N)
        if e < N:
            sp[e] += s[k]
        else:
            sp[e - N] -= s[k]
    P = math.prod(int(ctx.primes[ctx.L + j]) for j in range(ctx.alpha))
    for j in range(key.shape[0]):
        for p in range(K):
            q = int(ctx.primes[p])
            b = ctx.intt(key[j, 0, p].copy(), p)
            a = ctx.intt(key[j, 1, p].copy(), p)
            # a s mod (X^N + 1) via NTT
            As = ctx.intt(np.array([int(x) * int(y) % q for x, y in
                                    zip(key[j, 1, p], ctx.ntt(np.array([v % q for v in s], dtype=np.uint64), p))],
                                   dtype=np.uint64), p)
            val = [(int(b[k]) + int(As[k])) % q for k in range(N)]
            if p < ctx.L and j * ctx.ds <= p < (j + 1) * ctx.ds:
                val = [(v - (P % q) * int(sp[k])) % q for k, v in enumerate(val)]
            e = [_centered(v, q) for v in val]
            assert max(abs(x) for x in e) <= 21
            del a


def test_encryption_error_is_small():
    ctx = oracle_context("small")
    slots = ctx.N // 2
    z = np.random.default_rng(10).uniform(-1, 1, slots)
    ct = ctx.encrypt(z, slots=slots, scale=2.0**40, limbs=ctx.L, enc_id=3)
    m = ctx.decrypt_poly(ct)
    pt = ctx.encode(z, slots=slots, scale=2.0**40, limbs=ctx.L)
    diff = ctx.intt((m[0] + ctx.primes[0] - pt[0]) % ctx.primes[0], 0)
    e = [_centered(int(v), int(ctx.primes[0])) for v in diff]
    assert max(abs(x) for x in e) <= 21


@pytest.fixture(scope="module")
def small_keys():
    ctx = oracle_context("small")
    for r in (1, 3, -2, ctx.N * 2 - 1):
        ctx.gen_rotation_key(ctx.galois_elt(r))
    ctx.gen_relin_key()
    return ctx


def test_rotation_semantics(small_keys):
    ctx = small_keys
    slots = ctx.N // 2
    rng = np.random.default_rng(11)
    z = rng.uniform(-1, 1, slots) + 1j * rng.uniform(-1, 1, slots)
    ct = ctx.encrypt(z, slots=slots, scale=2.0**40, limbs=ctx.L, enc_id=1)
    for r in (1, 3, -2):
        out = ctx.rotate_g(ct, ctx.galois_elt(r))
        assert np.abs(ctx.decrypt(out, slots=slots, scale=2.0**40) - np.roll(z, -r)).max() < 1e-7
    conj = ctx.rotate_g(ct, ctx.galois_elt(ctx.N * 2 - 1))
    assert np.abs(ctx.decrypt(conj, slots=slots, scale=2.0**40) - np.conj(z)).max() < 1e-7
    mi = ctx.mul_i(ct)
    assert np.abs(ctx.decrypt(mi, slots=slots, scale=2.0**40) - 1j * z).max() < 1e-8
    mn = ctx.mul_i(ct, negative=True)
    assert np.abs(ctx.decrypt(mn, slots=slots, scale=2.0**40) + 1j * z).max() < 1e-8


def test_mul_relin_rescale_semantics(small_keys):
    ctx = small_keys
    slots = ctx.N // 2
    rng = np.random.default_rng(12)
    x = rng.uniform(-1, 1, slots)
    y = rng.uniform(-1, 1, slots)
    a = ctx.encrypt(x, slots=slots, scale=2.0**40, limbs=ctx.L, enc_id=1)
    b = ctx.encrypt(y, slots=slots, scale=2.0**40, limbs=ctx.L, enc_id=2)
    t = ctx.tensor(a, b)
    assert np.abs(ctx.decrypt(t, slots=slots, scale=2.0**80) - x * y).max() < 1e-8
    r = ctx.rescale(ctx.relinearize(t))
    sc = 2.0**80 / float(ctx.primes[ctx.L - 1])
    assert np.abs(ctx.decrypt(r, slots=slots, scale=sc) - x * y).max() < 1e-7


def test_bsgs_matvec_decrypts_to_wx():
    """The matvec workload on the oracle: decrypt(rescale(MAC)) = W x."""
    ctx = oracle_context("matvec")
    D, lanes, B, G = 128, 32, 16, 8
    for o in list(range(lanes, B * lanes, lanes)) + [B * lanes]:
        ctx.gen_rotation_key(ctx.galois_elt(o))
    slots = ctx.N // 2
    rng = np.random.default_rng(0)
    W = rng.uniform(-1, 1, (D, D))
    x = rng.uniform(-1, 1, D)
    packed = np.zeros(slots)
    packed[np.arange(D) * lanes] = x
    ct = ctx.encrypt(packed, slots=slots, scale=2.0**40, limbs=ctx.L, enc_id=41)
    feat = np.arange(slots) // lanes
    rows = [W[(feat - g * B) % D, (feat + b) % D] for g in range(G) for b in range(B)]
    pts = np.stack([ctx.encode(r, slots=slots, scale=2.0**40, limbs=ctx.L) for r in rows])
    acc = ctx.hoisted_mac_sum(ct, [ctx.galois_elt(lanes * b) for b in range(B)], pts,
                              ctx.galois_elt(B * lanes), G)
    out = ctx.rescale(acc)
    sc = 2.0**80 / float(ctx.primes[ctx.L - 1])
    dec = ctx.decrypt(out, slots=slots, scale=sc).real[np.arange(D) * lanes]
    assert np.abs(dec - W @ x).max() < 1e-5


def test_bsgs_matvec_ext_schedule_decrypts_to_wx():
    """The extended-basis schedule (one ModDown per giant group) on the
    oracle: decrypt(rescale(MAC)) = W x, and its limbs differ from the normal
    schedule's (different rounding, same value)."""
    ctx = oracle_context("matvec")
    D, lanes, B, G = 128, 32, 16, 8
    for o in list(range(lanes, B * lanes, lanes)) + [B * lanes]:
        ctx.gen_rotation_key(ctx.galois_elt(o))
    slots = ctx.N // 2
    rng = np.random.default_rng(0)
    W = rng.uniform(-1, 1, (D, D))
    x = rng.uniform(-1, 1, D)
    packed = np.zeros(slots)
    packed[np.arange(D) * lanes] = x
    ct = ctx.encrypt(packed, slots=slots, scale=2.0**40, limbs=ctx.L, enc_id=41)
    feat = np.arange(slots) // lanes
    rows = [W[(feat - g * B) % D, (feat + b) % D] for g in range(G) for b in range(B)]
    pts = np.stack([ctx.encode(r, slots=slots, scale=2.0**40, limbs=ctx.L, is_ext=True)
                    for r in rows])
    gs = [ctx.galois_elt(lanes * b) for b in range(B)]
    acc = ctx.hoisted_mac_sum_ext(ct, gs, pts, ctx.galois_elt(B * lanes), G)
    sc = 2.0**80 / float(ctx.primes[ctx.L - 1])
    dec = ctx.decrypt(ctx.rescale(acc), slots=slots, scale=sc).real[np.arange(D) * lanes]
    assert np.abs(dec - W @ x).max() < 1e-5
    normal = ctx.hoisted_mac_sum(ct, gs, np.ascontiguousarray(pts[:, : ctx.L]),
                                 ctx.galois_elt(B * lanes), G)
    assert not np.array_equal(acc, normal)



def test_bsgs_matvec_double_hoist_decrypts_to_wx():
    """The double-hoisted schedule (every giant group rotated in Q u P by its
    own key, one ModDown of the sum) on the oracle: decrypt(rescale(MAC)) =
    W x; its decrypted value agrees with the extended schedule's to the
    rounding of a key switch, and its limbs differ (another rounding).  A
    giant Galois element of 1 adds the group unrotated: the matvec with its
    diagonals' giant offsets all 0 (G copies of one group) decrypts to G W x
    restricted to the first group."""
    ctx = oracle_context("matvec")
    D, lanes, B, G = 128, 32, 16, 8
    for o in list(range(lanes, B * lanes, lanes)) + [g * B * lanes for g in range(1, G)]:
        ctx.gen_rotation_key(ctx.galois_elt(o))
    slots = ctx.N // 2
    rng = np.random.default_rng(0)
    W = rng.uniform(-1, 1, (D, D))
    x = rng.uniform(-1, 1, D)
    packed = np.zeros(slots)
    packed[np.arange(D) * lanes] = x
    ct = ctx.encrypt(packed, slots=slots, scale=2.0**40, limbs=ctx.L, enc_id=41)
    feat = np.arange(slots) // lanes
    rows = [W[(feat - g * B) % D, (feat + b) % D] for g in range(G) for b in range(B)]
    pts = np.stack([ctx.encode(r, slots=slots, scale=2.0**40, limbs=ctx.L, is_ext=True)
                    for r in rows])
    gs = [ctx.galois_elt(lanes * b) for b in range(B)]
    ggs = [ctx.galois_elt(g * B * lanes) for g in range(G)]
    acc = ctx.hoisted_mac_sum_double(ct, gs, pts, ggs)
    sc = 2.0**80 / float(ctx.primes[ctx.L - 1])
    dec = ctx.decrypt(ctx.rescale(acc), slots=slots, scale=sc).real[np.arange(D) * lanes]
    assert np.abs(dec - W @ x).max() < 1e-5
    ext = ctx.hoisted_mac_sum_ext(ct, gs, pts, ctx.galois_elt(B * lanes), G)
    dext = ctx.decrypt(ctx.rescale(ext), slots=slots, scale=sc).real[np.arange(D) * lanes]
    assert np.abs(dec - dext).max() < 1e-7
    assert not np.array_equal(acc, ext)
    # identity giants: the group-0 diagonals G times
    same = np.concatenate([pts[:B]] * G)
    acc1 = ctx.hoisted_mac_sum_double(ct, gs, same, [1] * G)
    d1 = ctx.decrypt(ctx.rescale(acc1), slots=slots, scale=sc).real[np.arange(D) * lanes]
    Wb = np.zeros((D, D))
    f = np.arange(D)
    for b in range(B):
        Wb[f, (f + b) % D] = W[f, (f + b) % D]
    assert np.abs(d1 - G * (Wb @ x)).max() < 1e-5


@pytest.mark.parametrize("special,first", [(60, 60), (44, 40)])
def test_fast_build_gives_the_same_words(special, first):
    """The ORC_FAST build (Shoup reductions of 128-bit sums, the build the CPU
    baseline times) equals the pinned `%` build word for word: encryption,
    rotation, relinearisation, rescale, ModUp / ModDown and the BSGS MAC, on
    60-bit and on 40/44-bit primes at N = 2^12."""
    fast = O.load(O.fast_library_path())
    kw = dict(log_n=12, limbs=6, alpha=2, dnum=3, first_bits=first, dcrt_bits=40,
              special_bits=special, seed=3)
    a, b = O.OracleContext(**kw), O.OracleContext(**kw, library=fast)
    assert np.array_equal(a.primes, b.primes)
    g = a.galois_elt(5)
    for ctx in (a, b):
        ctx.gen_rotation_key(g)
        ctx.gen_relin_key()
    rng = np.random.default_rng(special)
    z = rng.uniform(-1, 1, 2048) + 1j * rng.uniform(-1, 1, 2048)
    ca = a.encrypt(z, slots=2048, scale=2.0**40, limbs=6, enc_id=7)
    cb = b.encrypt(z, slots=2048, scale=2.0**40, limbs=6, enc_id=7)
    assert np.array_equal(ca, cb)
    # the timed build's lazy (Harvey) butterflies end on the same words,
    # including the edge values 0 and q - 1
    for pi in (0, 3, 7):
        q = int(a.primes[pi])
        poly = rng.integers(0, q, 4096, dtype=np.uint64)
        poly[:3] = [0, q - 1, 1]
        assert np.array_equal(a.ntt(poly, pi), b.ntt(poly, pi))
        assert np.array_equal(a.intt(poly, pi), b.intt(poly, pi))
    assert np.array_equal(a.rotate_g(ca, g), b.rotate_g(cb, g))
    assert np.array_equal(a.relinearize(a.tensor(ca, ca)), b.relinearize(b.tensor(cb, cb)))
    assert np.array_equal(a.rescale(ca), b.rescale(cb))
    ext = a.modup(ca[1])
    assert np.array_equal(ext, b.modup(cb[1]))
    acc = ext[0]
    assert np.array_equal(a.moddown(acc), b.moddown(acc))
    pts = [a.encode(rng.uniform(-1, 1, 2048), slots=2048, scale=2.0**40, limbs=6)
           for _ in range(4)]
    assert np.array_equal(a.hoisted_mac_sum(ca, [1, g], pts, g, 2),
                          b.hoisted_mac_sum(cb, [1, g], pts, g, 2))
