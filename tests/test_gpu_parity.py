"""Bit-exact parity of the gfx950 library with the CPU oracle.

Every test drives the library through the C ABI (via the ``easyfhe`` binding)
and compares ciphertext / key / polynomial limbs with the oracle on the same
parameters, seeds and inputs.  Integer results must be identical; decrypted
values are compared with the fp64 expectation at the tolerance stated in
each test.
"""

from __future__ import annotations

import numpy as np
import pytest

from conftest import PARAMS, device_context, oracle_context

pytestmark = pytest.mark.gpu


def _fhe():
    from easyfhe import fhe

    return fhe


def _rand_poly(rng, primes, shape_limbs, N, q_limbs=None):
    """Random residues, limb l drawn below the prime of limb l."""
    out = np.zeros((shape_limbs, N), dtype=np.uint64)
    for l in range(shape_limbs):
        out[l] = rng.integers(0, int(primes[l]), N, dtype=np.uint64)
    return out


# ---------------------------------------------------------------------------
# context: primes, secret, NTT
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("name", ["small", "matvec", "keyswitch"])
def test_context_parity(name):
    client, ctx = device_context(name, relin=False)
    orc = oracle_context(name)
    assert np.array_equal(ctx.primes(), orc.primes)
    assert np.array_equal(ctx.secret(), orc.secret())
    assert ctx.L == orc.L and ctx.alpha == orc.alpha


@pytest.mark.parametrize("log_n,first_mod,special_bits",
                         [(10, 60, 60), (11, 60, 60), (12, 60, 60), (13, 60, 60), (14, 60, 60),
                          (15, 60, 60), (16, 60, 60), (16, 40, 44), (16, 40, 60)])
def test_ntt_parity(log_n, first_mod, special_bits):
    """Both arithmetic paths at N = 2^16: 64-bit integer (primes >= 2^45) and
    fp64 (primes < 2^45), mixed within one call, on Q and special limbs, with
    edge values."""
    from easyfhe import _native

    p = dict(log_n=log_n, depth=3, dnum=2, dcrt_bits=40, first_mod=first_mod,
             special_bits=special_bits)
    client, ctx = device_context(p, relin=False)
    orc = oracle_context(p)
    rng = np.random.default_rng(log_n)
    primes = orc.primes
    L, A, N = orc.L, orc.alpha, orc.N
    # Q limbs then the special limbs (extended basis), 3 polynomials
    order = [primes[i] for i in range(L)] + [primes[L + j] for j in range(A)]
    a = np.stack([_rand_poly(rng, order, L + A, N) for _ in range(3)])
    # edge values: zeros, ones, q - 1
    a[0, :, :4] = 0
    a[0, :, 4:8] = 1
    for l in range(L + A):
        a[1, l, :8] = order[l] - 1
    fwd = np.zeros_like(a)
    _native.check(_native.lib.ckks_poly_ntt(ctx.handle, a.ctypes.data_as(_native.U64P),
                                            fwd.ctypes.data_as(_native.U64P), 3, L + A, L, 0))
    exp = np.stack([orc.ntt_limbs(a[i], q_limbs=L) for i in range(3)])
    assert np.array_equal(fwd, exp)
    inv = np.zeros_like(a)
    _native.check(_native.lib.ckks_poly_ntt(ctx.handle, fwd.ctypes.data_as(_native.U64P),
                                            inv.ctypes.data_as(_native.U64P), 3, L + A, L, 1))
    assert np.array_equal(inv, a)


# ---------------------------------------------------------------------------
# encryption, keys, key-switch stages
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("name", ["small", "matvec"])
def test_encrypt_decrypt_parity(name):
    fhe = _fhe()
    client, ctx = device_context(name, relin=False)
    orc = oracle_context(name)
    rng = np.random.default_rng(1)
    slots = ctx.max_slots
    z = rng.uniform(-1, 1, slots) + 1j * rng.uniform(-1, 1, slots)
    for limbs in (ctx.L, 2):
        ct = client.encrypt(z, slots=slots, cur_limbs=limbs, scaling_factor=2.0**40, enc_id=5)
        ref = orc.encrypt(z, slots=slots, scale=2.0**40, limbs=limbs, enc_id=5)
        assert np.array_equal(ct.download(), ref)
        dec = client.decrypt_complex(ct)
        # fresh-encryption error: sigma ~ 3.2 per coefficient, well below 1e-7
        assert np.abs(dec - z).max() < 1e-7
        assert np.abs(dec - orc.decrypt(ref, slots=slots, scale=2.0**40)).max() < 1e-12
    # sparse slot packing
    zs = z[:64]
    ct = client.encrypt(zs, slots=64, cur_limbs=ctx.L, scaling_factor=2.0**40, enc_id=9)
    ref = orc.encrypt(zs, slots=64, scale=2.0**40, limbs=ctx.L, enc_id=9)
    assert np.array_equal(ct.download(), ref)
    assert np.abs(client.decrypt_complex(ct) - zs).max() < 1e-7


def test_encode_parity_large_scale():
    """Encoder integer path for |coefficients| >= 2^63 (scale 2^80)."""
    fhe = _fhe()
    client, ctx = device_context("small", relin=False)
    orc = oracle_context("small")
    rng = np.random.default_rng(2)
    z = rng.uniform(-1, 1, (3, ctx.max_slots))
    pts = fhe.encode_rows(ctx, z, limbs=ctx.L, scale=2.0**80, slots=ctx.max_slots, is_ext=True)
    for r in range(3):
        ref = orc.encode(z[r], slots=ctx.max_slots, scale=2.0**80, limbs=ctx.L, is_ext=True)
        assert np.array_equal(pts[r].download()[0], ref)


@pytest.mark.parametrize("name", ["small", "matvec"])
def test_key_parity(name):
    client, ctx = device_context(name, rotations=(1, -3))
    orc = oracle_context(name)
    orc.gen_relin_key()
    assert np.array_equal(ctx.download_key(0), orc.get_key(0))
    for r in (1, -3):
        g = orc.galois_elt(r)
        assert g == ctx.galois_element(r)
        orc.gen_rotation_key(g)
        assert np.array_equal(ctx.download_key(g), orc.get_key(g))


@pytest.mark.parametrize("name", ["small", "matvec"])
def test_modup_moddown_parity(name):
    from easyfhe import _native

    client, ctx = device_context(name, relin=False)
    orc = oracle_context(name)
    rng = np.random.default_rng(3)
    for limbs in (ctx.L, ctx.L - 1, 1):
        d = _rand_poly(rng, orc.primes, limbs, orc.N)
        digits = -(-limbs // orc.ds)
        ext = np.zeros((digits, limbs + orc.alpha, orc.N), dtype=np.uint64)
        _native.check(_native.lib.ckks_poly_modup(ctx.handle, d.ctypes.data_as(_native.U64P),
                                                  limbs, ext.ctypes.data_as(_native.U64P)))
        assert np.array_equal(ext, orc.modup(d))
        order = [orc.primes[i] for i in range(limbs)] + [orc.primes[orc.L + j]
                                                         for j in range(orc.alpha)]
        acc = _rand_poly(rng, order, limbs + orc.alpha, orc.N)
        out = np.zeros((limbs, orc.N), dtype=np.uint64)
        _native.check(_native.lib.ckks_poly_moddown(ctx.handle, acc.ctypes.data_as(_native.U64P),
                                                    limbs, out.ctypes.data_as(_native.U64P)))
        assert np.array_equal(out, orc.moddown(acc))


# ---------------------------------------------------------------------------
# evaluation operations
# ---------------------------------------------------------------------------


def _pair(name, rotations=()):
    client, ctx = device_context(name, rotations=rotations)
    orc = oracle_context(name)
    orc.gen_relin_key()
    for r in rotations:
        orc.gen_rotation_key(orc.galois_elt(r))
    return client, ctx, orc


@pytest.mark.parametrize("name", ["small", "matvec"])
def test_rotation_parity(name):
    fhe = _fhe()
    rots = (1, 2, -1, 5)
    client, ctx, orc = _pair(name, rotations=rots + (2 * (2 ** PARAMS[name]["log_n"]) - 1,))
    rng = np.random.default_rng(4)
    slots = ctx.max_slots
    z = rng.uniform(-1, 1, slots) + 1j * rng.uniform(-1, 1, slots)
    for limbs in (ctx.L, 2):
        ct = client.encrypt(z, slots=slots, cur_limbs=limbs, scaling_factor=2.0**40, enc_id=11)
        ref = orc.encrypt(z, slots=slots, scale=2.0**40, limbs=limbs, enc_id=11)
        for r in rots:
            out = fhe.homo_rotate(ct, r, ctx)
            exp = orc.rotate_g(ref, orc.galois_elt(r))
            assert np.array_equal(out.download(), exp), (limbs, r)
            # rotation semantics: np.roll(z, -r); key-switch noise stays below 1e-6
            assert np.abs(client.decrypt_complex(out) - np.roll(z, -r)).max() < 1e-6
        conj = fhe.homo_rotate(ct, ctx.M - 1, ctx)
        assert np.array_equal(conj.download(), orc.rotate_g(ref, ctx.M - 1))
        assert np.abs(client.decrypt_complex(conj) - np.conj(z)).max() < 1e-6
        # hoisted: one ModUp, several rotations (0 is the identity)
        hs = fhe.prepare_hoisted_baby_rotations(ct, [0, 1, 2, 5], ctx)
        hexp = orc.hoisted_rotate(ref, [orc.galois_elt(r) for r in (0, 1, 2, 5)])
        for i in range(4):
            assert np.array_equal(hs[i].download(), hexp[i])
        # batched rotation of several ciphertexts with one key stream
        many = fhe.homo_rotate_many([ct, ct, ct], 2, ctx)
        for m in many:
            assert np.array_equal(m.download(), orc.rotate_g(ref, orc.galois_elt(2)))


@pytest.mark.parametrize("name", ["small", "matvec"])
def test_mul_relin_rescale_parity(name):
    fhe = _fhe()
    client, ctx, orc = _pair(name)
    rng = np.random.default_rng(5)
    slots = ctx.max_slots
    x = rng.uniform(-1, 1, slots)
    y = rng.uniform(-1, 1, slots)
    a = client.encrypt(x, slots=slots, enc_id=21)
    b = client.encrypt(y, slots=slots, enc_id=22)
    ra = orc.encrypt(x, slots=slots, scale=ctx.scale_at(ctx.L), limbs=ctx.L, enc_id=21)
    rb = orc.encrypt(y, slots=slots, scale=ctx.scale_at(ctx.L), limbs=ctx.L, enc_id=22)
    t = fhe.homo_mul_no_relin(a, b, ctx)
    rt = orc.tensor(ra, rb)
    assert np.array_equal(t.download(), rt)
    rl = fhe.homo_relinearize(t, ctx)
    rrl = orc.relinearize(rt)
    assert np.array_equal(rl.download(), rrl)
    rs = fhe.rescale(rl, ctx)
    rrs = orc.rescale(rrl)
    assert np.array_equal(rs.download(), rrs)
    assert rs.state.cur_limbs == ctx.L - 1
    # x*y after one rescale: error budget 1e-6 (key switch + rescale rounding)
    assert np.abs(client.decrypt(rs) - x * y).max() < 1e-6
    # batched form gives identical limbs
    many = fhe.homo_mul_relin_rescale_many([a, a], [b, b], ctx)
    for m in many:
        assert np.array_equal(m.download(), rrs)
    # rescale of a degree-2 ciphertext (tensor) as well
    assert np.array_equal(fhe.rescale(t, ctx).download(), orc.rescale(rt))
    # several primes in one pass = that many rescales in a row, after a
    # relinearisation as well as merged into its ModDown
    for k in range(2, ctx.L):
        want = rrl
        for _ in range(k):
            want = orc.rescale(want)
        for m in fhe.rescale_many([rl, rl], ctx, primes=k):
            assert np.array_equal(m.download(), want), k
            assert m.state.cur_limbs == ctx.L - k
        if k <= 4:
            for m in fhe.homo_mul_relin_rescale_many([a, a], [b, b], ctx, primes=k):
                assert np.array_equal(m.download(), want), k
    # one level down (an even number of limbs left after the rescale)
    lim = ctx.L - 1
    a2 = client.encrypt(x, slots=slots, cur_limbs=lim, enc_id=23)
    b2 = client.encrypt(y, slots=slots, cur_limbs=lim, enc_id=24)
    ra2 = orc.encrypt(x, slots=slots, scale=ctx.scale_at(lim), limbs=lim, enc_id=23)
    rb2 = orc.encrypt(y, slots=slots, scale=ctx.scale_at(lim), limbs=lim, enc_id=24)
    assert np.array_equal(a2.download(), ra2)
    exp2 = orc.rescale(orc.relinearize(orc.tensor(ra2, rb2)))
    for m in fhe.homo_mul_relin_rescale_many([a2, a2, a2], [b2, b2, b2], ctx):
        assert np.array_equal(m.download(), exp2)


@pytest.mark.parametrize("name", ["small", "keyswitch"])
def test_mod_raise_parity(name):
    """ModRaise of a bottom-level ciphertext to every limb, bit-exact."""
    fhe = _fhe()
    client, ctx = device_context(name, relin=False)
    orc = oracle_context(name)
    slots = orc.N // 2
    rng = np.random.default_rng(21)
    z = rng.uniform(-1, 1, slots)
    ct = orc.encrypt(z, slots=slots, scale=2.0**40, limbs=1, enc_id=5)
    dev = fhe.upload(ctx, ct, slots=slots, scale=2.0**40)
    for target in (orc.L, 2):
        out = fhe.mod_raise(dev, target, ctx).download()
        assert np.array_equal(out, orc.mod_raise(ct, target)), target


@pytest.mark.parametrize("name", ["small", "matvec"])
def test_elementwise_parity(name):
    fhe = _fhe()
    client, ctx, orc = _pair(name)
    rng = np.random.default_rng(6)
    slots = ctx.max_slots
    x = rng.uniform(-1, 1, slots) + 1j * rng.uniform(-1, 1, slots)
    y = rng.uniform(-1, 1, slots)
    a = client.encrypt(x, slots=slots, enc_id=31)
    b = client.encrypt(y, slots=slots, enc_id=32)
    sc = ctx.scale_at(ctx.L)
    ra = orc.encrypt(x, slots=slots, scale=sc, limbs=ctx.L, enc_id=31)
    rb = orc.encrypt(y, slots=slots, scale=sc, limbs=ctx.L, enc_id=32)
    assert np.array_equal(fhe.homo_add(a, b, ctx).download(), orc.add(ra, rb))
    assert np.array_equal(fhe.homo_sub(a, b, ctx).download(), orc.sub(ra, rb))
    for neg in (False, True):
        mi = fhe.homo_mul_i(a, ctx, negative=neg)
        assert np.array_equal(mi.download(), orc.mul_i(ra, negative=neg))
        want = (-1j if neg else 1j) * x
        assert np.abs(client.decrypt_complex(mi) - want).max() < 1e-7
    pt = fhe.encode_rows(ctx, y, limbs=ctx.L, scale=sc, slots=slots)[0]
    rpt = orc.encode(y, slots=slots, scale=sc, limbs=ctx.L)
    assert np.array_equal(pt.download()[0], rpt)
    mp = fhe.homo_mul_pt(a, pt, ctx)
    assert np.array_equal(mp.download(), orc.mul_pt(ra, rpt))
    mp_r = fhe.rescale(mp, ctx)
    assert np.abs(client.decrypt_complex(mp_r) - x * y).max() < 1e-6
    # scalar constants: add 0.25, multiply by -1.5 (then rescale)
    s_add = fhe.encode_scalar(0.25, cur_limbs=ctx.L, scaling_factor=sc, context=ctx)
    s_mul = fhe.encode_scalar(-1.5, cur_limbs=ctx.L, scaling_factor=sc, context=ctx)
    assert np.abs(client.decrypt_complex(fhe.homo_add_scalar(a, s_add, ctx)) - (x + 0.25)).max() < 1e-7
    prod = fhe.homo_mul_scalar_rescale(a, s_mul, ctx)
    assert np.abs(client.decrypt_complex(prod) - (-1.5 * x)).max() < 1e-6
    dropped = fhe.align_to(a, a.state.replace(cur_limbs=2), ctx)
    assert np.array_equal(dropped.download(), ra[:, :2])


# ---------------------------------------------------------------------------
# BSGS diagonal matvec (feature-major token-lane packing)
# ---------------------------------------------------------------------------


def _diagonals(W, *, slots, lanes, baby, giant_base, giant_count):
    """row(g, b)[slot] = W[(slot // lanes - g B) mod D, (slot // lanes + b) mod D]
    (the diagonal layout of reference operators/linear/weight.py:27-43)."""
    D = W.shape[0]
    feat = np.arange(slots) // lanes
    rows = []
    for gr in range(giant_count):
        g = giant_base + gr
        out_f = (feat - g * baby) % D
        for b in range(baby):
            rows.append(W[out_f, (feat + b) % D])
    return np.stack(rows)


def test_bsgs_matvec_parity():
    """Matvec workload: N = 2^13, 4096 slots, 4 x 40-bit limbs + 1 special,
    scale 2^40, W and x uniform[-1, 1] from seed 0, B = 16, G = 8, lanes 32."""
    fhe = _fhe()
    D, lanes, B, G = 128, 32, 16, 8
    rots = tuple(lanes * b for b in range(1, B)) + (B * lanes,)
    client, ctx, orc = _pair("matvec", rotations=rots)
    slots = ctx.max_slots
    rng = np.random.default_rng(0)
    W = rng.uniform(-1, 1, (D, D))
    x = rng.uniform(-1, 1, D)
    packed = np.zeros(slots)
    packed[np.arange(D) * lanes] = x
    sc = ctx.scale_at(ctx.L)
    ct = client.encrypt(packed, slots=slots, enc_id=41)
    ref = orc.encrypt(packed, slots=slots, scale=sc, limbs=ctx.L, enc_id=41)
    rows = _diagonals(W, slots=slots, lanes=lanes, baby=B, giant_base=0, giant_count=G)
    pts = fhe.encode_rows(ctx, rows, limbs=ctx.L, scale=sc, slots=slots)
    rpts = np.stack([orc.encode(r, slots=slots, scale=sc, limbs=ctx.L) for r in rows])
    for i in range(len(rows)):
        assert np.array_equal(pts[i].download()[0], rpts[i])
    offsets = [lanes * b for b in range(B)]
    acc = fhe.hoisted_mac_sum(ct, offsets, pts, B * lanes, G, ctx)
    racc = orc.hoisted_mac_sum(ref, [orc.galois_elt(o) for o in offsets], rpts,
                               orc.galois_elt(B * lanes), G)
    assert np.array_equal(acc.download(), racc)
    out = fhe.rescale(acc, ctx)
    dec = client.decrypt(out)[np.arange(D) * lanes]
    # fp64 W @ x; measured error ~1e-7 (128 products at scale 2^40)
    assert np.abs(dec - W @ x).max() < 1e-5


@pytest.mark.parametrize("name", ["matvec", "ext44"])
def test_bsgs_matvec_ext_parity(name):
    """The matvec workload with strategy "ext_normal": babies in Q u P, one
    ModDown per giant group; bit-exact with the oracle's extended schedule,
    on a 60-bit special prime (64-bit arithmetic on P) and on 44-bit ones
    (the fp64 path of the extended MAC and the babies' key products)."""
    fhe = _fhe()
    D, lanes, B, G = 128, 32, 16, 8
    rots = tuple(lanes * b for b in range(1, B)) + (B * lanes,)
    client, ctx, orc = _pair(name, rotations=rots)
    slots = ctx.max_slots
    rng = np.random.default_rng(0)
    W = rng.uniform(-1, 1, (D, D))
    x = rng.uniform(-1, 1, D)
    packed = np.zeros(slots)
    packed[np.arange(D) * lanes] = x
    sc = ctx.scale_at(ctx.L)
    ct = client.encrypt(packed, slots=slots, enc_id=41)
    ref = orc.encrypt(packed, slots=slots, scale=sc, limbs=ctx.L, enc_id=41)
    rows = _diagonals(W, slots=slots, lanes=lanes, baby=B, giant_base=0, giant_count=G)
    pts = fhe.encode_rows(ctx, rows, limbs=ctx.L, scale=sc, slots=slots, is_ext=True)
    rpts = np.stack([orc.encode(r, slots=slots, scale=sc, limbs=ctx.L, is_ext=True)
                     for r in rows])
    offsets = [lanes * b for b in range(B)]
    acc = fhe.hoisted_mac_sum(ct, offsets, pts, B * lanes, G, ctx, strategy="ext_normal")
    racc = orc.hoisted_mac_sum_ext(ref, [orc.galois_elt(o) for o in offsets], rpts,
                                   orc.galois_elt(B * lanes), G)
    assert np.array_equal(acc.download(), racc)
    dec = client.decrypt(fhe.rescale(acc, ctx))[np.arange(D) * lanes]
    assert np.abs(dec - W @ x).max() < 1e-5


# every prime of 59 or 60 bits, as on the reference's chain: both MACs take
# their 64-bit kernels on every limb
WIDE59 = dict(log_n=13, depth=3, dnum=2, dcrt_bits=59, first_mod=60, special_bits=60)


@pytest.mark.parametrize("strategy,B,G", [("normal", 40, 12), ("ext_normal", 40, 3),
                                          ("ext_normal", 24, 5)])
def test_bsgs_mac_wide_primes_parity(strategy, B, G):
    """The BSGS MAC with every prime of 2^45 or more (the 64-bit MAC kernels,
    which keep 16 babies' products as sums of 30-bit half products before a
    reduction): 40 babies (reductions after babies 16, 32 and 40) or 24
    (after 16 and 24); 12 giant groups on the Q basis (passes of 8 and 4),
    with extended plaintexts one group per pass (40 babies) or two and one
    (24 babies); three ciphertexts (a block's pair of inputs and a lone one).
    Every result bit-exact with the oracle's schedule and decrypting to the
    plaintext BSGS sum."""
    fhe = _fhe()
    lanes = 32
    ext = strategy != "normal"
    rots = tuple(lanes * b for b in range(1, B)) + (B * lanes,)
    client, ctx, orc = _pair(WIDE59, rotations=rots)
    assert all(int(p) >= 1 << 45 for p in orc.primes)
    slots, sc = ctx.max_slots, 2.0**50
    rng = np.random.default_rng(3)
    xs = [rng.uniform(-1, 1, slots) for _ in range(3)]
    rows = rng.uniform(-1, 1, (G * B, slots))
    pts = fhe.encode_rows(ctx, rows, limbs=ctx.L, scale=sc, slots=slots, is_ext=ext)
    rpts = np.stack([orc.encode(r, slots=slots, scale=sc, limbs=ctx.L, is_ext=ext)
                     for r in rows])
    cts = [client.encrypt(x, slots=slots, scaling_factor=sc, enc_id=60 + i)
           for i, x in enumerate(xs)]
    refs = [orc.encrypt(x, slots=slots, scale=sc, limbs=ctx.L, enc_id=60 + i)
            for i, x in enumerate(xs)]
    offsets = [lanes * b for b in range(B)]
    bgs, gg = [orc.galois_elt(o) for o in offsets], orc.galois_elt(B * lanes)
    if ext:
        accs = fhe.hoisted_mac_sum_ext_many(cts, offsets, pts, B * lanes, G, ctx,
                                            strategy="ext_normal")
    else:
        babies = [fhe.prepare_hoisted_baby_rotations(ct, offsets, ctx) for ct in cts]
        accs = fhe.hoisted_mac_sum_many(babies, pts, B * lanes, G, ctx)
        one = fhe.hoisted_mac_sum(cts[2], offsets, pts, B * lanes, G, ctx)
        assert np.array_equal(one.download(), accs[2].download())
    for acc, ref, x in zip(accs, refs, xs):
        racc = (orc.hoisted_mac_sum_ext if ext else orc.hoisted_mac_sum)(ref, bgs, rpts, gg, G)
        assert np.array_equal(acc.download(), racc)
        want = sum(np.roll(sum(rows[g * B + b] * np.roll(x, -b * lanes) for b in range(B)),
                           -g * B * lanes) for g in range(G))
        # up to 480 products at scale 2^50, one rescale by a 59-bit prime: ~1e-8
        assert np.abs(client.decrypt(fhe.rescale(acc, ctx)) - want).max() < 1e-6


@pytest.mark.parametrize("G", [1, 8])
def test_mac_wide_sums_at_maximal_words(G):
    """The 64-bit MAC's 30-bit half sums where their middle sum carries past
    2^64: babies and plaintexts of q - 1 (both 30-bit halves near 2^30 on the
    60-bit primes) with a few random ones, 40 babies, G giant groups with the
    identity as giant rotation, three inputs; every word equal to
    sum_g sum_b x_b w_(g B + b) mod q in exact integers."""
    fhe = _fhe()
    client, ctx = device_context(WIDE59, relin=False)
    L, N = ctx.L, ctx.N
    q = [int(p) for p in ctx.primes()[:L]]
    # q - 1 of a prime above 1.5 2^59 has both halves above 2^29.5: the sums
    # x0 w1 and x1 w0 of 16 such products each exceed 2^63
    assert max(q) > 3 << 58
    rng = np.random.default_rng(6)
    B, n = 40, 3

    def words(rand):
        if rand:
            return np.stack([rng.integers(0, q[l], N, dtype=np.uint64) for l in range(L)])
        return np.repeat(np.array(q, dtype=np.uint64)[:, None] - np.uint64(1), N, axis=1)

    xs = [[np.stack([words((b + i) % 7 == 3), words(False)]) for b in range(B)]
          for i in range(n)]
    ws = [words(k % 9 == 5)[None] for k in range(G * B)]
    babies = [[fhe.upload(ctx, x, slots=ctx.max_slots, scale=2.0**50) for x in row] for row in xs]
    pts = [fhe.upload(ctx, w, slots=ctx.max_slots, scale=2.0**50) for w in ws]
    accs = fhe.hoisted_mac_sum_many(babies, pts, 0, G, ctx)
    wsum = [sum(ws[g * B + b][0].astype(object) for g in range(G)) for b in range(B)]
    qo = np.array(q, dtype=object)[None, :, None]
    for i in range(n):
        want = sum(xs[i][b].astype(object) * wsum[b][None] for b in range(B)) % qo
        assert np.array_equal(accs[i].download(), want.astype(np.uint64)), i


# 14 special primes of 60 bits (one digit of 14 limbs), and 59/60-bit primes
# in 6 digits
SP14 = dict(log_n=12, depth=13, dnum=1, dcrt_bits=40, first_mod=60, special_bits=60)
DIG6 = dict(log_n=12, depth=11, dnum=6, dcrt_bits=59, first_mod=60, special_bits=60)


@pytest.mark.parametrize("params", [SP14, DIG6, WIDE59], ids=["sp14", "dig6", "wide59"])
def test_wide_prime_product_sums_parity(params):
    """The 64-bit sums of products kept as 30-bit half sums outside the MACs:
    the integer ModDown conversion fused with 1..4 rescales (its sums over
    the special limbs and the lifts: 14 + 4 terms in two sets on SP14) and
    the multi-key inner product of hoisted rotations (6 digits on DIG6);
    limbs equal to the oracle's relinearise, rescales and rotations."""
    fhe = _fhe()
    rots = (1, 3, 7)
    client, ctx, orc = _pair(params, rotations=rots)
    slots, L = ctx.max_slots, ctx.L
    rng = np.random.default_rng(12)
    x, y = rng.uniform(-1, 1, slots), rng.uniform(-1, 1, slots)
    a = client.encrypt(x, slots=slots, enc_id=81)
    b = client.encrypt(y, slots=slots, enc_id=82)
    ra = orc.encrypt(x, slots=slots, scale=ctx.scale_at(L), limbs=L, enc_id=81)
    rb = orc.encrypt(y, slots=slots, scale=ctx.scale_at(L), limbs=L, enc_id=82)
    want = [orc.relinearize(orc.tensor(ra, rb)), orc.relinearize(orc.tensor(rb, rb))]
    for k in range(1, min(4, L - 1) + 1):
        want = [orc.rescale(w) for w in want]
        got = fhe.homo_mul_relin_rescale_many([a, b], [b, b], ctx, primes=k)
        for i in range(2):
            assert np.array_equal(got[i].download(), want[i]), (k, i)
    sq = fhe.homo_mul_relin_rescale_many([b], [b], ctx)[0]
    assert np.array_equal(sq.download(), orc.rescale(orc.relinearize(orc.tensor(rb, rb))))
    hs = fhe.prepare_hoisted_baby_rotations(a, (0,) + rots, ctx)
    hw = orc.hoisted_rotate(ra, [orc.galois_elt(r) for r in (0,) + rots])
    for h, w in zip(hs, hw):
        assert np.array_equal(h.download(), w)
    assert np.abs(client.decrypt(hs[2]) - np.roll(x, -3)).max() < 1e-6


@pytest.mark.parametrize("name", ["matvec", "ext44"])
@pytest.mark.parametrize("n_cts", [1, 3])
def test_bsgs_matvec_double_hoist_parity(n_cts, name):
    """The matvec workload with strategy "ext_double_hoist": babies and
    giant groups in Q u P, every giant group rotated by its own key, one
    ModDown of the sum; bit-exact with the oracle's double-hoisted schedule
    for one ciphertext and for a batch of three (each equal to its own
    single-ciphertext result), decrypting to W x; on 60-bit and on 44-bit
    special primes (the fp64 paths of the extended MAC, the multi-key
    product and the giant groups' ModDown and re-ModUp)."""
    fhe = _fhe()
    D, lanes, B, G = 128, 32, 16, 8
    rots = tuple(lanes * b for b in range(1, B)) + tuple(g * B * lanes for g in range(1, G))
    client, ctx, orc = _pair(name, rotations=rots)
    slots = ctx.max_slots
    rng = np.random.default_rng(0)
    W = rng.uniform(-1, 1, (D, D))
    xs = [rng.uniform(-1, 1, D) for _ in range(n_cts)]
    sc = ctx.scale_at(ctx.L)
    rows = _diagonals(W, slots=slots, lanes=lanes, baby=B, giant_base=0, giant_count=G)
    pts = fhe.encode_rows(ctx, rows, limbs=ctx.L, scale=sc, slots=slots, is_ext=True)
    rpts = np.stack([orc.encode(r, slots=slots, scale=sc, limbs=ctx.L, is_ext=True)
                     for r in rows])
    offsets = [lanes * b for b in range(B)]
    cts, refs = [], []
    for i, x in enumerate(xs):
        packed = np.zeros(slots)
        packed[np.arange(D) * lanes] = x
        cts.append(client.encrypt(packed, slots=slots, enc_id=41 + i))
        refs.append(orc.encrypt(packed, slots=slots, scale=sc, limbs=ctx.L, enc_id=41 + i))
    if n_cts == 1:
        accs = [fhe.hoisted_mac_sum(cts[0], offsets, pts, B * lanes, G, ctx,
                                    strategy="ext_double_hoist")]
    else:
        accs = fhe.hoisted_mac_sum_ext_many(cts, offsets, pts, B * lanes, G, ctx,
                                            strategy="ext_double_hoist")
    ggs = [orc.galois_elt(g * B * lanes) for g in range(G)]
    for acc, ref, x in zip(accs, refs, xs):
        racc = orc.hoisted_mac_sum_double(ref, [orc.galois_elt(o) for o in offsets], rpts, ggs)
        assert np.array_equal(acc.download(), racc)
        dec = client.decrypt(fhe.rescale(acc, ctx))[np.arange(D) * lanes]
        assert np.abs(dec - W @ x).max() < 1e-5


@pytest.mark.parametrize("name", ["small", "matvec"])
def test_fast_rotate_ext_moddown_is_rotation(name):
    """ModDown(P sigma(c0) + acc_0, acc_1) is the rotation bit for bit (P
    sigma(c0) vanishes on the special limbs); offset 0 gives the input back;
    an extended pairwise MAC brought back by one ModDown decrypts to the sum."""
    fhe = _fhe()
    rots = (1, 3)
    client, ctx, orc = _pair(name, rotations=rots)
    slots = ctx.max_slots
    rng = np.random.default_rng(17)
    z = rng.uniform(-1, 1, slots)
    ct = client.encrypt(z, slots=slots, enc_id=9)
    batch = fhe.fast_rotate(ct, [0, 1, 3], ctx, output_ext=True)
    assert all(b.is_ext for b in batch.cv)
    plain = [fhe.homo_rotate(ct, r, ctx) for r in (1, 3)]
    assert np.array_equal(fhe.moddown_from_ext(batch.cv[0], ctx).download(), ct.download())
    for b, ref in zip(batch.cv[1:], plain):
        assert np.array_equal(fhe.moddown_from_ext(b, ctx).download(), ref.download())
    w = [rng.uniform(-1, 1, slots) for _ in range(3)]
    sc = ctx.scale_at(ctx.L)
    pts = [fhe.encode_rows(ctx, v, limbs=ctx.L, scale=sc, slots=slots, is_ext=True)[0] for v in w]
    acc = fhe.grouped_pairwise_mac(batch, pts, [[0, 1, 2]], ctx)[0]
    assert acc.is_ext
    out = fhe.rescale(fhe.moddown_from_ext(acc, ctx), ctx)
    want = w[0] * z + w[1] * np.roll(z, -1) + w[2] * np.roll(z, -3)
    assert np.abs(client.decrypt(out) - want).max() < 1e-6


def _composed_mac(fhe, ctx, cts, pts):
    acc = None
    for c, p in zip(cts, pts):
        t = fhe.homo_mul_pt(c, p, ctx)
        acc = t if acc is None else fhe.homo_add(acc, t, ctx)
    return acc


@pytest.mark.slow
def test_grouped_pairwise_mac_matches_composed_full_size():
    """N = 2^16 on the key-switch chain at 13 limbs: eight extended hoisted
    rotations times extended plaintexts, as the reference calls it (the
    rotations of one target packed into a batch of four, group count 1: one
    ciphertext back; and the eight as two groups of four), and the same on
    Q-basis rotations; every result equal word for word to homo_mul_pt then
    homo_add, and its ModDown to the plain rotations' weighted sum."""
    fhe = _fhe()
    offs = list(range(8))
    client, ctx = device_context("keyswitch", rotations=tuple(o for o in offs if o))
    slots, limbs = ctx.max_slots, 13
    rng = np.random.default_rng(23)
    z = rng.uniform(-1, 1, slots)
    ct = client.encrypt(z, cur_limbs=limbs, enc_id=31)
    sc = ct.state.scaling_factor
    w = [rng.uniform(-1, 1, slots) for _ in offs]
    for ext in (True, False):
        batch = fhe.fast_rotate(ct, offs, ctx, output_ext=ext)
        assert all(b.is_ext == ext for b in batch.cv)
        pts = [fhe.encode_rows(ctx, v, limbs=limbs, scale=sc, slots=slots, is_ext=ext)[0]
               for v in w]
        two = fhe.grouped_pairwise_mac(batch, pts, 2, ctx)
        assert len(two) == 2
        for g in range(2):
            want = _composed_mac(fhe, ctx, batch.cv[4 * g:4 * g + 4], pts[4 * g:4 * g + 4])
            assert two[g].is_ext == ext
            assert np.array_equal(two[g].download(), want.download()), (ext, g)
        one = fhe.grouped_pairwise_mac(fhe.pack_cipher_batch(batch.cv[4:]), pts[4:], 1, ctx)
        assert not isinstance(one, list) and one.is_ext == ext
        assert np.array_equal(one.download(), two[1].download())
        picked = fhe.grouped_pairwise_mac(batch, pts, [[7, 0, 3]], ctx)[0]
        want = _composed_mac(fhe, ctx, [batch.cv[i] for i in (7, 0, 3)],
                             [pts[i] for i in (7, 0, 3)])
        assert np.array_equal(picked.download(), want.download())
        if ext:
            out = fhe.rescale(fhe.moddown_from_ext(one, ctx), ctx)
            want = sum(w[k] * np.roll(z, -k) for k in range(4, 8))
            assert np.abs(client.decrypt(out) - want).max() < 1e-6
    with pytest.raises(ValueError):
        fhe.grouped_pairwise_mac(batch, pts, 3, ctx)  # 8 terms into 3 groups
    ctx.close()


# ---------------------------------------------------------------------------
# keyswitch workload size (N = 2^16, 36 + 12 limbs, dnum 3)
# ---------------------------------------------------------------------------


@pytest.mark.slow
def test_keyswitch_size_parity():
    fhe = _fhe()
    rots = (1, 1 << 14)
    client, ctx, orc = _pair("keyswitch", rotations=rots)
    slots = ctx.max_slots
    rng = np.random.default_rng(0)
    zs = [rng.uniform(-1, 1, slots) for _ in range(2)]
    cts = [client.encrypt(z, slots=slots, enc_id=100 + i) for i, z in enumerate(zs)]
    refs = [orc.encrypt(z, slots=slots, scale=ctx.scale_at(ctx.L), limbs=ctx.L, enc_id=100 + i)
            for i, z in enumerate(zs)]
    for i in range(2):
        assert np.array_equal(cts[i].download(), refs[i])
    for r in rots:
        outs = fhe.homo_rotate_many(cts, r, ctx)
        for i in range(2):
            assert np.array_equal(outs[i].download(), orc.rotate_g(refs[i], orc.galois_elt(r)))
            assert np.abs(client.decrypt(outs[i]) - np.roll(zs[i], -r)).max() < 1e-6
    prods = fhe.homo_mul_relin_rescale_many(cts, cts, ctx)
    for i in range(2):
        exp = orc.rescale(orc.relinearize(orc.tensor(refs[i], refs[i])))
        assert np.array_equal(prods[i].download(), exp)
        assert np.abs(client.decrypt(prods[i]) - zs[i] ** 2).max() < 1e-6
    # rescales at this size (the combine runs in the NTT's last pass), by 1..3
    # primes at once, and of a degree-2 ciphertext
    want = refs[0]
    for k in (1, 2, 3):
        want = orc.rescale(want)
        got = fhe.rescale_many(cts[:1], ctx, primes=k)[0]
        assert np.array_equal(got.download(), want), k
    t3 = fhe.homo_mul_no_relin(cts[0], cts[1], ctx)
    r3 = orc.tensor(refs[0], refs[1])
    assert np.array_equal(fhe.rescale_many([t3], ctx, primes=2)[0].download(),
                          orc.rescale(orc.rescale(r3)))
    # relinearise + two rescales as one ModDown
    got = fhe.homo_mul_relin_rescale_many(cts[:1], cts[1:], ctx, primes=2)[0]
    assert np.array_equal(got.download(), orc.rescale(orc.rescale(orc.relinearize(r3))))


@pytest.mark.slow
@pytest.mark.parametrize("env", [{"CKKS_KS_DEFER": "0"}, {"CKKS_KS_TILE": "0"},
                                 {"CKKS_KS_SPECIAL_INV": "0"}, {"CKKS_SPLIT_STREAMS": "1"}])
def test_keyswitch_kernel_choices_full_size(env, monkeypatch):
    """The key-switch kernel choices read at context creation give the
    oracle's words at N = 2^16 on the key-switch chain: without the deferred
    combine (CKKS_KS_DEFER=0: the product's addend d0, d1 then written whole
    before the ModDown), without the tile-resident conversion (CKKS_KS_TILE=0:
    d2 = a1 b1 written before the ModUp instead of formed as it loads),
    without the special limbs' inverse pass in the key product
    (CKKS_KS_SPECIAL_INV=0) and with every batch on one stream
    (CKKS_SPLIT_STREAMS=1).  Rotations, products of distinct factors and
    squares (the addend formed from one factor), by one and by two primes, and
    a relinearisation alone."""
    fhe = _fhe()
    for k, v in env.items():
        monkeypatch.setenv(k, v)
    r = 1 << 5
    client, ctx, orc = _pair("keyswitch", rotations=(r,))
    slots, L = ctx.max_slots, ctx.L
    rng = np.random.default_rng(9)
    zs = [rng.uniform(-1, 1, slots) for _ in range(3)]
    cts = [client.encrypt(z, slots=slots, enc_id=300 + i) for i, z in enumerate(zs)]
    refs = [orc.encrypt(z, slots=slots, scale=ctx.scale_at(L), limbs=L, enc_id=300 + i)
            for i, z in enumerate(zs)]
    for out, ref in zip(fhe.homo_rotate_many(cts, r, ctx), refs):
        assert np.array_equal(out.download(), orc.rotate_g(ref, orc.galois_elt(r)))
    pairs = [(0, 1), (2, 0)]
    prods = fhe.homo_mul_relin_rescale_many([cts[i] for i, _ in pairs],
                                            [cts[j] for _, j in pairs], ctx)
    for (i, j), got in zip(pairs, prods):
        want = orc.rescale(orc.relinearize(orc.tensor(refs[i], refs[j])))
        assert np.array_equal(got.download(), want), (env, i, j)
        # key switch + rescale rounding: 1e-6
        assert np.abs(client.decrypt(got) - zs[i] * zs[j]).max() < 1e-6
    sq = fhe.homo_mul_relin_rescale_many(cts[1:], cts[1:], ctx, primes=2)
    for i, got in zip((1, 2), sq):
        want = orc.rescale(orc.rescale(orc.relinearize(orc.tensor(refs[i], refs[i]))))
        assert np.array_equal(got.download(), want), (env, i)
    t = fhe.homo_mul_no_relin(cts[2], cts[1], ctx)
    assert np.array_equal(fhe.homo_relinearize(t, ctx).download(),
                          orc.relinearize(orc.tensor(refs[2], refs[1])))
    ctx.close()


def test_linear_combination_matches_composed_ops():
    """One fused launch = mul_scalar + add + add_scalar on the same words,
    with terms holding more limbs than the output."""
    fhe = _fhe()
    client, ctx, orc = _pair("small")
    slots = ctx.max_slots
    rng = np.random.default_rng(23)
    n, limbs = 3, ctx.L - 2
    terms = [[client.encrypt(rng.uniform(-1, 1, slots), cur_limbs=ctx.L - t, enc_id=200 + 10 * t + i)
              for i in range(n)] for t in range(3)]
    weights = [3.0 * 2**30, -7.5 * 2**30, 2.0**33 + 0.25]
    const, scale = -0.375 * 2**70, 2.0**70
    fused = fhe.linear_combination(terms, weights, const, limbs, scale, 2, ctx)
    for i in range(n):
        acc = None
        for t in range(3):
            x = fhe.align_to(terms[t][i], terms[t][i].state.replace(cur_limbs=limbs,
                                                                    scaling_factor=None), ctx)
            enc = fhe.encode_scalar(weights[t], limbs, scaling_factor=1.0, context=ctx)
            term = fhe.homo_mul_scalar(x, enc, ctx)
            acc = term if acc is None else fhe.homo_add(acc, term, ctx)
        acc = fhe.homo_add_scalar(acc, fhe.encode_scalar(const, limbs, scaling_factor=1.0,
                                                         context=ctx), ctx)
        assert np.array_equal(fused[i].download(), acc.download()), i


def test_objects_outliving_their_context():
    """Ciphertexts and tensors freed after their context was destroyed only
    drop their host record, also when a new context takes the old address."""
    _fhe()
    from easyfhe.tensor import DeviceTensor

    client, ctx = device_context("small", relin=False)
    ct = client.encrypt(np.ones(ctx.max_slots), enc_id=1)
    t = DeviceTensor(np.ones(16, dtype=np.float32), context=ctx)
    ctx.close()
    client2, ctx2 = device_context("small", relin=False)
    ct.release()
    t.release()
    ct2 = client2.encrypt(np.full(ctx2.max_slots, 0.5), enc_id=2)
    assert np.abs(client2.decrypt(ct2) - 0.5).max() < 1e-6


def test_scalar_constants_and_invalid_objects():
    """A scalar constant (one word per limb) drops limbs without writing past
    its own words; entry points that need a ciphertext reject it with
    ValueError instead of reading N words per limb; uploads check the slot
    count and the array shape."""
    fhe = _fhe()
    client, ctx = device_context("small", relin=False)
    primes = [int(q) for q in ctx.primes()[: ctx.L]]
    sc = 2.0**40
    s = fhe.encode_scalar(-1.5, cur_limbs=ctx.L, scaling_factor=sc, context=ctx)
    want = np.array([(-int(1.5 * sc)) % q for q in primes], dtype=np.uint64)
    assert np.array_equal(s.download(), want)
    guard = client.encrypt(np.linspace(-1, 1, ctx.max_slots), enc_id=9)
    before = guard.download()
    dropped = fhe.align_to(s, s.state.replace(cur_limbs=2), ctx)
    assert np.array_equal(dropped.download(), want[:2])
    ctx.synchronize()
    assert np.array_equal(guard.download(), before)
    for op in (lambda: fhe.rescale(s, ctx), lambda: fhe.homo_mul_i(s, ctx),
               lambda: fhe.homo_add(s, s, ctx), lambda: fhe.homo_mul_scalar(s, s, ctx)):
        with pytest.raises(ValueError):
            op()
    for bad in (0, 3, 2 * ctx.max_slots):
        with pytest.raises(ValueError):
            fhe.upload(ctx, before, slots=bad, scale=sc)
    with pytest.raises(ValueError):
        fhe.upload(ctx, before[:, :, :-1], slots=ctx.max_slots, scale=sc)


# a chain whose special primes are too wide for the merged relinearise-rescale
# ModDown (12 x 60-bit P: the postop then runs as separate launches)
WIDE_P = dict(log_n=12, depth=35, dnum=3, dcrt_bits=40, first_mod=60, special_bits=60)


@pytest.mark.parametrize("name", ["small", "matvec", "keyswitch", "wide_p"])
def test_mul_relin_rescale_postop_matches_composed(name):
    """homo_mul_relin_rescale_postop (x2, - sub, + scalar folded into the
    ModDown epilogue) equals the oracle's relinearise, rescale, add, sub and
    scalar add on the same words (reference operators/nonlinear/
    polynomial.py:115-203: 2 T_i T_j - T_1 and 2 T_i T_j - 1)."""
    fhe = _fhe()
    p = WIDE_P if name == "wide_p" else name
    client, ctx = device_context(p)
    orc = oracle_context(p)
    orc.gen_relin_key()
    slots, L = ctx.max_slots, ctx.L
    n = 2 if name == "keyswitch" else 3
    rng = np.random.default_rng(31)
    sc = ctx.scale_at(L)
    xs = [rng.uniform(-1, 1, slots) for _ in range(n)]
    ys = [rng.uniform(-1, 1, slots) for _ in range(n)]
    zs = [rng.uniform(-1, 1, slots) for _ in range(n)]
    a = [client.encrypt(x, enc_id=500 + i) for i, x in enumerate(xs)]
    b = [client.encrypt(y, enc_id=520 + i) for i, y in enumerate(ys)]
    subs = [client.encrypt(z, enc_id=540 + i) for i, z in enumerate(zs)]
    ra = [orc.encrypt(x, slots=slots, scale=sc, limbs=L, enc_id=500 + i) for i, x in enumerate(xs)]
    rb = [orc.encrypt(y, slots=slots, scale=sc, limbs=L, enc_id=520 + i) for i, y in enumerate(ys)]
    rs = [orc.encrypt(z, slots=slots, scale=sc, limbs=L, enc_id=540 + i) for i, z in enumerate(zs)]
    base = [orc.rescale(orc.relinearize(orc.tensor(ra[i], rb[i]))) for i in range(n)]
    out_scale = sc * sc / ctx.rescale_divisor_at(L - 1)
    scal = fhe.encode_scalar(-1.0, cur_limbs=L, scaling_factor=out_scale, context=ctx)
    words = scal.download()[: L - 1].astype(np.uint64)
    primes = ctx.primes()[: L - 1].astype(np.uint64)
    cases = [(True, True, False), (True, False, True), (False, True, True), (False, False, False)]
    for dbl, use_sub, use_scal in cases[: 2 if name == "keyswitch" else 4]:
        outs = fhe.homo_mul_relin_rescale_postop_many(
            a, b, ctx, apply_double=dbl, sub=subs if use_sub else None,
            scalar=scal if use_scal else None)
        for i in range(n):
            want = base[i]
            if dbl:
                want = orc.add(want, want)
            if use_sub:
                want = orc.sub(want, orc.drop_limbs(rs[i], L - 1))
            if use_scal:
                want = want.copy()
                want[0] = (want[0] + words[:, None]) % primes[:, None]
            assert np.array_equal(outs[i].download(), want), (dbl, use_sub, use_scal, i)
        # the subtrahend enters at its own scale (fixed-scale bookkeeping): on a
        # 40-bit chain the product's scale 2^80 / q differs from it by ~2^-15
        got = client.decrypt(outs[0])
        exp = ((2 if dbl else 1) * xs[0] * ys[0] - (zs[0] * sc / out_scale if use_sub else 0)
               - (1 if use_scal else 0))
        assert np.abs(got - exp).max() < 1e-5
    # the single-pair form aligns operands at different levels first
    low = fhe.align_to(b[0], b[0].state.replace(cur_limbs=L - 1, scaling_factor=None), ctx)
    one = fhe.homo_mul_relin_rescale_postop(a[0], low, ctx, apply_double=True, sub=subs[0])
    assert one.state.cur_limbs == L - 2
    ratio = subs[0].state.scaling_factor / one.state.scaling_factor
    assert np.abs(client.decrypt(one) - (2 * xs[0] * ys[0] - zs[0] * ratio)).max() < 1e-5


def test_align_to_changes_the_scale():
    """A target scaling factor different from the source's is reached by an
    integer multiply and a rescale on the levels the drop sheds; without a
    spare level only the fixed-scale tolerance is accepted."""
    fhe = _fhe()
    client, ctx = device_context("small", relin=False)
    L = ctx.L
    rng = np.random.default_rng(41)
    z = rng.uniform(-1, 1, ctx.max_slots)
    ct = client.encrypt(z, enc_id=600)
    for target, ratio in ((2, 1.37), (3, 0.61), (L - 1, 1.0 + 2.0**-20)):
        want = ct.state.scaling_factor * ratio
        out = fhe.align_to(ct, ct.state.replace(cur_limbs=target, scaling_factor=want), ctx)
        assert out.state.cur_limbs == target
        assert abs(out.state.scaling_factor / want - 1.0) < 2.0**-30
        assert np.abs(client.decrypt(out) - z).max() < 1e-6
    # same limbs: within 2^-10 kept as is, beyond it refused
    near = ct.state.replace(scaling_factor=ct.state.scaling_factor * (1 + 2.0**-12))
    assert fhe.align_to(ct, near, ctx) is ct
    with pytest.raises(ValueError):
        fhe.align_to(ct, ct.state.replace(scaling_factor=ct.state.scaling_factor * 1.5), ctx)
