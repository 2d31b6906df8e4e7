"""Both basis-conversion kernels give the same words as the oracle's fast
basis conversion: ModUp of every digit and the centered ModDown at several
levels, on chains with a 60-bit q_0 among 40-bit primes (a wide source digit
and a wide target) and with 60-bit special primes, then rotations and
products through them at the key-switch workload's size, with the key
product fused into the forward NTT's low pass and without.

The kernel is chosen when a context is created: the int8-MFMA kernel
(k_basis_convert_mfma) by default, the VALU kernels (k_basis_convert_fp and
the integer ones) with CKKS_BASIS_CONVERT=valu.  Every case here runs once
with each.
"""

from __future__ import annotations

import numpy as np
import pytest

from conftest import PARAMS, device_context, oracle_context

pytestmark = pytest.mark.gpu

# digits of 11 limbs with 11 60-bit special primes; and one digit of 16 (the
# largest digit a conversion takes: four source quads)
WIDE = dict(log_n=12, depth=32, dnum=3, dcrt_bits=40, first_mod=60, special_bits=60)
SIXTEEN = dict(log_n=12, depth=15, dnum=1, dcrt_bits=40, first_mod=60, special_bits=44)


@pytest.fixture(autouse=True, params=["mfma", "valu"])
def conversion_kernel(request, monkeypatch):
    monkeypatch.setenv("CKKS_BASIS_CONVERT", request.param)
    return request.param


def _rand(rng, primes, n, N):
    return np.stack([rng.integers(0, int(primes[l]), N, dtype=np.uint64) for l in range(n)])


@pytest.mark.parametrize("name", ["small", "matvec", "wide", "sixteen", "keyswitch"])
def test_mfma_modup_moddown_parity(name):
    from easyfhe import _native

    p = {"wide": WIDE, "sixteen": SIXTEEN}.get(name, name)
    client, ctx = device_context(p, relin=False)
    orc = oracle_context(p)
    rng = np.random.default_rng(7)
    levels = (ctx.L, ctx.L - 1, 1) if name != "keyswitch" else (ctx.L, 13)
    for limbs in levels:
        d = _rand(rng, orc.primes, limbs, orc.N)
        d[:, :4] = 0
        d[0, 4:8] = int(orc.primes[0]) - 1
        digits = -(-limbs // orc.ds)
        ext = np.zeros((digits, limbs + orc.alpha, orc.N), dtype=np.uint64)
        _native.check(_native.lib.ckks_poly_modup(ctx.handle, d.ctypes.data_as(_native.U64P),
                                                  limbs, ext.ctypes.data_as(_native.U64P)))
        assert np.array_equal(ext, orc.modup(d)), (name, limbs)
        order = [orc.primes[i] for i in range(limbs)] + [orc.primes[orc.L + j]
                                                         for j in range(orc.alpha)]
        acc = _rand(rng, order, limbs + orc.alpha, orc.N)
        out = np.zeros((limbs, orc.N), dtype=np.uint64)
        _native.check(_native.lib.ckks_poly_moddown(ctx.handle, acc.ctypes.data_as(_native.U64P),
                                                    limbs, out.ctypes.data_as(_native.U64P)))
        assert np.array_equal(out, orc.moddown(acc)), (name, limbs)
    ctx.close()


@pytest.mark.slow
@pytest.mark.parametrize("fused", ["1", "0"])
def test_mfma_keyswitch_full_size(fused, monkeypatch):
    """Rotation, multiply-relinearise-rescale and a hoisted rotation at
    N = 2^16 on the key-switch chain, limbs equal to the oracle's; with the
    extended digits' low NTT pass fused with the key product (the default)
    and with the separate kernels (CKKS_KEYSWITCH_FUSED=0)."""
    from easyfhe import fhe

    monkeypatch.setenv("CKKS_KEYSWITCH_FUSED", fused)
    rot = 1 << 7
    client, ctx = device_context("keyswitch", rotations=(rot, 3))
    orc = oracle_context("keyswitch")
    orc.gen_relin_key()
    for r in (rot, 3):
        orc.gen_rotation_key(orc.galois_elt(r))
    slots, L = ctx.max_slots, ctx.L
    rng = np.random.default_rng(2)
    zs = [rng.uniform(-1, 1, slots) for _ in range(2)]
    cts = [client.encrypt(z, enc_id=700 + i) for i, z in enumerate(zs)]
    refs = [orc.encrypt(z, slots=slots, scale=ctx.scale_at(L), limbs=L, enc_id=700 + i)
            for i, z in enumerate(zs)]
    rots = fhe.homo_rotate_many(cts, rot, ctx)
    for i in range(2):
        assert np.array_equal(rots[i].download(), orc.rotate_g(refs[i], orc.galois_elt(rot)))
    prod = fhe.homo_mul_relin_rescale_many(cts[:1], cts[1:], ctx)[0]
    assert np.array_equal(prod.download(),
                          orc.rescale(orc.relinearize(orc.tensor(refs[0], refs[1]))))
    hs = fhe.prepare_hoisted_baby_rotations(cts[0], [0, 3, rot], ctx)
    want = orc.hoisted_rotate(refs[0], [orc.galois_elt(r) for r in (0, 3, rot)])
    for h, w in zip(hs, want):
        assert np.array_equal(h.download(), w)
    assert np.abs(client.decrypt(rots[0]) - np.roll(zs[0], -rot)).max() < 1e-6
    ctx.close()


# N = 2^16 with every prime of 2^45 or more (as on the reference's 59-bit
# chain): the tile-resident conversion keeps the 64-bit high passes inside
# when a launch holds wide primes only
ALL_WIDE = dict(log_n=16, depth=5, dnum=2, dcrt_bits=59, first_mod=60, special_bits=60)


@pytest.mark.slow
def test_keyswitch_all_wide_primes_full_size():
    """Rotation, multiply-relinearise-rescale and hoisted rotations at
    N = 2^16 on a chain of 59- and 60-bit primes, limbs equal to the
    oracle's."""
    from easyfhe import fhe

    rot = 1 << 9
    client, ctx = device_context(ALL_WIDE, rotations=(rot, 5))
    orc = oracle_context(ALL_WIDE)
    orc.gen_relin_key()
    for r in (rot, 5):
        orc.gen_rotation_key(orc.galois_elt(r))
    slots, L = ctx.max_slots, ctx.L
    rng = np.random.default_rng(11)
    zs = [rng.uniform(-1, 1, slots) for _ in range(2)]
    cts = [client.encrypt(z, enc_id=740 + i) for i, z in enumerate(zs)]
    refs = [orc.encrypt(z, slots=slots, scale=ctx.scale_at(L), limbs=L, enc_id=740 + i)
            for i, z in enumerate(zs)]
    rots = fhe.homo_rotate_many(cts, rot, ctx)
    for i in range(2):
        assert np.array_equal(rots[i].download(), orc.rotate_g(refs[i], orc.galois_elt(rot)))
    prod = fhe.homo_mul_relin_rescale_many(cts[:1], cts[1:], ctx)[0]
    assert np.array_equal(prod.download(),
                          orc.rescale(orc.relinearize(orc.tensor(refs[0], refs[1]))))
    hs = fhe.prepare_hoisted_baby_rotations(cts[0], [0, 5, rot], ctx)
    want = orc.hoisted_rotate(refs[0], [orc.galois_elt(r) for r in (0, 5, rot)])
    for h, w in zip(hs, want):
        assert np.array_equal(h.download(), w)
    assert np.abs(client.decrypt(rots[0]) - np.roll(zs[0], -rot)).max() < 1e-6
    ctx.close()


@pytest.mark.slow
def test_mfma_relin_rescale_two_primes_full_size():
    """Relinearise + two rescales as one ModDown at N = 2^16 on the key-switch
    chain: at 36 limbs the two dropped primes' targets share a target group
    (the int8-MFMA conversion with both lifts in its epilogue), at 33 limbs
    they do not (the fp64 VALU kernel); limbs equal to the oracle's
    relinearise then two rescales."""
    from easyfhe import fhe

    client, ctx = device_context("keyswitch")
    orc = oracle_context("keyswitch")
    orc.gen_relin_key()
    slots = ctx.max_slots
    rng = np.random.default_rng(5)
    zs = [rng.uniform(-1, 1, slots) for _ in range(2)]
    for limbs in (36, 33):
        # two rescales by ~2^40 primes: inputs at 2^60 leave the product near 2^40
        sc = 2.0**60
        cts = [client.encrypt(z, cur_limbs=limbs, scaling_factor=sc, enc_id=720 + i)
               for i, z in enumerate(zs)]
        refs = [orc.encrypt(z, slots=slots, scale=sc, limbs=limbs, enc_id=720 + i)
                for i, z in enumerate(zs)]
        prod = fhe.homo_mul_relin_rescale_many(cts[:1], cts[1:], ctx, primes=2)[0]
        want = orc.rescale(orc.rescale(orc.relinearize(orc.tensor(refs[0], refs[1]))))
        assert np.array_equal(prod.download(), want), limbs
        assert np.abs(client.decrypt(prod) - zs[0] * zs[1]).max() < 1e-4, limbs
    ctx.close()
