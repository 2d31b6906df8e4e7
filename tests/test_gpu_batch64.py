"""Batched key switching at the batch size the keyswitch benchmark runs.

The benchmark rotates and multiplies 64 ciphertexts per call, so the 64-entry
pointer tables, the fused ModDown's 2n = 128 grid rows and the split of
larger batches into launches of 64 are checked here limb for limb against
the oracle: at N = 2^16 on the benchmark's chain (1 x 60-bit + 35 x 40-bit
primes, dnum 3, 12 special primes) for items 0, 31 and 63, and at N = 2^12 for
every item of batches of 64 and 65.
"""

from __future__ import annotations

import numpy as np
import pytest

from conftest import device_context, oracle_context

pytestmark = pytest.mark.gpu


def _setup(name, rotations):
    client, ctx = device_context(name, rotations=rotations)
    orc = oracle_context(name)
    orc.gen_relin_key()
    for r in rotations:
        orc.gen_rotation_key(orc.galois_elt(r))
    return client, ctx, orc


@pytest.mark.slow
def test_keyswitch_batch_of_64_full_size():
    from easyfhe import fhe

    rot = 1 << 9
    client, ctx, orc = _setup("keyswitch", (rot,))
    slots, L = ctx.max_slots, ctx.L
    rng = np.random.default_rng(0)
    zs = [rng.uniform(-1, 1, slots) for _ in range(64)]
    cts = [client.encrypt(z, slots=slots, enc_id=3000 + i) for i, z in enumerate(zs)]
    rots = fhe.homo_rotate_many(cts, rot, ctx)
    prods = fhe.homo_mul_relin_rescale_many(cts, rots, ctx)
    for i in (0, 31, 63):
        ref = orc.encrypt(zs[i], slots=slots, scale=ctx.scale_at(L), limbs=L, enc_id=3000 + i)
        rref = orc.rotate_g(ref, orc.galois_elt(rot))
        assert np.array_equal(rots[i].download(), rref), i
        pref = orc.rescale(orc.relinearize(orc.tensor(ref, rref)))
        assert np.array_equal(prods[i].download(), pref), i
        # decrypted: one key switch, then a product (tolerance 1e-6 as for the
        # single-ciphertext path)
        assert np.abs(client.decrypt(rots[i]) - np.roll(zs[i], -rot)).max() < 1e-6
        assert np.abs(client.decrypt(prods[i]) - zs[i] * np.roll(zs[i], -rot)).max() < 1e-6


@pytest.mark.parametrize("n", [64, 65])
def test_keyswitch_batches_every_item(n):
    from easyfhe import fhe

    client, ctx, orc = _setup("small", (3,))
    slots, L = ctx.max_slots, ctx.L
    rng = np.random.default_rng(n)
    zs = [rng.uniform(-1, 1, slots) for _ in range(n)]
    cts = [client.encrypt(z, slots=slots, enc_id=4000 + i) for i, z in enumerate(zs)]
    rots = fhe.homo_rotate_many(cts, 3, ctx)
    prods = fhe.homo_mul_relin_rescale_many(cts, rots, ctx)
    ext = fhe.homo_mul_relin_rescale_many(cts, cts, ctx, primes=2)
    for i in range(n):
        ref = orc.encrypt(zs[i], slots=slots, scale=ctx.scale_at(L), limbs=L, enc_id=4000 + i)
        rref = orc.rotate_g(ref, orc.galois_elt(3))
        assert np.array_equal(rots[i].download(), rref), i
        assert np.array_equal(prods[i].download(),
                              orc.rescale(orc.relinearize(orc.tensor(ref, rref)))), i
        assert np.array_equal(ext[i].download(),
                              orc.rescale(orc.rescale(orc.relinearize(orc.tensor(ref, ref))))), i
    # the rescale path splits 2-polynomial batches at 32 ciphertexts
    many = fhe.rescale_many(prods, ctx, primes=1)
    for i in (0, 31, 32, n - 1):
        assert np.array_equal(many[i].download(), orc.rescale(prods[i].download())), i


@pytest.mark.parametrize("name", ["small", "keyswitch"])
def test_postop_batches_past_64_match_single(name):
    """The fused product's post-operation (x2, - sub) indexes each launch of
    64 ciphertexts' subtrahends from that launch's first item: items 0, 63,
    64 and 65 of a batch of 66 equal the same pair multiplied alone (each
    single-pair form is held to the oracle by the parity tests)."""
    from easyfhe import fhe

    client, ctx = device_context(name)
    slots = ctx.max_slots
    rng = np.random.default_rng(66)
    n = 66
    zs = [rng.uniform(-1, 1, slots) for _ in range(n)]
    cts = [client.encrypt(z, slots=slots, enc_id=5000 + i) for i, z in enumerate(zs)]
    b = cts[::-1]
    subs = cts[1:] + cts[:1]
    outs = fhe.homo_mul_relin_rescale_postop_many(cts, b, ctx, apply_double=True, sub=subs)
    for i in (0, 63, 64, 65):
        one = fhe.homo_mul_relin_rescale_postop_many([cts[i]], [b[i]], ctx, apply_double=True,
                                                    sub=[subs[i]])[0]
        assert np.array_equal(outs[i].download(), one.download()), i
    ratio = subs[65].state.scaling_factor / outs[65].state.scaling_factor
    want = 2 * zs[65] * zs[0] - zs[0] * ratio
    assert np.abs(client.decrypt(outs[65]) - want).max() < 1e-5
