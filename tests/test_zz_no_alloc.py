"""ckks_rotate_many_noalloc through the C ABI: the rotation into caller-given
outputs with every intermediate in the library's fixed device buffer.

Its outputs must equal ckks_rotate_many's word for word (the same kernels,
the same order of operations), on two calls in a row with the second one
smaller, at N = 2^16 on the key-switch chain and at N = 2^12 with a full
batch of 64, on the default kernels and on the separate key product and
special-limb inverse pass; the context's pool must see no allocation during
the calls.  Two contexts (two streams) that call it alternately without any
host synchronisation share the buffer one call after another.
"""

from __future__ import annotations

import numpy as np
import pytest

from conftest import device_context

pytestmark = pytest.mark.gpu


def _noalloc(ctx, ins, rotation, outs):
    from easyfhe import _native

    _native.check(_native.lib.ckks_rotate_many_noalloc(
        ctx.handle, _native.ptr_array([c.handle for c in ins]), len(ins), int(rotation),
        _native.ptr_array([o.handle for o in outs])))


def _pool(ctx):
    m = ctx.memory_info()
    return m["device_allocations"], m["live_bytes"]


def _check_calls(client, ctx, calls):
    """calls: (limbs, count, rotation) in order; each runs the noalloc entry
    point into fresh outputs, then ckks_rotate_many on the same inputs."""
    from easyfhe import fhe

    rng = np.random.default_rng(5)
    for limbs, count, rot in calls:
        ins = [client.encrypt(rng.uniform(-1, 1, ctx.max_slots), cur_limbs=limbs,
                              enc_id=9000 + 100 * limbs + i) for i in range(count)]
        outs = [client.encrypt(np.zeros(ctx.max_slots), cur_limbs=limbs, enc_id=9500 + i)
                for i in range(count)]
        ctx.synchronize()
        before = _pool(ctx)
        _noalloc(ctx, ins, rot, outs)
        ctx.synchronize()
        assert _pool(ctx) == before, (limbs, count)
        want = fhe.homo_rotate_many(ins, rot, ctx)
        for i in range(count):
            assert np.array_equal(outs[i].download(), want[i].download()), (limbs, count, i)
            assert outs[i].state.cur_limbs == limbs
        for c in ins + outs + want:
            c.release()


def test_noalloc_rotation_full_size_two_calls():
    """One ciphertext at 36 limbs (186 MiB of scratch), then one at 12 limbs."""
    client, ctx = device_context("keyswitch", rotations=(5, 1 << 12))
    _check_calls(client, ctx, [(ctx.L, 1, 5), (12, 1, 1 << 12)])
    # two ciphertexts at 36 limbs need 372 MiB: rejected before any launch
    from easyfhe import fhe  # noqa: F401

    ins = [client.encrypt(np.zeros(ctx.max_slots), enc_id=9900 + i) for i in range(2)]
    outs = [client.encrypt(np.zeros(ctx.max_slots), enc_id=9910 + i) for i in range(2)]
    with pytest.raises(ValueError, match="scratch"):
        _noalloc(ctx, ins, 5, outs)
    with pytest.raises(ValueError):
        _noalloc(ctx, ins[:1], 5, ins[:1])  # output aliasing its input
    ctx.close()


@pytest.mark.parametrize("env", [{}, {"CKKS_KEYSWITCH_FUSED": "0"},
                                 {"CKKS_KS_SPECIAL_INV": "0"}])
def test_noalloc_rotation_batches_two_calls(env, monkeypatch):
    """64 ciphertexts at N = 2^12, then 3 at a lower level; the identity
    rotation copies.  The key-switch kernel choices are read at context
    creation."""
    for k, v in env.items():
        monkeypatch.setenv(k, v)
    client, ctx = device_context("small", rotations=(1, -3))
    _check_calls(client, ctx, [(ctx.L, 64, 1), (ctx.L - 2, 3, -3), (ctx.L, 2, 0)])
    ctx.close()


def test_noalloc_two_contexts_alternate_without_sync():
    """Contexts A and B (own streams, own keys) call the entry point in turn,
    four calls each, with no synchronisation between the calls; every output
    equals that context's ckks_rotate_many afterwards."""
    from easyfhe import fhe

    rng = np.random.default_rng(11)
    pairs = [device_context("small", seed=s, rotations=(1, 7)) for s in (3, 4)]
    calls = []
    for step in range(8):
        client, ctx = pairs[step % 2]
        rot = (1, 7)[(step // 2) % 2]
        count = 64 if step < 2 else 8
        ins = [client.encrypt(rng.uniform(-1, 1, ctx.max_slots), enc_id=7000 + 100 * step + i)
               for i in range(count)]
        outs = [client.encrypt(np.zeros(ctx.max_slots), enc_id=7900 + i) for i in range(count)]
        calls.append((ctx, ins, rot, outs))
    for client, ctx in pairs:
        ctx.synchronize()
    for ctx, ins, rot, outs in calls:
        _noalloc(ctx, ins, rot, outs)  # no host wait between the calls
    for ctx, ins, rot, outs in calls:
        want = fhe.homo_rotate_many(ins, rot, ctx)
        for i in range(len(ins)):
            assert np.array_equal(outs[i].download(), want[i].download()), (rot, i)
    for client, ctx in pairs:
        ctx.close()
