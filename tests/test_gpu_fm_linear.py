"""Feature-major linear engine on the GPU (matvec context: N = 2^13, 4096
slots, 4 x 40-bit limbs): D = 128, 32 token lanes, B = 16 and 2-giant chunks
(4 chunks), three input ciphertexts (96 tokens).

* the batched chunk MAC (fhe.hoisted_mac_sum_many) gives the same words as one
  hoisted_mac_sum per input with the same babies and plaintexts, also for a
  chunk of 16 giants (B = 8, one 128-row chunk: the 16-group pass);
* the decrypted outputs are W x for every token (fp64 reference).
"""

from __future__ import annotations

import numpy as np
import pytest

from conftest import device_context

pytestmark = pytest.mark.gpu

D, LANES = 128, 32


def _setup(cfg, extra=(), chain="matvec", lanes=LANES):
    from feature_major import FeatureMajorPrefillLayout, linear_rotations

    rots = linear_rotations(dimension=D, token_lanes=lanes, operator_config=cfg)
    client, ctx = device_context(chain, rotations=tuple(sorted(set(rots) | set(extra))))
    lay = FeatureMajorPrefillLayout(seq_len=3 * lanes, hidden_dim=D, slots=ctx.max_slots)
    rng = np.random.default_rng(0)
    W = rng.uniform(-1, 1, (D, D))
    X = rng.uniform(-1, 1, (lay.seq_len, D))
    packed = lay.pack(X)
    cts = [client.encrypt(packed[i], enc_id=300 + i) for i in range(lay.cipher_count)]
    return client, ctx, lay, W, X, cts


# (babies, anchor step, plaintext rows per chunk, chain, token lanes): chunks
# of 2 giants, and one chunk of 16 giants (the batched MAC's 16-group pass) on
# the matvec chain (every limb on the fp64 kernel) and on a chain whose 60-bit
# q_0 takes the 64-bit kernel (N = 2^12: 16 lanes of 128 features)
@pytest.mark.parametrize("schedule", [(16, 16, 32, "matvec", LANES), (8, 8, 128, "matvec", LANES),
                                      (8, 8, 128, "small", 16)])
def test_fm_linear_matches_per_input_bsgs_and_wx(schedule):
    from easyfhe import fhe
    from feature_major import LinearOperator, LinearOperatorConfig, LinearWeight

    b, anchor, rows, chain, lanes = schedule
    cfg = LinearOperatorConfig(baby_steps=b, baby_anchor_step=anchor, max_plaintext_rows=rows)
    client, ctx, lay, W, X, cts = _setup(cfg, chain=chain, lanes=lanes)
    op = LinearOperator(context=ctx, token_lanes=lanes, config=cfg)
    with LinearWeight(W, context=ctx) as weight:
        outs, profile = op.apply(cts, weight)
        assert set(profile) >= {"baby_precompute", "pack_encode", "online", "rescale"}
        # the same schedule input by input through the single-ciphertext API
        plan = op.plan(D)
        limbs = int(cts[0].state.cur_limbs)
        for i, ct in enumerate(cts):
            babies = fhe.prepare_hoisted_baby_rotations(ct, plan.baby_offsets, ctx,
                                                        baby_anchor_step=plan.baby_anchor_step)
            acc = None
            for chunk in plan.chunks:
                pts = weight.plaintext(plan, chunk, limbs=limbs, operator_config=cfg)
                r = fhe.hoisted_mac_sum(ct, plan.baby_offsets, pts, plan.giant_offset,
                                        chunk.giant_count, ctx, baby_rotations=babies)
                if chunk.giant_base:
                    r = fhe.homo_rotate(r, chunk.giant_base * plan.giant_offset, ctx)
                acc = r if acc is None else fhe.homo_add(acc, r, ctx)
            want = fhe.rescale(acc, ctx)
            assert np.array_equal(outs[i].download(), want.download()), i
    assert op.cache_info()["baby_entries"] == len(cts)
    # a second weight on the same inputs reuses the cached babies
    W2 = np.eye(D)[::-1].copy()
    outs2, _ = op.project(cts, W2)
    assert op.cache_info()["baby_hits"] >= len(cts)
    got = lay.unpack(np.stack([client.decrypt(o) for o in outs]))
    assert np.abs(got - X @ W.T).max() < 1e-5
    got2 = lay.unpack(np.stack([client.decrypt(o) for o in outs2]))
    assert np.abs(got2 - X @ W2.T).max() < 1e-5
    op.close()


@pytest.mark.parametrize("strategy", ["ext_normal", "ext_double_hoist"])
def test_fm_linear_extended_schedule(strategy):
    from feature_major import LinearOperator, LinearOperatorConfig

    cfg = LinearOperatorConfig(baby_steps=16, baby_anchor_step=-1, max_plaintext_rows=32,
                               hoist_strategy=strategy)
    client, ctx, lay, W, X, cts = _setup(cfg)
    with LinearOperator(context=ctx, token_lanes=LANES, config=cfg) as op:
        outs, _ = op.project(cts, W)
    got = lay.unpack(np.stack([client.decrypt(o) for o in outs]))
    assert np.abs(got - X @ W.T).max() < 1e-5


def test_batched_babies_match_single():
    """prepare_hoisted_baby_rotations_many (one ModUp per input, one key read
    per rotation for the batch) = the single-ciphertext form, with and
    without anchored blocks."""
    from easyfhe import fhe
    from feature_major import LinearOperatorConfig

    cfg = LinearOperatorConfig(baby_steps=16, baby_anchor_step=4, max_plaintext_rows=32)
    offs = [LANES * b for b in range(16)]
    client, ctx, lay, W, X, cts = _setup(cfg, extra=offs[1:])
    for anchor in (-1, 4):
        many = fhe.prepare_hoisted_baby_rotations_many(cts, offs, ctx, baby_anchor_step=anchor)
        for ct, got in zip(cts, many):
            want = fhe.prepare_hoisted_baby_rotations(ct, offs, ctx, baby_anchor_step=anchor)
            assert len(got) == len(want) == 16
            for g, w in zip(got, want):
                assert np.array_equal(g.download(), w.download())
