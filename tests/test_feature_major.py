"""Feature-major layouts and the linear plan (CPU).

Pinned by the reference's statements of its production schedule
(llama3fhe/operators/linear/config.py:108-123: B = 64, one anchor block,
512-row chunks -> 8 chunks of 8 giants for D = 4096, lanes 8) and by the
slot formula slot(d, t) = d * lanes + t of layouts/feature_major.py:15-18.
"""

from __future__ import annotations

import numpy as np
import pytest

from feature_major import (FeatureMajorPrefillLayout, LinearCarrierLayout, LinearOperatorConfig,
                           LinearPlan, linear_rotations)


def test_layout_slots_and_round_trip():
    lay = FeatureMajorPrefillLayout(seq_len=20, hidden_dim=8, slots=32)
    assert (lay.token_lanes, lay.cipher_count) == (4, 5)
    rng = np.random.default_rng(0)
    rows = rng.standard_normal((20, 8))
    packed = lay.pack(rows)
    for tok in range(20):
        c, t = divmod(tok, 4)
        for d in range(8):
            assert packed[c, lay.slot(d, t)] == rows[tok, d]
    assert np.array_equal(lay.unpack(packed), rows.astype(np.float32))
    assert [lay.active_tokens(i) for i in range(5)] == [4, 4, 4, 4, 4]
    short = FeatureMajorPrefillLayout(seq_len=18, hidden_dim=8, slots=32)
    assert short.active_tokens(4) == 2 and np.all(short.pack(rows[:18])[4, 2::4] == 0)
    prod = FeatureMajorPrefillLayout()
    assert (prod.tokens_per_cipher, prod.cipher_count) == (8, 16)
    carrier = LinearCarrierLayout(seq_len=8, dimension=4096)
    assert carrier.unpack(carrier.pack(np.ones((8, 4096))), output_dim=3072).shape == (8, 3072)
    with pytest.raises(ValueError):
        FeatureMajorPrefillLayout(seq_len=8, hidden_dim=12, slots=48)


def test_production_plan():
    cfg = LinearOperatorConfig()
    plan = cfg.plan(dimension=4096, token_lanes=8)
    assert plan.giant_steps == 64 and plan.chunk_giants == 8
    assert [(c.giant_base, c.giant_count) for c in plan.chunks] == [(8 * i, 8) for i in range(8)]
    assert plan.giant_offset == 512 and plan.baby_offsets[:3] == (0, 8, 16)
    assert not plan.anchor_enabled
    assert plan.baby_key_offsets == tuple(8 * b for b in range(1, 64))
    keys = linear_rotations(dimension=4096, token_lanes=8)
    assert set(keys) == set(8 * b for b in range(1, 65)) | {512 * 8 * i for i in range(1, 8)}
    conj = linear_rotations(dimension=4096, token_lanes=8, slots=32768, include_conjugation=True)
    assert 4 * 32768 - 1 in conj


def test_anchored_and_uneven_plans():
    plan = LinearPlan(dimension=128, token_lanes=32, baby_steps=16, baby_anchor_step=4,
                      max_plaintext_rows=48)
    assert plan.anchor_enabled
    assert plan.baby_key_offsets == (32, 64, 96, 128)
    assert [(c.giant_base, c.giant_count) for c in plan.chunks] == [(0, 3), (3, 3), (6, 2)]
    for bad in (dict(baby_steps=24), dict(baby_anchor_step=1), dict(max_plaintext_rows=8)):
        kw = dict(dimension=128, token_lanes=32, baby_steps=16, baby_anchor_step=-1,
                  max_plaintext_rows=32)
        kw.update(bad)
        with pytest.raises(ValueError):
            LinearPlan(**kw)
    with pytest.raises(ValueError):
        LinearOperatorConfig(hoist_strategy="fast")
