"""Batched limb-wise sums: homo_add_many / homo_sub_many give, word for
word, what homo_add / homo_sub give pair by pair, past one launch's 64
pairs, and refuse pairs of different shapes."""

from __future__ import annotations

import numpy as np
import pytest

from conftest import device_context

pytestmark = pytest.mark.gpu


def test_add_many_matches_pairwise_adds():
    from easyfhe import fhe

    client, ctx = device_context("small")
    rng = np.random.default_rng(5)
    n = 70  # two launches
    a = [client.encrypt(rng.uniform(-1, 1, ctx.max_slots), enc_id=3000 + i) for i in range(n)]
    b = [client.encrypt(rng.uniform(-1, 1, ctx.max_slots), enc_id=4000 + i) for i in range(n)]
    for op_many, op in ((fhe.homo_add_many, fhe.homo_add), (fhe.homo_sub_many, fhe.homo_sub)):
        got = op_many(a, b, ctx)
        for x, y, g in zip(a, b, got):
            want = op(x, y, ctx)
            assert np.array_equal(g.download(), want.download())
            want.release()
        for g in got:
            g.release()
    # one operand a level lower: refused before any output exists
    low = fhe.align_to(b[1], b[1].state.replace(cur_limbs=ctx.L - 1, scaling_factor=None), ctx)
    with pytest.raises(ValueError, match="limb count"):
        fhe.homo_add_many(a[:2], [b[0], low], ctx)
    for c in a + b + [low]:
        c.release()
    ctx.close()
