"""The per-context plaintext cache of constant rows: a hit returns the same
device objects with the same words as a fresh encode, callers' release() is
a no-op while cached, different scales or levels do not collide, and the
least recently used entries go back to the device beyond the byte cap."""

from __future__ import annotations

import numpy as np
import pytest

from conftest import device_context

pytestmark = pytest.mark.gpu


def test_cached_rows_match_a_fresh_encode_and_survive_release(monkeypatch):
    from easyfhe import fhe

    client, ctx = device_context("small")
    rng = np.random.default_rng(3)
    rows = rng.uniform(-1, 1, (3, ctx.max_slots))
    L, sc = ctx.L, ctx.scale_at(ctx.L)
    a = fhe.encode_rows_cached(ctx, rows, limbs=L, scale=sc, slots=ctx.max_slots)
    fresh = fhe.encode_rows(ctx, rows, limbs=L, scale=sc, slots=ctx.max_slots)
    for p, q in zip(a, fresh):
        assert np.array_equal(p.download(), q.download())
    for p in a:
        p.release()  # pinned: stays valid
    b = fhe.encode_rows_cached(ctx, rows.copy(), limbs=L, scale=sc, slots=ctx.max_slots)
    assert [p.handle for p in b] == [p.handle for p in a]
    for p, q in zip(b, fresh):
        assert np.array_equal(p.download(), q.download())
    # another scale, another level, other rows: other entries
    c = fhe.encode_rows_cached(ctx, rows, limbs=L, scale=2 * sc, slots=ctx.max_slots)
    d = fhe.encode_rows_cached(ctx, rows, limbs=L - 1, scale=sc, slots=ctx.max_slots)
    e = fhe.encode_rows_cached(ctx, rows[::-1], limbs=L, scale=sc, slots=ctx.max_slots)
    handles = {p.handle for p in a}
    for other in (c, d, e):
        assert not handles & {p.handle for p in other}
    # a cap below two entries keeps only the most recent one
    monkeypatch.setattr(fhe, "PLAINTEXT_CACHE_BYTES", 1)
    f = fhe.encode_rows_cached(ctx, rows[:1], limbs=L, scale=sc, slots=ctx.max_slots)
    assert len(ctx._pt_cache) == 1
    assert all(p._h is None for p in a)  # dropped and released
    assert f[0]._h is not None
    fhe.clear_plaintext_cache(ctx)
    assert f[0]._h is None
    for q in fresh:
        q.release()
    ctx.close()
