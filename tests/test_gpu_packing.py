"""Device diagonal packers (token-lane and structured) against the oracle.

The packed plaintexts must be bit-identical to the oracle's encoding of the
diagonal rows computed here in numpy from the layout formula
row(g, b)[slot] = W[(f - g B) mod D, (f + b) mod D], f = slot // lanes
(reference operators/linear/weight.py:18-47), and for the structured packer
of the physical matrix W[o, i] = cs[i] (rs[o] src[rsrc[o]][rrow[o], col[i]] +
1j is[o] src[isrc[o]][irow[o], col[i]]) (reference structured_weight.py:1-20).
"""

from __future__ import annotations

import numpy as np
import pytest

from conftest import device_context, oracle_context

pytestmark = pytest.mark.gpu


def _rows(W, slots, lanes, B, g0, G):
    D = W.shape[0]
    f = np.arange(slots) // lanes
    return np.stack([W[(f - (g0 + g) * B) % D, (f + b) % D] for g in range(G) for b in range(B)])


def _materialize(sources, m, D):
    W = np.zeros((D, D), dtype=np.complex128)
    for o in range(D):
        for i in range(D):
            c = m["column"][i]
            if c < 0:
                continue
            v = 0j
            if m["real_source"][o] >= 0:
                v += m["real_scale"][o] * sources[m["real_source"][o]][m["real_row"][o], c]
            if m["imag_source"][o] >= 0:
                v += 1j * m["imag_scale"][o] * sources[m["imag_source"][o]][m["imag_row"][o], c]
            W[o, i] = m["column_scale"][i] * v
    return W


@pytest.fixture(scope="module")
def matvec_pair():
    client, ctx = device_context("matvec", relin=False)
    return client, ctx, oracle_context("matvec")


@pytest.mark.parametrize("dtype,is_ext", [(np.float64, False), (np.float32, False),
                                          (np.complex128, False), (np.float64, True)])
def test_token_lane_packer_bit_exact(matvec_pair, dtype, is_ext):
    import easyfhe
    from easyfhe import fhe, packing

    client, ctx, orc = matvec_pair
    slots, D, lanes, B, g0, G = ctx.max_slots, 128, 32, 16, 2, 3
    rng = np.random.default_rng(3)
    W = rng.uniform(-1, 1, (D, D))
    if dtype == np.complex128:
        W = W + 1j * rng.uniform(-1, 1, (D, D))
    W = W.astype(dtype)
    dev = easyfhe.from_numpy(W).to("cuda", context=ctx)
    assert dev.is_cuda and np.array_equal(dev.numpy(), W)
    chunk = packing.pack_token_lane_bsgs_weight_chunk(dev, slots=slots, dimension=D,
                                                      token_lanes=lanes, baby_steps=B,
                                                      giant_base=g0, giant_count=G)
    bundle = fhe.ConstantBundle({"w": fhe.PackedRaw(chunk)}, cache_mode="plain")
    sc = 2.0**40
    state = fhe.CipherState(cur_limbs=ctx.L, scaling_factor=sc)
    pts = bundle.plaintext("w", state=state, slots=slots, context=ctx, is_ext=is_ext)
    rows = _rows(W.astype(np.complex128), slots, lanes, B, g0, G)
    assert len(pts) == len(rows)
    for i in range(len(rows)):
        want = orc.encode(rows[i], slots=slots, scale=sc, limbs=ctx.L, is_ext=is_ext)
        assert np.array_equal(pts[i].download()[0], want), i
    assert bundle.cache_info()["entries"] == len(rows)


def test_structured_packer_bit_exact(matvec_pair):
    import easyfhe
    from easyfhe import fhe, packing

    client, ctx, orc = matvec_pair
    slots, D, lanes, B, g0, G = ctx.max_slots, 128, 32, 8, 1, 2
    rng = np.random.default_rng(4)
    src = [rng.uniform(-1, 1, (64, 100)), rng.uniform(-1, 1, (80, 100))]
    m = {
        "real_source": rng.integers(-1, 2, D),
        "imag_source": rng.integers(-1, 2, D),
        "real_scale": rng.uniform(0.5, 2, D),
        "imag_scale": rng.uniform(0.5, 2, D),
        "column": np.concatenate([rng.permutation(100), -np.ones(D - 100, dtype=np.int64)]),
        "column_scale": rng.uniform(0.5, 2, D),
    }
    for part in ("real", "imag"):
        s = m[f"{part}_source"]
        m[f"{part}_row"] = np.where(s == 0, rng.integers(0, 64, D),
                                    np.where(s == 1, rng.integers(0, 80, D), -1))
    devs = [easyfhe.from_numpy(a).to("cuda", context=ctx) for a in src]
    chunk = packing.pack_structured_token_lane_bsgs_weight_chunk(
        devs, m, slots=slots, dimension=D, token_lanes=lanes, baby_steps=B, giant_base=g0,
        giant_count=G)
    pts = chunk.encode(ctx, limbs=ctx.L, scale=2.0**40)
    rows = _rows(_materialize(src, m, D), slots, lanes, B, g0, G)
    for i in range(len(rows)):
        want = orc.encode(rows[i], slots=slots, scale=2.0**40, limbs=ctx.L)
        assert np.array_equal(pts[i].download()[0], want), i
    # indices outside the sources are rejected before any device work
    bad = dict(m, real_row=np.where(m["real_source"] == 0, 64, m["real_row"]))
    with pytest.raises(ValueError):
        packing.pack_structured_token_lane_bsgs_weight_chunk(
            devs, bad, slots=slots, dimension=D, token_lanes=lanes, baby_steps=B,
            giant_base=g0, giant_count=G).encode(ctx, limbs=ctx.L, scale=2.0**40)
    bad = dict(m, column=np.where(m["column"] == 0, 100, m["column"]))
    with pytest.raises(ValueError):
        packing.pack_structured_token_lane_bsgs_weight_chunk(
            devs, bad, slots=slots, dimension=D, token_lanes=lanes, baby_steps=B,
            giant_base=g0, giant_count=G).encode(ctx, limbs=ctx.L, scale=2.0**40)


def test_packed_matvec_decrypts_to_wx():
    """The matvec workload with device-packed, extended plaintexts."""
    import easyfhe
    from easyfhe import fhe, packing

    D, lanes, B, G = 128, 32, 16, 8
    rots = tuple(lanes * b for b in range(1, B)) + (B * lanes,)
    client, ctx = device_context("matvec", rotations=rots)
    slots = ctx.max_slots
    rng = np.random.default_rng(0)
    W = rng.uniform(-1, 1, (D, D))
    x = rng.uniform(-1, 1, D)
    packed = np.zeros(slots)
    packed[np.arange(D) * lanes] = x
    ct = client.encrypt(packed, slots=slots, enc_id=41)
    chunk = packing.pack_token_lane_bsgs_weight_chunk(
        easyfhe.from_numpy(W).to("cuda", context=ctx), slots=slots, dimension=D,
        token_lanes=lanes, baby_steps=B, giant_base=0, giant_count=G)
    bundle = fhe.ConstantBundle({"w": fhe.UnpackedRaw(None, lambda src, s, c: chunk)})
    pts = bundle.plaintext("w", state=fhe.CipherState(cur_limbs=ctx.L), slots=slots,
                           context=ctx, is_ext=True)
    acc = fhe.hoisted_mac_sum(ct, [lanes * b for b in range(B)], pts, B * lanes, G, ctx,
                              strategy="ext_normal")
    dec = client.decrypt(fhe.rescale(acc, ctx))[np.arange(D) * lanes]
    assert np.abs(dec - W @ x).max() < 1e-5
