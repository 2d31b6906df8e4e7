"""Host side of the encrypted prefill: the client's embedding lookup and
final logits, and the per-layer series selection from calibrated ranges."""

from __future__ import annotations

import numpy as np
import pytest

from feature_major.model import (LayerRanges, RangeMargins, approximations_for, embed_tokens,
                                 final_logits, layer_ranges)


def test_embed_tokens_rows_and_bounds():
    table = np.arange(20.0).reshape(5, 4)
    assert np.array_equal(embed_tokens([4, 0, 4], table), table[[4, 0, 4]])
    with pytest.raises(IndexError):
        embed_tokens([5], table)
    with pytest.raises(ValueError):
        embed_tokens([], table)


def test_final_logits_is_scale_free_and_picks_the_token():
    rng = np.random.default_rng(0)
    h, head = rng.normal(0, 3, (6, 16)), rng.normal(0, 1, (11, 16))
    gamma = rng.uniform(0.5, 2.0, 16)
    base = final_logits(h, norm_weight=gamma, lm_head=head, eps=0.0)
    # RMSNorm removes any positive scale of the token's row
    assert np.allclose(final_logits(7.5 * h, norm_weight=gamma, lm_head=head, eps=0.0), base)
    # only the chosen token's row matters
    h2 = h.copy()
    h2[:-1] = 0.0
    assert np.allclose(final_logits(h2, norm_weight=gamma, lm_head=head, eps=0.0), base)
    # a unit-RMS row with unit gamma and an identity head returns the row
    row = np.array([1.0, -1.0, 1.0, -1.0])
    assert np.allclose(final_logits(row[None], norm_weight=np.ones(4), lm_head=np.eye(4),
                                    eps=0.0), row)
    assert np.allclose(final_logits(h, norm_weight=gamma, lm_head=head, token_index=2, eps=0.0),
                       final_logits(h[:3], norm_weight=gamma, lm_head=head, eps=0.0))
    with pytest.raises(IndexError):
        final_logits(h, norm_weight=gamma, lm_head=head, token_index=6)
    with pytest.raises(ValueError):
        final_logits(h, norm_weight=gamma, lm_head=head[:, :8])


def test_layer_ranges_reads_the_causal_scores_only():
    x = np.array([[1.0, -1.0], [2.0, 2.0]])
    h1 = np.array([[3.0, 0.0], [0.0, -5.0]])
    scores = np.array([[[0.5, 99.0], [-2.0, 1.5]]])
    r = layer_ranges(x, h1, np.array([[-7.0, 2.0]]), scores)
    assert r.input_mean_square == (1.0, 4.0)
    assert r.post_attention_mean_square == (4.5, 12.5)
    assert r.residual_abs_max == 5.0 and r.gate_abs_max == 7.0
    assert r.score_max == 1.5 and r.score_min == -2.0


def test_approximations_cover_the_ranges():
    r = LayerRanges((0.9, 1.2), (3.0, 5.0), 40.0, 6.5, 9.03, -8.0)
    ap, bound = approximations_for(r)
    lo, hi = ap.input_norm["fit_interval"]
    assert lo <= 0.9 / 4 + 1e-12 and hi >= 1.2 * 4 - 1e-12
    lo, hi = ap.post_attention_norm["fit_interval"]
    assert lo <= 3.0 / 4 + 1e-12 and hi >= 5.0 * 4 - 1e-12
    lo, hi = ap.silu["fit_interval"]
    assert lo <= -6.5 and hi >= 6.5
    assert ap.softmax.shift >= 9.03 + 1.0 and ap.softmax.shift == int(ap.softmax.shift)
    assert ap.softmax.shift + ap.softmax.bound == RangeMargins().score_span
    assert bound == 80.0
    with pytest.raises(ValueError):
        approximations_for(LayerRanges((1, 2), (1, 2), 1.0, 1.0, 19.0, -1.0))


def test_slim_rmsnorm_refresh_shortens_the_last_block():
    """With the post-attention RMSNorm's slim refresh, the last block is the
    smallest depth at which both paths fit: the stream (one level for the
    norm's product, then the MLP, leaving the two limbs the next refresh
    takes) and the slim path (square, pack mask and series below the
    block's input, then a bootstrap input).  The other blocks are unchanged."""
    from easyfhe.chebyshev import chebyshev_depth
    from feature_major.layer import refreshed_layer_depths
    from feature_major.mlp import mlp_depth

    for r in (LayerRanges((0.9, 1.2), (3.0, 5.0), 40.0, 6.5, 9.03, -8.0),
              LayerRanges((1e-4, 5e-4), (1.0, 4.0), 8.0, 6.0, 4.0, -4.0)):
        ap, _ = approximations_for(r)
        d = chebyshev_depth(ap.post_attention_norm["coefficients"])
        for lim in (1, 2):
            for rn in (False, True):
                a0, b0, c0 = refreshed_layer_depths(ap, 128, refresh_normalisers=rn,
                                                    input_limbs=lim)
                a, b, c = refreshed_layer_depths(ap, 128, refresh_normalisers=rn,
                                                 input_limbs=lim, slim_rmsnorm=True)
                assert (a, b) == (a0, b0) and c < c0

                def fits(depth):
                    block_in = depth + 2
                    stream_ok = block_in - 1 - mlp_depth(ap.silu) >= 2
                    slim_ok = block_in - 2 - d >= lim
                    return stream_ok and slim_ok

                assert fits(c) and not fits(c - 1)


def test_refreshed_blocks_partition_the_layer_depth():
    """The three blocks between refreshes use, together, exactly the levels
    of the refresh-free layer, for the prefill's default series."""
    from feature_major.layer import decoder_layer_depth, refreshed_layer_depths

    for r in (LayerRanges((0.9, 1.2), (3.0, 5.0), 40.0, 6.5, 9.03, -8.0),
              LayerRanges((1e-4, 5e-4), (1.0, 4.0), 8.0, 6.0, 4.0, -4.0)):
        ap, _ = approximations_for(r)
        a, b, c = refreshed_layer_depths(ap, 128)
        assert a + b + c == decoder_layer_depth(ap, 128)
        # the score block is the deepest: its bootstrap returns the most limbs
        assert b > max(a, c)
