"""Polynomial evaluation and bootstrapping on the device (decrypted values).

Bootstrapping has no bit-level oracle (the reference's EasyFHE program is
absent); it is pinned by precision: -log2 max |dec(bts(ct)) - m| against the
encrypted fp64 message, and by its CPU model (test_bootstrap_model.py).  The
Chebyshev evaluator is compared with the fp64 series value.
"""

from __future__ import annotations

import math

import numpy as np
import pytest

from conftest import device_context

pytestmark = pytest.mark.gpu

# N = 2^12, 60-bit q_0 + 30 x 40-bit, dnum 3 (11-limb digits), 11 x 60-bit P
BOOT = dict(log_n=12, depth=30, dnum=3, dcrt_bits=40, first_mod=60, special_bits=60)


@pytest.fixture(scope="module")
def boot_ctx():
    return device_context(BOOT)


def test_chebyshev_series_cipher(boot_ctx):
    from easyfhe import chebyshev as cheb

    client, ctx = boot_ctx
    coeffs = cheb.chebyshev_coefficients(math.tanh, -4.0, 4.0, 27)
    rng = np.random.default_rng(5)
    x = rng.uniform(-4, 4, ctx.max_slots)
    ct = client.encrypt(x, cur_limbs=ctx.L, enc_id=71)
    out = cheb.eval_chebyshev_series_cipher(ct, coeffs, lower_bound=-4.0, upper_bound=4.0,
                                            crypto_context=ctx)
    assert out.state.cur_limbs == ctx.L - cheb.series_depth(coeffs)
    got = client.decrypt(out)
    want = cheb.evaluate_direct(x, coeffs, -4.0, 4.0)
    err = np.abs(got - want).max()
    print(f"tanh deg 27: depth {cheb.series_depth(coeffs)}, max err {err:.3e}")
    assert err < 1e-6


def test_chebyshev_two_prime_ladder(boot_ctx):
    """A ladder with two primes per level keeps scales exact at ~2^80."""
    from easyfhe import chebyshev as cheb
    from easyfhe import fhe

    client, ctx = boot_ctx
    primes = [int(q) for q in ctx.primes()[: ctx.L]]
    coeffs = cheb.chebyshev_coefficients(lambda v: math.cos(3.0 * v), -1.0, 1.0, 20)
    depth = cheb.chebyshev_depth(coeffs)
    top = ctx.L - 1
    lad = cheb.Ladder(primes, top - 1, float(primes[top - 3]) * float(primes[top - 2]), 2, depth)
    ops = cheb.LadderOps(ctx, lad)
    rng = np.random.default_rng(6)
    x = rng.uniform(-1, 1, ctx.max_slots)
    ct = client.encrypt(x, cur_limbs=ctx.L, enc_id=72)
    y = ops.combine([(ct, 1.0)], 0.0, 0)
    out = cheb.evaluate(ops, y, coeffs)
    assert out.ct.state.cur_limbs == lad.limbs[depth]
    err = np.abs(client.decrypt(out.ct) - cheb.evaluate_direct(x, coeffs)).max()
    print(f"cos(3x) deg 20 at 2^80: max err {err:.3e}")
    assert err < 1e-8
    fhe.homo_add(out.ct, out.ct, ctx)  # scales equal on the ladder


@pytest.mark.parametrize("budget", [(3, 3), (2, 2)])
def test_bootstrap_precision(boot_ctx, budget):
    from easyfhe.bs import openfhe as bs

    client, ctx = boot_ctx
    n = ctx.max_slots
    spec = bs.BootstrapSpec(log_slots=ctx.logN - 1, level_budget=budget, output_levels=3)
    prog = bs.generate(ctx, spec)
    rng = np.random.default_rng(7)
    z = rng.uniform(-1, 1, n) + 1j * rng.uniform(-1, 1, n)
    ct = client.encrypt(z, cur_limbs=1, enc_id=73)
    out = bs.bootstrap(ct, ctx, prog)
    assert out.state.cur_limbs == spec.output_levels + 1
    err = np.abs(client.decrypt_complex(out) - z).max()
    bits = -math.log2(err)
    print(f"bootstrap {budget}: raise to {prog.raise_limbs} limbs, {bits:.1f} bits")
    assert bits > 14
    # the refreshed ciphertext computes: square it and rescale
    from easyfhe import fhe

    sq = fhe.rescale(fhe.homo_mul_relin(out, out, ctx), ctx)
    err2 = np.abs(client.decrypt_complex(sq) - z * z).max()
    assert err2 < 4 * err + 1e-6
    prog.release()


def test_bootstrap_two_pass_gains_precision(boot_ctx):
    """From a deliberately coarse first pass (CoeffToSlot diagonals at 2^45,
    ~17 bits) the second pass removes the first one's error."""
    from easyfhe.bs import openfhe as bs

    client, ctx = boot_ctx
    n = ctx.max_slots
    spec = bs.BootstrapSpec(log_slots=ctx.logN - 1, level_budget=(3, 3), output_levels=3)
    prog = bs.generate(ctx, spec, bs.BootstrapParams(cts_pt_bits=45))
    rng = np.random.default_rng(8)
    z = rng.uniform(-1, 1, n)
    ct = client.encrypt(z, cur_limbs=2, enc_id=74)
    one = bs.bootstrap(ct, ctx, prog)
    two = bs.bootstrap_iterated(ct, ctx, prog, iterations=2, precision_bits=8)
    assert two.state.cur_limbs == one.state.cur_limbs - 1
    e1 = np.abs(client.decrypt_complex(one) - z).max()
    e2 = np.abs(client.decrypt_complex(two) - z).max()
    print(f"one pass {-math.log2(e1):.1f} bits, two passes {-math.log2(e2):.1f} bits")
    assert e1 > 2.0**-20
    assert e2 < e1 / 16


def test_reference_meta_bts_sequence_gains_precision(boot_ctx):
    """The reference's two-pass refresh (operators/nonlinear/bootstrap.py:404-433)
    restated with the fhe calls it makes, on an input whose scale (1.37 x 2^40)
    differs from the bootstrap output's: its first align_to must change the
    scale (a ValueError there makes the reference fall back to one pass), and
    the second pass must gain at least 4 bits over a coarse first pass."""
    from easyfhe import fhe
    from easyfhe.bs import openfhe as bs

    client, ctx = boot_ctx
    n = ctx.max_slots
    prog = bs.generate(ctx, bs.BootstrapSpec(log_slots=ctx.logN - 1, level_budget=(3, 3),
                                             output_levels=3), bs.BootstrapParams(cts_pt_bits=45))
    rng = np.random.default_rng(18)
    z = rng.uniform(-1, 1, n)
    original = client.encrypt(z, cur_limbs=2, scaling_factor=1.37 * 2.0**40, enc_id=76)
    factor = 1 << 8

    def times_int(ct, v):
        enc = fhe.encode_scalar(int(v), cur_limbs=int(ct.state.cur_limbs), scale_degree=0,
                                mode="integer", context=ctx)
        return fhe.homo_mul_scalar(ct, enc, ctx)

    first = bs.bootstrap(original, ctx, prog)
    first_scaled = times_int(first, factor)
    first_down = fhe.align_to(first_scaled, original.state, ctx)
    assert first_down.state.cur_limbs == 2
    original_scaled = fhe.align_to(times_int(original, factor), first_down.state, ctx)
    error = bs.bootstrap(fhe.homo_sub(first_down, original_scaled, ctx), ctx, prog)
    first_aligned = fhe.align_to(first_scaled, error.state, ctx)
    error_aligned = fhe.align_to(error, first_aligned.state, ctx)
    corrected = fhe.homo_sub(first_aligned, error_aligned, ctx)
    enc = fhe.encode_scalar(1.0 / factor, cur_limbs=int(corrected.state.cur_limbs),
                            scale_degree=1, scaling_factor=corrected.state.scaling_factor,
                            context=ctx)
    two = fhe.homo_mul_scalar_rescale(corrected, enc, ctx)
    e1 = np.abs(client.decrypt(first) - z).max()
    e2 = np.abs(client.decrypt(two) - z).max()
    print(f"reference Meta-BTS: one pass {-math.log2(e1):.1f} bits, two {-math.log2(e2):.1f}")
    assert e2 < e1 / 16
    prog.release()


def test_bootstrap_many_matches_single(boot_ctx):
    """Batched groups run the same arithmetic per ciphertext: identical limbs."""
    from easyfhe.bs import openfhe as bs

    client, ctx = boot_ctx
    n = ctx.max_slots
    prog = bs.generate(ctx, bs.BootstrapSpec(log_slots=ctx.logN - 1, level_budget=(3, 3),
                                             output_levels=3))
    rng = np.random.default_rng(9)
    zs = [rng.uniform(-1, 1, n) for _ in range(3)]
    cts = [client.encrypt(z, cur_limbs=1, enc_id=80 + i) for i, z in enumerate(zs)]
    many = bs.bootstrap_many(cts, ctx, prog, group=2)
    for ct, got in zip(cts, many):
        assert np.array_equal(got.download(), bs.bootstrap(ct, ctx, prog).download())
    for z, got in zip(zs, many):
        assert -math.log2(np.abs(client.decrypt_complex(got) - z).max()) > 14


def test_bootstrap_pair_refreshes_two_real_streams(boot_ctx):
    from easyfhe.bs import openfhe as bs

    client, ctx = boot_ctx
    n = ctx.max_slots
    prog = bs.generate(ctx, bs.BootstrapSpec(log_slots=ctx.logN - 1, level_budget=(3, 3),
                                             output_levels=3))
    rng = np.random.default_rng(10)
    a, b = rng.uniform(-1, 1, n), rng.uniform(-1, 1, n)
    ca = client.encrypt(a, cur_limbs=1, enc_id=90)
    cb = client.encrypt(b, cur_limbs=1, enc_id=91)
    ra, rb = bs.bootstrap_pair(ca, cb, ctx, prog)
    for got, want in ((ra, a), (rb, b)):
        err = np.abs(client.decrypt_complex(got) - want).max()
        assert -math.log2(err) > 14, err


@pytest.mark.parametrize("log_slots,budget,packed", [(7, (3, 3), True), (7, (3, 3), False),
                                                     (4, (2, 2), True), (10, (3, 3), True),
                                                     (10, (3, 3), False)])
def test_bootstrap_sparse_slots(boot_ctx, log_slots, budget, packed):
    """A sparse ciphertext (128 slots: the reference's slim RMSNorm program
    shape) through the sparse program: the sub-sum (rotations by n, 2n, ..
    N/4) leaves the raised polynomial's coefficients at multiples of
    N / 2n, then the n-slot CoeffToSlot, EvalMod and SlotToCoeff.  With
    ``packed`` the real and imaginary parts share one 2n-periodic vector
    (one EvalMod per ciphertext), else they run through two.  One
    bootstrap and a batched group of three agree with each other and with
    the message."""
    from easyfhe.bs import openfhe as bs

    client, ctx = boot_ctx
    slots = 1 << log_slots
    prog = bs.generate(ctx, bs.BootstrapSpec(log_slots=log_slots, level_budget=budget,
                                             output_levels=3),
                       bs.BootstrapParams(packed_evalmod=packed))
    assert prog.spec.slots == slots and prog.packed == packed
    assert prog.subsum == [slots << k for k in range(ctx.logN - 1 - log_slots)]
    rng = np.random.default_rng(11)
    zs = [rng.uniform(-1, 1, slots) for _ in range(3)]
    cts = [client.encrypt(z, slots=slots, cur_limbs=1, enc_id=95 + i) for i, z in enumerate(zs)]
    out = bs.bootstrap(cts[0], ctx, prog)
    assert out.slots == slots and out.state.cur_limbs == 4
    err = np.abs(client.decrypt_complex(out) - zs[0]).max()
    assert -math.log2(err) > 14, err
    many = bs.bootstrap_many(cts, ctx, prog, group=3)
    assert np.array_equal(many[0].download(), out.download())
    for o, z in zip(many, zs):
        assert -math.log2(np.abs(client.decrypt_complex(o) - z).max()) > 14


def test_refresh_point_pairs_and_clamped_drop(boot_ctx):
    """A residual refresh point: 4 real streams refreshed by 2 paired
    bootstraps, then the modulus drop clamped to the consumer budget
    (reference operators/norm/refresh.py:70-93, 207-242)."""
    from easyfhe.bs import openfhe as bs
    from easyfhe.bs import placement as pl

    client, ctx = boot_ctx
    n = ctx.max_slots
    prog = bs.generate(ctx, bs.BootstrapSpec(log_slots=ctx.logN - 1, level_budget=(3, 3),
                                             output_levels=3))
    rng = np.random.default_rng(12)
    zs = [rng.uniform(-1, 1, n) for _ in range(4)]
    cts = [client.encrypt(z, cur_limbs=1, enc_id=110 + i) for i, z in enumerate(zs)]
    sched = pl.RefreshSchedule(residual_bootstrap_level_drop=3)
    res = pl.refresh_and_drop(cts, ctx, prog, schedule=sched, rmsnorm_depth=1,
                              minimum_output_limbs=2)
    top = prog.output_limbs
    want_drop = pl.adaptive_bootstrap_output_level_drop(
        current_limbs=top, requested_level_drop=3, rmsnorm_depth=1, minimum_output_limbs=2)
    assert want_drop == min(3, top - 3) and res.level_drops == [want_drop] * 4
    assert res.output_limbs == (top - want_drop,)
    for got, z in zip(res.ciphers, zs):
        err = np.abs(client.decrypt(got) - z).max()
        assert -math.log2(err) > 14, err
    # the reference's explicit halving spends one more limb, same values
    halved = pl.refresh_ciphers(cts[:2], ctx, prog, halve=True)
    for got, z in zip(halved, zs[:2]):
        assert int(got.state.cur_limbs) == top - 1
        assert -math.log2(np.abs(client.decrypt(got) - z).max()) > 14
