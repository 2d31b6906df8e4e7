"""Level-free real/imaginary multiplexing of feature-major streams (reference
llama3fhe/operators/linear/complex.py:1-87).

Two real streams share one ciphertext as ``x + i y``: a linear layer with
real weights acts on both at once, and one bootstrap refreshes both.  The
split uses one conjugation (rotation index M - 1) and returns twice each
component, ``2 Re z`` and ``2 Im z``; callers either fold the factor into a
later constant or, on this backend, into the recorded scale (``halve=True``
below), which costs no level.
"""

from __future__ import annotations

from easyfhe import fhe


def _ctx(context):
    return getattr(context, "context", context)


def _release(values) -> None:
    for v in values or ():
        if v is not None:
            v.release()


def pair_real_ciphers(ciphers, *, crypto_context) -> tuple:
    """``x[2r] + i x[2r+1]`` for adjacent real streams (complex.py:10-37)."""
    ctx = _ctx(crypto_context)
    cts = tuple(ciphers)
    if len(cts) % 2:
        raise ValueError("complex pairing requires an even ciphertext count.")
    out = []
    for i in range(0, len(cts), 2):
        imag = fhe.homo_mul_i(cts[i + 1], ctx)
        try:
            out.append(fhe.homo_add(cts[i], imag, ctx))
        finally:
            imag.release()
    return tuple(out)


def split_complex_cipher_twice(cipher, *, crypto_context, halve: bool = False) -> tuple:
    """``(2 Re z, 2 Im z)`` without a level (complex.py:40-67).  With
    ``halve`` the factor 2 is taken into the recorded scale, so the outputs
    decrypt to ``Re z`` and ``Im z`` exactly (the words are the same)."""
    ctx = _ctx(crypto_context)
    conj = fhe.homo_rotate(cipher, 2 * ctx.N - 1, ctx)
    delta = None
    try:
        real = fhe.homo_add(cipher, conj, ctx)
        delta = fhe.homo_sub(conj, cipher, ctx)
        imag = fhe.homo_mul_i(delta, ctx)
    finally:
        conj.release()
        if delta is not None:
            delta.release()
    if halve:
        for t in (real, imag):
            t.set_scale(2.0 * float(t.state.scaling_factor), 1)
    return real, imag


def split_complex_ciphers_twice(ciphers, *, crypto_context, halve: bool = False) -> tuple:
    """Interleaved ``2 Re, 2 Im`` of every input (complex.py:70-87); the
    conjugations of all inputs run as one batched key switch."""
    ctx = _ctx(crypto_context)
    cts = list(ciphers)
    if not cts:
        return ()
    conjs = fhe.homo_rotate_many(cts, 2 * ctx.N - 1, ctx)
    out = []
    try:
        for z, c in zip(cts, conjs):
            real = fhe.homo_add(z, c, ctx)
            delta = fhe.homo_sub(c, z, ctx)
            imag = fhe.homo_mul_i(delta, ctx)
            delta.release()
            if halve:
                for t in (real, imag):
                    t.set_scale(2.0 * float(t.state.scaling_factor), 1)
            out.extend((real, imag))
    finally:
        _release(conjs)
    return tuple(out)


__all__ = ["pair_real_ciphers", "split_complex_cipher_twice", "split_complex_ciphers_twice"]
