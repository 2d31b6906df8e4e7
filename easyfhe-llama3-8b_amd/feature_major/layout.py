"""Token-lane slot maps of the feature-major stream (interface of reference
llama3fhe/layouts/feature_major.py and layouts/linear.py).

One ciphertext holds ``lanes = slots // width`` consecutive tokens.  Token ``k``
of the sequence lives in ciphertext ``k // lanes`` on lane ``k % lanes``, and
its feature ``d`` occupies slot ``d * lanes + k % lanes``.  Rotating a
ciphertext by ``j * lanes`` therefore moves feature ``d + j`` of every token
onto feature ``d`` at once, which is what the diagonal method needs.

``pack`` and ``unpack`` are the scatter and gather of that map, computed from
index arrays; tokens past ``seq_len`` in the last ciphertext are zero.
"""

from __future__ import annotations

import numpy as np


def _require(ok: bool, what: str) -> None:
    if not ok:
        raise ValueError(f"feature-major layout: {what}")


class _TokenLanes:
    """The slot map for ``seq_len`` tokens of ``width`` features each."""

    __slots__ = ("_seq", "_width", "_slots", "_lanes")

    def __init__(self, seq_len: int, width: int, slots: int):
        seq, width, slots = int(seq_len), int(width), int(slots)
        _require(width >= 1 and (width & (width - 1)) == 0,
                 f"the feature width {width} is not a power of two")
        _require(seq >= 1, f"a sequence needs at least one token (seq_len={seq})")
        _require(slots >= width and slots % width == 0,
                 f"{slots} slots do not hold a whole number of {width}-feature rows")
        self._seq, self._width, self._slots = seq, width, slots
        self._lanes = slots // width

    # -- geometry -------------------------------------------------------------
    @property
    def seq_len(self) -> int:
        return self._seq

    @property
    def slots(self) -> int:
        return self._slots

    @property
    def token_lanes(self) -> int:
        return self._lanes

    @property
    def cipher_count(self) -> int:
        return (self._seq + self._lanes - 1) // self._lanes

    def active_tokens(self, cipher_index: int) -> int:
        """Tokens of the sequence carried by ciphertext ``cipher_index``."""
        c = int(cipher_index)
        if c < 0 or c >= self.cipher_count:
            raise IndexError(f"ciphertext {c} does not exist (the layout has "
                             f"{self.cipher_count})")
        first = c * self._lanes
        return min(self._lanes, self._seq - first)

    def slot(self, dim: int, token: int) -> int:
        """Slot of feature ``dim`` for lane ``token`` of any ciphertext."""
        d, t = int(dim), int(token)
        if d < 0 or d >= self._width:
            raise IndexError(f"feature {d} is not below the width {self._width}")
        if t < 0 or t >= self._lanes:
            raise IndexError(f"lane {t} is not below the lane count {self._lanes}")
        return d * self._lanes + t

    # -- scatter / gather -----------------------------------------------------
    def _index(self):
        """(ciphertext of each token [seq, 1], slot of each (token, feature))."""
        cipher, lane = np.divmod(np.arange(self._seq), self._lanes)
        cols = np.arange(self._width)[None, :] * self._lanes + lane[:, None]
        return cipher[:, None], cols

    def pack(self, rows: np.ndarray, *, dtype=np.float64) -> np.ndarray:
        """``[seq_len, width]`` token rows -> ``[cipher_count, slots]`` payloads."""
        rows = np.asarray(rows, dtype=dtype)
        _require(rows.shape == (self._seq, self._width),
                 f"expected token rows of shape {(self._seq, self._width)}, got {rows.shape}")
        out = np.zeros((self.cipher_count, self._slots), dtype=dtype)
        cipher, cols = self._index()
        out[cipher, cols] = rows
        return out

    def unpack(self, packed: np.ndarray, *, output_dim: int | None = None) -> np.ndarray:
        """``[cipher_count, slots]`` payloads -> the first ``output_dim`` features of
        every token as float32 (the reference's client-side dtype)."""
        packed = np.asarray(packed)
        _require(packed.shape == (self.cipher_count, self._slots),
                 f"expected payloads of shape {(self.cipher_count, self._slots)}, "
                 f"got {packed.shape}")
        keep = self._width if output_dim is None else int(output_dim)
        _require(1 <= keep <= self._width,
                 f"cannot keep {keep} features of a {self._width}-feature row")
        cipher, cols = self._index()
        return packed[cipher, cols[:, :keep]].astype(np.float32)

    # -- value semantics (layouts are compared and used as cache keys) ----------
    def _key(self):
        return (type(self), self._seq, self._width, self._slots)

    def __eq__(self, other) -> bool:
        return isinstance(other, _TokenLanes) and self._key() == other._key()

    def __hash__(self) -> int:
        return hash(self._key())

    def __repr__(self) -> str:
        return (f"{type(self).__name__}(seq_len={self._seq}, width={self._width}, "
                f"slots={self._slots})")


class FeatureMajorPrefillLayout(_TokenLanes):
    """The hidden-state layout between layers: ``hidden_dim`` features per token
    (at S = 128, D = 4096 and 2^15 slots: 8 tokens in each of 16 ciphertexts)."""

    __slots__ = ()

    def __init__(self, seq_len: int = 128, hidden_dim: int = 4096, slots: int = 32768):
        super().__init__(seq_len, hidden_dim, slots)

    @property
    def hidden_dim(self) -> int:
        return self._width

    @property
    def tokens_per_cipher(self) -> int:
        return self._lanes


class LinearCarrierLayout(_TokenLanes):
    """A linear's output carrier: ``dimension`` is the power-of-two row width
    of the physical matrix; an operator may use only a prefix of it."""

    __slots__ = ()

    def __init__(self, seq_len: int, dimension: int, slots: int = 32768):
        super().__init__(seq_len, dimension, slots)

    @property
    def dimension(self) -> int:
        return self._width


__all__ = ["FeatureMajorPrefillLayout", "LinearCarrierLayout"]
