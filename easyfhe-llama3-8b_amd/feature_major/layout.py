"""Feature-major slot layouts (reference llama3fhe/layouts/feature_major.py:10-110,
layouts/linear.py:15-116).

A ciphertext carries ``lanes = slots / dimension`` tokens; feature ``d`` of
local token ``t`` sits at slot ``d * lanes + t``, so a rotation by
``k * lanes`` moves every token's feature ``d + k`` onto ``d`` at once.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np


def _power_of_two(value: int, name: str) -> int:
    value = int(value)
    if value <= 0 or value & (value - 1):
        raise ValueError(f"{name} must be a positive power of two, got {value}.")
    return value


@dataclass(frozen=True)
class _TokenLaneLayout:
    seq_len: int
    dimension: int
    slots: int = 32768

    def __post_init__(self) -> None:
        _power_of_two(self.dimension, "dimension")
        if int(self.seq_len) <= 0:
            raise ValueError(f"seq_len must be positive, got {self.seq_len}.")
        if int(self.slots) % int(self.dimension):
            raise ValueError(f"slots={self.slots} must be divisible by dimension={self.dimension}.")

    @property
    def token_lanes(self) -> int:
        return int(self.slots) // int(self.dimension)

    @property
    def cipher_count(self) -> int:
        return -(-int(self.seq_len) // self.token_lanes)

    def active_tokens(self, cipher_index: int) -> int:
        i = int(cipher_index)
        if not 0 <= i < self.cipher_count:
            raise IndexError(f"cipher_index={i} is outside [0, {self.cipher_count}).")
        return max(0, min(self.token_lanes, int(self.seq_len) - i * self.token_lanes))

    def slot(self, dim: int, token: int) -> int:
        dim, token = int(dim), int(token)
        if not 0 <= dim < int(self.dimension):
            raise IndexError(f"dim={dim} is outside [0, {self.dimension}).")
        if not 0 <= token < self.token_lanes:
            raise IndexError(f"token={token} is outside [0, {self.token_lanes}).")
        return dim * self.token_lanes + token

    def pack(self, rows: np.ndarray, *, dtype=np.float64) -> np.ndarray:
        """[seq_len, dimension] -> [cipher_count, slots] (zero padded tokens)."""
        rows = np.asarray(rows, dtype=dtype)
        want = (int(self.seq_len), int(self.dimension))
        if rows.shape != want:
            raise ValueError(f"rows must have shape {want}, got {rows.shape}.")
        lanes, n = self.token_lanes, self.cipher_count
        out = np.zeros((n * lanes, int(self.dimension)), dtype=dtype)
        out[: int(self.seq_len)] = rows
        # token t of cipher c, feature d -> cipher c, slot d * lanes + t
        return out.reshape(n, lanes, int(self.dimension)).swapaxes(1, 2).reshape(n, int(self.slots))

    def unpack(self, packed: np.ndarray, *, output_dim: int | None = None) -> np.ndarray:
        packed = np.asarray(packed)
        want = (self.cipher_count, int(self.slots))
        if packed.shape != want:
            raise ValueError(f"payload must have shape {want}, got {packed.shape}.")
        d = int(self.dimension if output_dim is None else output_dim)
        if not 0 < d <= int(self.dimension):
            raise ValueError(f"output_dim must be in [1, {self.dimension}], got {d}.")
        rows = packed.reshape(self.cipher_count, int(self.dimension), self.token_lanes)
        rows = rows.swapaxes(1, 2).reshape(-1, int(self.dimension))
        return np.asarray(rows[: int(self.seq_len), :d], dtype=np.float32)


class FeatureMajorPrefillLayout(_TokenLaneLayout):
    """The persistent layout of the model's hidden states: hidden_dim features
    per token (production S = 128, D = 4096, slots = 32768: 8 tokens per
    ciphertext, 16 ciphertexts)."""

    def __init__(self, seq_len: int = 128, hidden_dim: int = 4096, slots: int = 32768):
        super().__init__(seq_len=seq_len, dimension=hidden_dim, slots=slots)

    @property
    def hidden_dim(self) -> int:
        return int(self.dimension)

    @property
    def tokens_per_cipher(self) -> int:
        return self.token_lanes


class LinearCarrierLayout(_TokenLaneLayout):
    """The private carrier of a linear's output: ``dimension`` is the
    power-of-two physical row width; an operator may use a prefix of it."""
