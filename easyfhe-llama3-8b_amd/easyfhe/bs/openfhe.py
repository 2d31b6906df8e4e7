"""CKKS bootstrapping surface (reference operators/nonlinear/bootstrap.py:59-189).

The bootstrap program (ModRaise, CoeffToSlot, EvalMod, SlotToCoeff) is not
built in this backend yet; every entry point raises ``NotImplementedError``
so that a caller never receives a silently wrong refresh.
"""

from __future__ import annotations

from dataclasses import dataclass


@dataclass(frozen=True)
class BootstrapSpec:
    log_slots: int
    level_budget: tuple = (4, 4)
    output_levels: int = 0
    mode: str = "modraise_first"


def _missing(*_args, **_kwargs):
    raise NotImplementedError("bootstrapping is not implemented in this backend yet")


requirements = _missing
generate = _missing
bootstrap = _missing

__all__ = ["BootstrapSpec", "bootstrap", "generate", "requirements"]
