"""Bootstrapping namespace (reference ``easyfhe.bs``)."""

from . import openfhe

__all__ = ["openfhe"]
