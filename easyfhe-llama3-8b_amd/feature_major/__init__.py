"""Feature-major operators over the easyfhe backend: the layouts and the BSGS
linear engine that drive ``fhe.hoisted_mac_sum`` (counterparts of the
reference's llama3fhe/layouts and llama3fhe/operators/linear)."""

from .layout import FeatureMajorPrefillLayout, LinearCarrierLayout
from .linear import (
    LinearChunk,
    LinearOperator,
    LinearOperatorConfig,
    LinearPlan,
    LinearWeight,
    linear_rotations,
)

__all__ = [
    "FeatureMajorPrefillLayout", "LinearCarrierLayout", "LinearChunk", "LinearOperator",
    "LinearOperatorConfig", "LinearPlan", "LinearWeight", "linear_rotations",
]
