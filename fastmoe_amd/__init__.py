"""fastmoe_amd: fastmoe's grouped pointer-indirection MoE combine on MI355X (gfx950).

The operator API mirrors ``fastmoe.kernels.ops``; the work runs in hand-written HIP kernels of
``libfastmoe_amd.so`` through its C ABI (``include/fastmoe_amd.h``).
"""
from .consts import MoEImplementation
from .ops import (
    GroupedMetadata,
    GroupedWeightedScatterAdd,
    build_plan,
    grouped_weighted_scatter_add,
    prepare_grouped_metadata,
    weighted_scatter_add,
)

__all__ = [
    "GroupedMetadata",
    "GroupedWeightedScatterAdd",
    "MoEImplementation",
    "build_plan",
    "grouped_weighted_scatter_add",
    "prepare_grouped_metadata",
    "weighted_scatter_add",
]
