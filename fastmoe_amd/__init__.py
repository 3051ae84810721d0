"""fastmoe_amd: fastmoe's grouped pointer-indirection MoE combine on MI355X (gfx950).

The operator API mirrors ``fastmoe.kernels.ops``; the work runs in hand-written HIP kernels of
``libfastmoe_amd.so`` through its C ABI (``include/fastmoe_amd.h``).
"""
from .consts import MoEImplementation
from .dispatch import PermutedTokens, permute_tokens
from .moe import MoEFeedForward, compute_experts, gate_and_sort, unpermute
from .ops import (
    GroupedMetadata,
    GroupedWeightedScatterAdd,
    build_plan,
    grouped_weighted_scatter_add,
    invert_scatter_index,
    prepare_grouped_metadata,
    prepare_metadata_and_plan,
    weighted_scatter_add,
)

__all__ = [
    "GroupedMetadata",
    "GroupedWeightedScatterAdd",
    "MoEFeedForward",
    "MoEImplementation",
    "PermutedTokens",
    "compute_experts",
    "gate_and_sort",
    "permute_tokens",
    "unpermute",
    "build_plan",
    "grouped_weighted_scatter_add",
    "invert_scatter_index",
    "prepare_grouped_metadata",
    "prepare_metadata_and_plan",
    "weighted_scatter_add",
]
