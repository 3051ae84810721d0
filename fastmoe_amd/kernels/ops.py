"""Import path of the reference (``fastmoe.kernels.ops``): the same names as ``fastmoe_amd.ops``."""
from ..ops import (  # noqa: F401
    GroupedMetadata,
    GroupedWeightedScatterAdd,
    _launch_grouped_kernel,
    build_plan,
    grouped_weighted_scatter_add,
    prepare_grouped_metadata,
    weighted_scatter_add,
)
