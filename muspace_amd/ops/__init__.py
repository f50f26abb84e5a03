"""Canonical operator exports (the MSDA path of /root/reference/mu_space/ops/__init__.py:24-28)."""

from .multi_scale_deformable_attn import (
    explain_dispatch,
    level_start_index_from_shapes,
    multi_scale_deformable_attn,
    multi_scale_deformable_attn_pytorch,
    multi_scale_deformable_attn_pytorch_compat,
)
from .scatter_div import multi_scale_deformable_attn_scatter_div
from .msda_softmax import attention_softmax, multi_scale_deformable_attn_softmax
from .deformable_aggregation import (
    deformable_aggregation,
    deformable_aggregation_function,
    deformable_aggregation_reference,
    feature_maps_format,
)

__all__ = [
    "attention_softmax",
    "deformable_aggregation",
    "deformable_aggregation_function",
    "deformable_aggregation_reference",
    "feature_maps_format",
    "explain_dispatch",
    "level_start_index_from_shapes",
    "multi_scale_deformable_attn",
    "multi_scale_deformable_attn_pytorch",
    "multi_scale_deformable_attn_pytorch_compat",
    "multi_scale_deformable_attn_scatter_div",
    "multi_scale_deformable_attn_softmax",
]
