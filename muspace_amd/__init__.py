"""MI355X-native multi-scale deformable attention with muSPACE's public API.

The exports mirror the MSDA part of the reference package
(/root/reference/mu_space/__init__.py:36,54-59): the canonical operator, its
dispatch explanation and the dispatch-report accessors. ``import muspace_amd
as mu_space`` gives code written against the reference the same names.
"""

from .ops import (
    explain_dispatch,
    multi_scale_deformable_attn,
    multi_scale_deformable_attn_pytorch,
    multi_scale_deformable_attn_pytorch_compat,
    multi_scale_deformable_attn_scatter_div,
    multi_scale_deformable_attn_softmax,
)
from .runtime.kernel_dispatch import (
    DispatchDecision,
    DispatchReport,
    clear_dispatch_report,
    get_dispatch_reports,
    get_last_dispatch_report,
)

__version__ = "0.1.0"

__all__ = [
    "DispatchDecision",
    "DispatchReport",
    "__version__",
    "clear_dispatch_report",
    "explain_dispatch",
    "get_dispatch_reports",
    "get_last_dispatch_report",
    "multi_scale_deformable_attn",
    "multi_scale_deformable_attn_pytorch",
    "multi_scale_deformable_attn_pytorch_compat",
    "multi_scale_deformable_attn_scatter_div",
    "multi_scale_deformable_attn_softmax",
]
