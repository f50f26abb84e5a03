"""Runtime patchers (the MSDA and deformable-aggregation parts of /root/reference/mu_space/patcher)."""

from .runtime import (
    DefaultPatcher,
    PatchError,
    PatchReport,
    QwenDrivePatcher,
    SparseDrivePatcher,
    default_patcher,
    qwendrive_patcher,
    sparsedrive_patcher,
)

__all__ = [
    "DefaultPatcher",
    "PatchError",
    "PatchReport",
    "QwenDrivePatcher",
    "SparseDrivePatcher",
    "default_patcher",
    "qwendrive_patcher",
    "sparsedrive_patcher",
]
