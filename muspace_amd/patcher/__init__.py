"""Runtime patchers (the MSDA part of /root/reference/mu_space/patcher)."""

from .runtime import (
    DefaultPatcher,
    PatchError,
    PatchReport,
    QwenDrivePatcher,
    default_patcher,
    qwendrive_patcher,
)

__all__ = [
    "DefaultPatcher",
    "PatchError",
    "PatchReport",
    "QwenDrivePatcher",
    "default_patcher",
    "qwendrive_patcher",
]
