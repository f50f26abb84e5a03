"""Backend selection and dispatch reports for the MSDA operator.

Mirrors /root/reference/mu_space/runtime/kernel_dispatch.py:13-103 with the
device test changed from MUSA to ROCm: the native backend is ``"hip"`` and runs
on tensors of torch's ``cuda`` device type under a HIP build of torch.
``"musa"`` is still accepted as a requested backend and means the same as
``"hip"``, so callers written against the reference keep working.

Differences from the reference, both deliberate:
  * the report history is bounded (``MAX_REPORTS`` most recent reports) where
    the reference appends to an unbounded list (kernel_dispatch.py:43,49);
  * ``auto`` on a ROCm tensor without the native library is an error by
    default rather than a silent switch to the PyTorch path: the HIP kernels
    are the product on that device, so a missing library must be visible.
    ``MUSPACE_AUTO_FALLBACK=1`` restores the reference's behaviour
    (kernel_dispatch.py:94-100): ``auto`` then selects the PyTorch path with
    the unavailability as the recorded reason, for callers such as patched
    mmcv models that prefer degrading to failing.
"""

from __future__ import annotations

import json
import os
import sys
from collections import deque
from dataclasses import asdict, dataclass
from typing import Literal

import torch

BackendName = Literal["auto", "hip", "musa", "reference"]
SelectedBackend = Literal["hip", "reference", "error"]

NATIVE_BACKEND = "hip"
NATIVE_ALIASES = frozenset({"hip", "musa"})
MAX_REPORTS = 4096
LOG_ENV = "MUSPACE_DISPATCH_LOG"
AUTO_FALLBACK_ENV = "MUSPACE_AUTO_FALLBACK"


@dataclass(frozen=True)
class DispatchDecision:
    backend: SelectedBackend
    device: str
    reason: str

    def as_dict(self) -> dict[str, object]:
        return asdict(self)


@dataclass(frozen=True)
class DispatchReport:
    operator: str
    requested_backend: str
    selected_backend: SelectedBackend
    device: str
    reason: str
    native_available: bool
    native_fallback: bool = False
    fallback_reason: str | None = None

    def as_dict(self) -> dict[str, object]:
        return asdict(self)


_last_dispatch_report: DispatchReport | None = None
_dispatch_reports: deque[DispatchReport] = deque(maxlen=MAX_REPORTS)


def _env_flag(name: str) -> bool:
    return os.environ.get(name, "").strip().lower() in {"1", "true", "yes", "on"}


def _log_enabled() -> bool:
    return _env_flag(LOG_ENV)


def record_dispatch_report(report: DispatchReport) -> DispatchReport:
    global _last_dispatch_report
    _last_dispatch_report = report
    _dispatch_reports.append(report)
    if _log_enabled():
        print("muSPACE dispatch: " + json.dumps(report.as_dict(), sort_keys=True), file=sys.stderr)
    return report


def get_last_dispatch_report() -> DispatchReport | None:
    return _last_dispatch_report


def get_dispatch_reports() -> tuple[DispatchReport, ...]:
    return tuple(_dispatch_reports)


def clear_dispatch_report() -> None:
    global _last_dispatch_report
    _last_dispatch_report = None
    _dispatch_reports.clear()


def is_rocm_tensor(tensor) -> bool:
    """True for a tensor on an AMD GPU under a HIP build of torch."""
    device = getattr(tensor, "device", None)
    return getattr(device, "type", None) == "cuda" and torch.version.hip is not None


def explain_dispatch(
    value: torch.Tensor,
    *,
    backend: str = "auto",
    native_available: bool = True,
) -> DispatchDecision:
    if backend not in {"auto", "reference"} | NATIVE_ALIASES:
        return DispatchDecision("error", value.device.type, f"unknown backend: {backend}")
    device = value.device.type
    if backend == "reference":
        return DispatchDecision("reference", device, "reference backend requested")

    unavailable = "muSPACE HIP native library is unavailable"
    if backend in NATIVE_ALIASES:
        if not is_rocm_tensor(value):
            return DispatchDecision("error", device, f"backend={backend} requires a ROCm tensor")
        if not native_available:
            return DispatchDecision("error", device, unavailable)
        return DispatchDecision(NATIVE_BACKEND, device, "forced HIP backend")

    if is_rocm_tensor(value):
        if not native_available:
            if _env_flag(AUTO_FALLBACK_ENV):
                return DispatchDecision(
                    "reference", device,
                    "HIP backend is unavailable; falling back to PyTorch reference")
            return DispatchDecision("error", device, unavailable)
        return DispatchDecision(NATIVE_BACKEND, device, "ROCm tensor selects native HIP backend")

    return DispatchDecision("reference", device, "non-ROCm tensors use the PyTorch reference")
