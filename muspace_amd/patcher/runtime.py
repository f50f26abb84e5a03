"""Runtime patches that route model code's MSDA calls to this operator.

The MSDA part of /root/reference/mu_space/patcher/runtime.py:
  * ``DefaultPatcher`` (reference :577-636) rebinds mmcv's 4-argument helper
    ``mmcv.ops.multi_scale_deform_attn.multi_scale_deformable_attn_pytorch``
    plus the copies already bound in imported BEVFormer / UniAD modules, and
    guards ``mmcv.utils.ext_loader.load_ext`` so models import without mmcv's
    compiled extension (:97-159); ``restore()`` undoes all of it;
  * the strict / compat wrappers (:398-439): strict forces the native backend,
    compat uses ``auto``; ``MUSPACE_STRICT_PATCH`` selects strict (:272-273);
  * the Qwen-Drive bf16 MSDA entry (:285-337) and a ``QwenDrivePatcher`` that
    installs it. The reference's Qwen-Drive patcher also replaces a voxel-pool
    operator and a frustum property, which are other operators and are not
    part of this package; only the two MSDA symbols are patched here.
The module paths below are the upstream models' own (interface data).
"""

from __future__ import annotations

import importlib
import os
import sys
from collections.abc import Callable
from dataclasses import asdict, dataclass
from types import ModuleType

PatchCallable = Callable[..., object]

STRICT_ENV = "MUSPACE_STRICT_PATCH"
MSDA_TARGET_MODULE = "mmcv.ops.multi_scale_deform_attn"
MSDA_TARGET_ATTR = "multi_scale_deformable_attn_pytorch"
EXT_LOADER_MODULE = "mmcv.utils.ext_loader"
BEVFORMER_IMPORTED_MODULES = (
    "projects.mmdet3d_plugin.bevformer.modules.decoder",
    "projects.mmdet3d_plugin.bevformer.modules.encoder",
    "projects.mmdet3d_plugin.bevformer.modules.spatial_cross_attention",
    "projects.mmdet3d_plugin.bevformer.modules.temporal_self_attention",
)
UNIAD_IMPORTED_MODULES = (
    "projects.mmdet3d_plugin.uniad.modules.decoder",
    "projects.mmdet3d_plugin.uniad.modules.spatial_cross_attention",
    "projects.mmdet3d_plugin.uniad.modules.temporal_self_attention",
    "projects.mmdet3d_plugin.uniad.dense_heads.motion_head_plugin.motion_deformable_attn",
)
QWENDRIVE_ATTENTION_MODULE = "qwen_drive_perception.attention"
QWENDRIVE_MSDA_ATTR = "multi_scale_deformable_attn_cuda"
QWENDRIVE_OPS_MODULE = "qwen_drive_perception.ops"
QWENDRIVE_MSDA_FORWARD_ATTR = "ms_deform_attn_bf16_forward"
# SparseDrive's deformable aggregation entry (reference runtime.py:61-66)
SPARSEDRIVE_OPS_MODULE = "projects.mmdet3d_plugin.ops"
SPARSEDRIVE_DAF_ATTR = "deformable_aggregation_function"
SPARSEDRIVE_IMPORTED_MODULES = ("projects.mmdet3d_plugin.models.blocks",)
SPARSEDRIVE_IMPORTED_ATTR = "DAF"
SPARSEDRIVE_PACKAGE = "projects"
SPARSEDRIVE_DAF_VALID_ATTR = "DAF_VALID"

_SAVED_LOAD_EXT = "_muspace_original_load_ext"


class PatchError(RuntimeError):
    """Raised when a runtime patch cannot be installed safely."""


@dataclass(frozen=True)
class PatchReport:
    target: str
    strict: bool
    action: str
    patched_modules: tuple[str, ...]

    def as_dict(self) -> dict[str, object]:
        return asdict(self)


def _env_strict() -> bool:
    return os.environ.get(STRICT_ENV, "").strip().lower() in {"1", "true", "yes", "on"}


# ------------------------------------------------ mmcv extension guard ---


class _MissingLegacyExtension:
    """Stands in for an mmcv compiled extension that failed to load.

    Attribute probes succeed (so ``hasattr`` checks at import time pass); a
    call raises ``PatchError`` naming the extension and the function.
    """

    def __init__(self, name: str, functions: object) -> None:
        self.name = name
        self.functions = functions

    def __getattr__(self, attr: str) -> object:
        if attr.startswith("__") and attr.endswith("__"):
            raise AttributeError(attr)
        if attr in {"get_compiler_version", "get_compiling_cuda_version"}:
            return lambda: "unavailable"
        ext = self.name

        def unavailable(*args: object, **kwargs: object) -> object:
            raise PatchError(
                f"Legacy extension mmcv.{ext} is unavailable; the muSPACE replacement must "
                f"handle this path before {attr} is called"
            )

        unavailable.__name__ = attr
        return unavailable


def _guard_legacy_mmcv_extensions() -> bool:
    """Make mmcv's ``load_ext`` return a placeholder instead of raising.

    Returns True when this call installed the guard (the caller then owns it).
    """
    try:
        loader = importlib.import_module(EXT_LOADER_MODULE)
    except ImportError:
        return False
    if hasattr(loader, _SAVED_LOAD_EXT):
        return False
    original = loader.load_ext

    def guarded_load_ext(name: str, functions: object):
        try:
            return original(name, functions)
        except (ImportError, OSError):
            return _MissingLegacyExtension(name, functions)

    setattr(loader, _SAVED_LOAD_EXT, original)
    loader.load_ext = guarded_load_ext
    return True


def _release_legacy_mmcv_extensions() -> bool:
    loader = sys.modules.get(EXT_LOADER_MODULE)
    if loader is None:
        return False
    original = getattr(loader, _SAVED_LOAD_EXT, None)
    if original is None:
        return False
    loader.load_ext = original
    delattr(loader, _SAVED_LOAD_EXT)
    return True


# ------------------------------------------------------- attr rebinding ---


def _patch_attr(
    originals: dict[tuple[str, str], object], module: ModuleType, attr: str, replacement: object
) -> bool:
    """Set ``module.attr`` if it exists, remembering the first original."""
    if not hasattr(module, attr):
        return False
    originals.setdefault((module.__name__, attr), getattr(module, attr))
    setattr(module, attr, replacement)
    return True


def _restore_attrs(originals: dict[tuple[str, str], object]) -> list[str]:
    """Put every recorded original back and forget it."""
    restored = []
    for (module_name, attr), original in list(originals.items()):
        module = sys.modules.get(module_name)
        if module is not None:
            setattr(module, attr, original)
            restored.append(module_name)
        del originals[(module_name, attr)]
    return restored


# ------------------------------------------------------------- wrappers ---


def _level_start_index(value_spatial_shapes):
    from ..ops.multi_scale_deformable_attn import level_start_index_from_shapes

    return level_start_index_from_shapes(value_spatial_shapes)


def _make_msda_wrapper(strict: bool) -> PatchCallable:
    """mmcv-signature replacement: strict forces the HIP backend, compat uses auto."""
    if strict:

        def strict_msda(value, value_spatial_shapes, sampling_locations, attention_weights):
            from ..ops import multi_scale_deformable_attn

            return multi_scale_deformable_attn(
                value,
                value_spatial_shapes,
                _level_start_index(value_spatial_shapes),
                sampling_locations,
                attention_weights,
                backend="hip",
            )

        strict_msda.__name__ = "muspace_multi_scale_deformable_attn_strict"
        strict_msda.__module__ = __name__
        return strict_msda

    def compat_msda(value, value_spatial_shapes, sampling_locations, attention_weights):
        from ..ops import multi_scale_deformable_attn_pytorch_compat

        return multi_scale_deformable_attn_pytorch_compat(
            value, value_spatial_shapes, sampling_locations, attention_weights
        )

    compat_msda.__name__ = "muspace_multi_scale_deformable_attn_compat"
    compat_msda.__module__ = __name__
    return compat_msda


def _accelerated_tensor(value) -> bool:
    """True for a tensor on a GPU: ``cuda`` (ROCm) or the reference's MUSA spellings."""
    device_type = getattr(getattr(value, "device", None), "type", None)
    return device_type in {"cuda", "musa", "privateuseone"} or bool(
        getattr(value, "is_cuda", False) or getattr(value, "is_musa", False)
    )


def _make_qwendrive_msda_wrapper(strict: bool, original: PatchCallable) -> PatchCallable:
    """Qwen-Drive's 6-argument bf16 MSDA entry (reference runtime.py:285-337).

    bfloat16 GPU tensors go through the autograd operator with the caller's
    ``im2col_step``; another dtype on a GPU is a ``TypeError``; tensors on
    other devices keep the original (PyTorch) implementation.
    """
    backend = "hip" if strict else "auto"

    def muspace_qwendrive_msda(
        value,
        value_spatial_shapes,
        value_level_start_index,
        sampling_locations,
        attention_weights,
        im2col_step,
    ):
        if not _accelerated_tensor(value):
            return original(
                value,
                value_spatial_shapes,
                value_level_start_index,
                sampling_locations,
                attention_weights,
                im2col_step,
            )
        import torch

        if value.dtype != torch.bfloat16:
            raise TypeError(
                "the ms_deform_attn kernel requires bfloat16 tensors on the GPU, "
                f"got {value.dtype}; run the model in bfloat16"
            )
        from .. import ops

        return ops.multi_scale_deformable_attn(
            value,
            value_spatial_shapes,
            value_level_start_index,
            sampling_locations,
            attention_weights,
            im2col_step=int(im2col_step),
            backend=backend,
        )

    muspace_qwendrive_msda.__name__ = (
        "muspace_qwendrive_msda_strict" if strict else "muspace_qwendrive_msda"
    )
    muspace_qwendrive_msda.__module__ = __name__
    return muspace_qwendrive_msda


# ------------------------------------------------------------- patchers ---


class DefaultPatcher:
    """Swap mmcv's MSDA helper for this operator without editing model code."""

    def __init__(self) -> None:
        self._originals: dict[tuple[str, str], object] = {}
        self._strict: bool | None = None
        self._guarded = False

    def apply(self, *, strict: bool | None = None) -> PatchReport:
        strict = _env_strict() if strict is None else strict
        patched = self._patch_mmcv_msda(_make_msda_wrapper(strict))
        action = "already-applied" if self._strict == strict else "applied"
        self._strict = strict
        return PatchReport(
            target=f"{MSDA_TARGET_MODULE}.{MSDA_TARGET_ATTR}",
            strict=strict,
            action=action,
            patched_modules=tuple(patched),
        )

    def restore(self) -> PatchReport:
        restored = _restore_attrs(self._originals)
        if self._guarded:
            _release_legacy_mmcv_extensions()
            self._guarded = False
        self._strict = None
        return PatchReport(
            target=f"{MSDA_TARGET_MODULE}.{MSDA_TARGET_ATTR}",
            strict=False,
            action="restored",
            patched_modules=tuple(restored),
        )

    def _patch_mmcv_msda(self, replacement: PatchCallable) -> list[str]:
        self._guarded = _guard_legacy_mmcv_extensions() or self._guarded
        try:
            target = importlib.import_module(MSDA_TARGET_MODULE)
        except ImportError as exc:
            raise PatchError(
                "mmcv MSDeformAttn helper is unavailable; install the BEVFormer "
                "OpenMMLab stack before calling default_patcher.apply()"
            ) from exc
        if not _patch_attr(self._originals, target, MSDA_TARGET_ATTR, replacement):
            raise PatchError(f"{MSDA_TARGET_MODULE}.{MSDA_TARGET_ATTR} is unavailable")
        patched = [target.__name__]
        # model modules bind the helper at import time: rebind those copies too
        for name in (*BEVFORMER_IMPORTED_MODULES, *UNIAD_IMPORTED_MODULES):
            module = sys.modules.get(name)
            if module is not None and _patch_attr(
                self._originals, module, MSDA_TARGET_ATTR, replacement
            ):
                patched.append(name)
        return patched


class QwenDrivePatcher:
    """Route Qwen-Drive's MSDA entry points to this operator (MSDA symbols only)."""

    def __init__(self) -> None:
        self._originals: dict[tuple[str, str], object] = {}
        self._strict: bool | None = None

    def apply(self, *, strict: bool | None = None) -> PatchReport:
        strict = _env_strict() if strict is None else strict
        try:
            attention = importlib.import_module(QWENDRIVE_ATTENTION_MODULE)
            ops = importlib.import_module(QWENDRIVE_OPS_MODULE)
        except ImportError as exc:
            raise PatchError(
                "qwen_drive_perception import failed. Add the Qwen-Drive checkout src "
                "directory to PYTHONPATH before qwendrive_patcher.apply()."
            ) from exc
        missing = [
            f"{module.__name__}.{attr}"
            for module, attr in ((attention, QWENDRIVE_MSDA_ATTR), (ops, QWENDRIVE_MSDA_FORWARD_ATTR))
            if not callable(getattr(module, attr, None))
        ]
        if missing:
            raise PatchError(
                "qwen_drive_perception is missing the symbols this patcher replaces: "
                + ", ".join(missing)
            )
        # a second apply must wrap the published fallback, not our own wrapper
        original = self._originals.get(
            (attention.__name__, QWENDRIVE_MSDA_ATTR), getattr(attention, QWENDRIVE_MSDA_ATTR)
        )
        wrapper = _make_qwendrive_msda_wrapper(strict, original)
        patched = []
        for module, attr in ((attention, QWENDRIVE_MSDA_ATTR), (ops, QWENDRIVE_MSDA_FORWARD_ATTR)):
            if _patch_attr(self._originals, module, attr, wrapper):
                patched.append(module.__name__)
        action = "already-applied" if self._strict == strict else "applied"
        self._strict = strict
        return PatchReport(
            target=f"{QWENDRIVE_ATTENTION_MODULE}.{QWENDRIVE_MSDA_ATTR}",
            strict=strict,
            action=action,
            patched_modules=tuple(patched),
        )

    def restore(self) -> PatchReport:
        restored = _restore_attrs(self._originals)
        self._strict = None
        return PatchReport(
            target=f"{QWENDRIVE_ATTENTION_MODULE}.{QWENDRIVE_MSDA_ATTR}",
            strict=False,
            action="restored",
            patched_modules=tuple(restored),
        )


def _make_deformable_aggregation_wrapper(strict: bool) -> PatchCallable:
    """SparseDrive's ``deformable_aggregation_function`` signature (reference
    runtime.py:519-545): strict forces the HIP backend, otherwise ``auto``."""
    backend = "hip" if strict else "auto"

    def muspace_deformable_aggregation(feature_maps, spatial_shape, scale_start_index,
                                       sampling_location, weights):
        from ..ops.deformable_aggregation import deformable_aggregation_function

        return deformable_aggregation_function(feature_maps, spatial_shape, scale_start_index,
                                               sampling_location, weights, backend=backend)

    muspace_deformable_aggregation.__name__ = (
        "muspace_deformable_aggregation_strict" if strict else "muspace_deformable_aggregation"
    )
    muspace_deformable_aggregation.__module__ = __name__
    return muspace_deformable_aggregation


class SparseDrivePatcher:
    """Route SparseDrive's deformable aggregation to this operator.

    Rebinds ``projects.mmdet3d_plugin.ops.deformable_aggregation_function``,
    the ``DAF`` copy already imported by ``models.blocks``, and sets
    ``DAF_VALID = True`` where the checkout cached a failed extension probe
    (reference ``SparseDrivePatcher._patch_sparsedrive_daf``,
    runtime.py:1471-1510). The reference patcher's flash-attention and CUDA-shim
    replacements are outside this operator and not installed.
    """

    def __init__(self) -> None:
        self._originals: dict[tuple[str, str], object] = {}
        self._strict: bool | None = None

    def apply(self, *, strict: bool | None = None) -> PatchReport:
        strict = _env_strict() if strict is None else strict
        try:
            ops = importlib.import_module(SPARSEDRIVE_OPS_MODULE)
        except ImportError as exc:
            raise PatchError(
                "SparseDrive ops package import failed. Ensure the SparseDrive checkout is "
                "on PYTHONPATH before sparsedrive_patcher.apply()."
            ) from exc
        if not hasattr(ops, SPARSEDRIVE_DAF_ATTR):
            raise PatchError(f"{SPARSEDRIVE_OPS_MODULE}.{SPARSEDRIVE_DAF_ATTR} is unavailable")
        wrapper = _make_deformable_aggregation_wrapper(strict)
        _patch_attr(self._originals, ops, SPARSEDRIVE_DAF_ATTR, wrapper)
        patched = [ops.__name__]
        for name in SPARSEDRIVE_IMPORTED_MODULES:
            module = sys.modules.get(name)
            if module is not None and _patch_attr(self._originals, module,
                                                  SPARSEDRIVE_IMPORTED_ATTR, wrapper):
                patched.append(name)
        prefix = f"{SPARSEDRIVE_PACKAGE}."
        for name, module in list(sys.modules.items()):
            if module is None or not (name == SPARSEDRIVE_PACKAGE or name.startswith(prefix)):
                continue
            if getattr(module, SPARSEDRIVE_DAF_VALID_ATTR, None) is False:
                _patch_attr(self._originals, module, SPARSEDRIVE_DAF_VALID_ATTR, True)
                patched.append(name)
        action = "already-applied" if self._strict == strict else "applied"
        self._strict = strict
        return PatchReport(
            target=f"{SPARSEDRIVE_OPS_MODULE}.{SPARSEDRIVE_DAF_ATTR}",
            strict=strict,
            action=action,
            patched_modules=tuple(dict.fromkeys(patched)),
        )

    def restore(self) -> PatchReport:
        restored = _restore_attrs(self._originals)
        self._strict = None
        return PatchReport(
            target=f"{SPARSEDRIVE_OPS_MODULE}.{SPARSEDRIVE_DAF_ATTR}",
            strict=False,
            action="restored",
            patched_modules=tuple(restored),
        )


default_patcher = DefaultPatcher()
qwendrive_patcher = QwenDrivePatcher()
sparsedrive_patcher = SparseDrivePatcher()

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
