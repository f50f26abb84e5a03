"""Runtime patches that route model code's MSDA calls to this operator.

Interface kept from /root/reference/mu_space/patcher/runtime.py (names, target
module paths, wrapper ``__name__``s, ``PatchReport`` fields, error types and
messages its tests match):
  * ``DefaultPatcher`` (reference :577-636) replaces mmcv's 4-argument helper
    ``mmcv.ops.multi_scale_deform_attn.multi_scale_deformable_attn_pytorch``
    plus the copies already bound in imported BEVFormer / UniAD modules, and
    keeps mmcv's ``load_ext`` from raising when the compiled ``mmcv._ext`` is
    absent (:97-159); ``restore()`` undoes all of it;
  * strict / compat routes (:398-439): strict forces the native backend,
    compat uses ``auto``; ``MUSPACE_STRICT_PATCH`` selects strict (:272-273);
  * ``QwenDrivePatcher``: the Qwen-Drive bf16 MSDA entry (:285-337). The
    reference's Qwen-Drive patcher also replaces a voxel-pool operator and a
    frustum property, which are other operators; only the two MSDA symbols
    are patched here;
  * ``SparseDrivePatcher``: SparseDrive's deformable aggregation (:1471-1510).

Design: every patcher is a list of *sites* (module, attribute) that a
``_BindingLedger`` rebinds and remembers, so ``restore()`` is one generic
undo. The mmcv extension loader guard is one more ledger entry whose owner
is marked on the loader module itself, so two patchers never stack guards.
"""

from __future__ import annotations

import importlib
import os
import sys
from collections.abc import Callable, Iterable
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

# the loader's own load_ext while it is guarded (interface: the reference's
# tests look for this attribute on the loader module)
_SAVED_LOAD_EXT = "_muspace_original_load_ext"
_VERSION_PROBES = frozenset({"get_compiler_version", "get_compiling_cuda_version"})


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


def _truthy(text: str | None) -> bool:
    return (text or "").strip().lower() in {"1", "true", "yes", "on"}


def _strict_requested(strict: bool | None) -> bool:
    return _truthy(os.environ.get(STRICT_ENV)) if strict is None else bool(strict)


def _named(fn: PatchCallable, name: str) -> PatchCallable:
    """Give a generated route a stable, patcher-owned identity."""
    fn.__name__ = fn.__qualname__ = name
    fn.__module__ = __name__
    return fn


# ------------------------------------------------------------ the ledger ---


class _BindingLedger:
    """Module attributes this process rebound, with what they held before.

    The first value seen for a (module, attribute) site is the one restored,
    however many times the site is rebound in between.
    """

    def __init__(self) -> None:
        self._before: dict[tuple[str, str], object] = {}

    def original(self, module: ModuleType, attr: str, default: object = None) -> object:
        return self._before.get((module.__name__, attr), getattr(module, attr, default))

    def rebind(self, module: ModuleType, attr: str, value: object) -> bool:
        """Replace an existing ``module.attr``; False (nothing done) if absent."""
        if not hasattr(module, attr):
            return False
        self._before.setdefault((module.__name__, attr), getattr(module, attr))
        setattr(module, attr, value)
        return True

    def undo(self) -> list[str]:
        """Restore every site still importable, newest first; forget them all."""
        restored = []
        for (module_name, attr), value in reversed(list(self._before.items())):
            module = sys.modules.get(module_name)
            if module is not None:
                setattr(module, attr, value)
                restored.append(module_name)
        self._before.clear()
        restored.reverse()
        return restored


# -------------------------------------------- mmcv compiled-extension guard ---


class _MissingLegacyExtension:
    """Returned by the guarded ``load_ext`` for an mmcv extension that failed to load.

    Model modules probe these objects at import time (``hasattr``), so any
    public attribute exists; the version queries answer "unavailable"; calling
    anything else raises ``PatchError`` naming the extension and the function.
    """

    def __init__(self, name: str, functions: object) -> None:
        self.name = name
        self.functions = functions

    def __getattr__(self, attr: str) -> object:
        if attr.startswith("__") and attr.endswith("__"):
            raise AttributeError(attr)
        if attr in _VERSION_PROBES:
            return _unavailable_version
        return _MissingFunction(self.name, attr)


def _unavailable_version() -> str:
    return "unavailable"


class _MissingFunction:
    """A function of a missing mmcv extension: raises when called."""

    def __init__(self, extension: str, name: str) -> None:
        self.extension = extension
        self.__name__ = name

    def __call__(self, *args: object, **kwargs: object) -> object:
        raise PatchError(
            f"Legacy extension mmcv.{self.extension} is unavailable; the muSPACE replacement "
            f"must handle this path before {self.__name__} is called"
        )


def _guarded(load_ext: PatchCallable) -> PatchCallable:
    def load_ext_or_placeholder(name: str, functions: object):
        try:
            return load_ext(name, functions)
        except (ImportError, OSError):
            return _MissingLegacyExtension(name, functions)

    return _named(load_ext_or_placeholder, "load_ext")


class _ExtensionGuard:
    """Owns the guard on mmcv's ``load_ext`` when this patcher installed it."""

    def __init__(self) -> None:
        self.owned = False

    def install(self) -> None:
        try:
            loader = importlib.import_module(EXT_LOADER_MODULE)
        except ImportError:
            return
        if hasattr(loader, _SAVED_LOAD_EXT):  # guarded already (by us or another patcher)
            return
        setattr(loader, _SAVED_LOAD_EXT, loader.load_ext)
        loader.load_ext = _guarded(loader.load_ext)
        self.owned = True

    def release(self) -> None:
        if not self.owned:
            return
        self.owned = False
        loader = sys.modules.get(EXT_LOADER_MODULE)
        saved = getattr(loader, _SAVED_LOAD_EXT, None) if loader is not None else None
        if saved is not None:
            loader.load_ext = saved
            delattr(loader, _SAVED_LOAD_EXT)


# ---------------------------------------------------------------- routes ---


def _msda_route(strict: bool) -> PatchCallable:
    """mmcv's 4-argument helper routed to the operator (level starts derived
    from the shapes): strict forces the HIP backend, compat uses ``auto``."""
    backend = "hip" if strict else "auto"

    def route(value, value_spatial_shapes, sampling_locations, attention_weights):
        from ..ops.multi_scale_deformable_attn import (
            level_start_index_from_shapes,
            multi_scale_deformable_attn,
        )

        return multi_scale_deformable_attn(
            value, value_spatial_shapes, level_start_index_from_shapes(value_spatial_shapes),
            sampling_locations, attention_weights, backend=backend)

    suffix = "strict" if strict else "compat"
    return _named(route, f"muspace_multi_scale_deformable_attn_{suffix}")


def _accelerated_tensor(value) -> bool:
    """True for a tensor on a GPU: ``cuda`` (ROCm) or the reference's MUSA spellings."""
    device_type = getattr(getattr(value, "device", None), "type", None)
    if device_type in {"cuda", "musa", "privateuseone"}:
        return True
    return bool(getattr(value, "is_cuda", False) or getattr(value, "is_musa", False))


def _qwendrive_route(strict: bool, fallback: PatchCallable) -> PatchCallable:
    """Qwen-Drive's 6-argument bf16 MSDA entry (reference runtime.py:285-337):
    bfloat16 GPU tensors go through the operator with the caller's
    ``im2col_step``; another dtype on a GPU is a ``TypeError``; tensors on
    other devices keep ``fallback`` (the published PyTorch implementation)."""
    backend = "hip" if strict else "auto"

    def route(value, value_spatial_shapes, value_level_start_index, sampling_locations,
              attention_weights, im2col_step):
        args = (value, value_spatial_shapes, value_level_start_index, sampling_locations,
                attention_weights)
        if not _accelerated_tensor(value):
            return fallback(*args, im2col_step)
        import torch

        if value.dtype != torch.bfloat16:
            raise TypeError(
                "the ms_deform_attn kernel requires bfloat16 tensors on the GPU, "
                f"got {value.dtype}; run the model in bfloat16")
        from .. import ops

        return ops.multi_scale_deformable_attn(*args, im2col_step=int(im2col_step),
                                               backend=backend)

    return _named(route, "muspace_qwendrive_msda_strict" if strict else "muspace_qwendrive_msda")


def _aggregation_route(strict: bool) -> PatchCallable:
    """SparseDrive's ``deformable_aggregation_function`` signature (reference
    runtime.py:519-545): strict forces the HIP backend, otherwise ``auto``."""
    backend = "hip" if strict else "auto"

    def route(feature_maps, spatial_shape, scale_start_index, sampling_location, weights):
        from ..ops.deformable_aggregation import deformable_aggregation_function

        return deformable_aggregation_function(feature_maps, spatial_shape, scale_start_index,
                                               sampling_location, weights, backend=backend)

    return _named(route, "muspace_deformable_aggregation_strict" if strict
                  else "muspace_deformable_aggregation")


# -------------------------------------------------------------- patchers ---


def _import_or_patch_error(names: Iterable[str], message: str) -> list[ModuleType]:
    try:
        return [importlib.import_module(name) for name in names]
    except ImportError as exc:
        raise PatchError(message) from exc


def _loaded(names: Iterable[str]) -> list[ModuleType]:
    return [sys.modules[n] for n in names if sys.modules.get(n) is not None]


class _RoutePatcher:
    """apply()/restore() over a ledger of rebound sites; subclasses say which
    sites to rebind (``_install``) and what ``target`` the reports name."""

    target = ""

    def __init__(self) -> None:
        self._ledger = _BindingLedger()
        self._strict: bool | None = None

    def apply(self, *, strict: bool | None = None) -> PatchReport:
        strict = _strict_requested(strict)
        modules = self._install(strict)
        action = "already-applied" if self._strict == strict else "applied"
        self._strict = strict
        return PatchReport(self.target, strict, action, tuple(dict.fromkeys(modules)))

    def restore(self) -> PatchReport:
        restored = self._ledger.undo()
        self._release()
        self._strict = None
        return PatchReport(self.target, False, "restored", tuple(restored))

    def _install(self, strict: bool) -> list[str]:
        raise NotImplementedError

    def _release(self) -> None:
        pass

    def _rebind_all(self, modules: Iterable[ModuleType], attr: str, value: object) -> list[str]:
        return [m.__name__ for m in modules if self._ledger.rebind(m, attr, value)]


class DefaultPatcher(_RoutePatcher):
    """Swap mmcv's MSDA helper for this operator without editing model code."""

    target = f"{MSDA_TARGET_MODULE}.{MSDA_TARGET_ATTR}"

    def __init__(self) -> None:
        super().__init__()
        self._guard = _ExtensionGuard()

    def _install(self, strict: bool) -> list[str]:
        self._guard.install()
        (helper,) = _import_or_patch_error(
            (MSDA_TARGET_MODULE,),
            "mmcv MSDeformAttn helper is unavailable; install the BEVFormer OpenMMLab stack "
            "before calling default_patcher.apply()")
        route = _msda_route(strict)
        if not self._ledger.rebind(helper, MSDA_TARGET_ATTR, route):
            raise PatchError(f"{MSDA_TARGET_MODULE}.{MSDA_TARGET_ATTR} is unavailable")
        # model modules bound the helper at import time: rebind those copies too
        copies = _loaded((*BEVFORMER_IMPORTED_MODULES, *UNIAD_IMPORTED_MODULES))
        return [helper.__name__, *self._rebind_all(copies, MSDA_TARGET_ATTR, route)]

    def _release(self) -> None:
        self._guard.release()


class QwenDrivePatcher(_RoutePatcher):
    """Route Qwen-Drive's MSDA entry points to this operator (MSDA symbols only)."""

    target = f"{QWENDRIVE_ATTENTION_MODULE}.{QWENDRIVE_MSDA_ATTR}"

    def _install(self, strict: bool) -> list[str]:
        attention, ops = _import_or_patch_error(
            (QWENDRIVE_ATTENTION_MODULE, QWENDRIVE_OPS_MODULE),
            "qwen_drive_perception import failed. Add the Qwen-Drive checkout src directory "
            "to PYTHONPATH before qwendrive_patcher.apply().")
        sites = ((attention, QWENDRIVE_MSDA_ATTR), (ops, QWENDRIVE_MSDA_FORWARD_ATTR))
        missing = [f"{m.__name__}.{a}" for m, a in sites if not callable(getattr(m, a, None))]
        if missing:
            raise PatchError("qwen_drive_perception is missing the symbols this patcher "
                             "replaces: " + ", ".join(missing))
        # the published PyTorch entry, even when a route of ours is bound now
        fallback = self._ledger.original(attention, QWENDRIVE_MSDA_ATTR)
        route = _qwendrive_route(strict, fallback)
        return [m.__name__ for m, a in sites if self._ledger.rebind(m, a, route)]


class SparseDrivePatcher(_RoutePatcher):
    """Route SparseDrive's deformable aggregation to this operator.

    Rebinds ``projects.mmdet3d_plugin.ops.deformable_aggregation_function``,
    the ``DAF`` copy already imported by ``models.blocks``, and sets
    ``DAF_VALID = True`` where the checkout cached a failed extension probe
    (reference ``SparseDrivePatcher._patch_sparsedrive_daf``,
    runtime.py:1471-1510). The reference patcher's flash-attention and CUDA-shim
    replacements are outside this operator and not installed.
    """

    target = f"{SPARSEDRIVE_OPS_MODULE}.{SPARSEDRIVE_DAF_ATTR}"

    def _install(self, strict: bool) -> list[str]:
        (ops,) = _import_or_patch_error(
            (SPARSEDRIVE_OPS_MODULE,),
            "SparseDrive ops package import failed. Ensure the SparseDrive checkout is on "
            "PYTHONPATH before sparsedrive_patcher.apply().")
        if not hasattr(ops, SPARSEDRIVE_DAF_ATTR):
            raise PatchError(f"{SPARSEDRIVE_OPS_MODULE}.{SPARSEDRIVE_DAF_ATTR} is unavailable")
        route = _aggregation_route(strict)
        patched = self._rebind_all((ops,), SPARSEDRIVE_DAF_ATTR, route)
        patched += self._rebind_all(_loaded(SPARSEDRIVE_IMPORTED_MODULES),
                                    SPARSEDRIVE_IMPORTED_ATTR, route)
        prefix = SPARSEDRIVE_PACKAGE + "."
        stale = [m for name, m in list(sys.modules.items())
                 if m is not None and (name == SPARSEDRIVE_PACKAGE or name.startswith(prefix))
                 and getattr(m, SPARSEDRIVE_DAF_VALID_ATTR, None) is False]
        patched += self._rebind_all(stale, SPARSEDRIVE_DAF_VALID_ATTR, True)
        return patched


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
