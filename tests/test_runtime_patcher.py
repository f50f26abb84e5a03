"""Drop-in swap tests, mirroring /root/reference/tests/test_runtime_patcher.py:20-111,191-233.

Fake mmcv / BEVFormer / UniAD / Qwen-Drive modules are installed in
``sys.modules``; the patcher must rebind the MSDA helper everywhere and undo
it on restore.
"""

import sys
import types

import pytest
import torch

from msda_testlib import reference_fixture
from muspace_amd.patcher import DefaultPatcher, PatchError, QwenDrivePatcher
from muspace_amd.patcher.runtime import _MissingLegacyExtension
from oracle import msda_torch

TARGET = "mmcv.ops.multi_scale_deform_attn"
ATTR = "multi_scale_deformable_attn_pytorch"
IMPORTED = "projects.mmdet3d_plugin.bevformer.modules.temporal_self_attention"
UNIAD_IMPORTED = "projects.mmdet3d_plugin.uniad.modules.temporal_self_attention"
EXT_LOADER = "mmcv.utils.ext_loader"


def _install_fake_module(monkeypatch, name: str):
    module = types.ModuleType(name)

    def original(*args, **kwargs):
        return "original"

    setattr(module, ATTR, original)
    monkeypatch.setitem(sys.modules, name, module)
    return module, original


def _install_fake_ext_loader(monkeypatch):
    module = types.ModuleType(EXT_LOADER)

    def load_ext(name, functions):
        raise ImportError(name)

    module.load_ext = load_ext
    monkeypatch.setitem(sys.modules, EXT_LOADER, module)
    return module, load_ext


def test_default_patcher_replaces_mmcv_msda_and_restores(monkeypatch):
    module, original = _install_fake_module(monkeypatch, TARGET)
    patcher = DefaultPatcher()
    report = patcher.apply()
    assert report.action == "applied"
    assert report.strict is False
    assert report.patched_modules == (TARGET,)
    assert getattr(module, ATTR) is not original
    assert getattr(module, ATTR).__name__ == "muspace_multi_scale_deformable_attn_compat"
    assert patcher.apply().action == "already-applied"
    restored = patcher.restore()
    assert restored.action == "restored"
    assert getattr(module, ATTR) is original


def test_patched_helper_computes_msda(monkeypatch):
    module, _ = _install_fake_module(monkeypatch, TARGET)
    patcher = DefaultPatcher()
    patcher.apply()
    value, shapes, _, loc, attn = reference_fixture(levels=((2, 3), (1, 2)), points=2)
    out = getattr(module, ATTR)(value, shapes, loc, attn)
    torch.testing.assert_close(out, msda_torch.msda_forward(value, shapes, loc, attn))
    patcher.restore()


def test_default_patcher_updates_already_imported_bevformer_modules(monkeypatch):
    module, _ = _install_fake_module(monkeypatch, TARGET)
    imported, imported_original = _install_fake_module(monkeypatch, IMPORTED)
    patcher = DefaultPatcher()
    report = patcher.apply()
    assert report.patched_modules == (TARGET, IMPORTED)
    assert getattr(module, ATTR) is getattr(imported, ATTR)
    assert getattr(imported, ATTR) is not imported_original
    patcher.restore()
    assert getattr(imported, ATTR) is imported_original


def test_default_patcher_updates_already_imported_uniad_modules(monkeypatch):
    module, _ = _install_fake_module(monkeypatch, TARGET)
    imported, imported_original = _install_fake_module(monkeypatch, UNIAD_IMPORTED)
    patcher = DefaultPatcher()
    report = patcher.apply()
    assert report.patched_modules == (TARGET, UNIAD_IMPORTED)
    assert getattr(module, ATTR) is getattr(imported, ATTR)
    assert getattr(imported, ATTR) is not imported_original
    patcher.restore()


def test_default_patcher_strict_mode_from_env(monkeypatch):
    module, _ = _install_fake_module(monkeypatch, TARGET)
    monkeypatch.setenv("MUSPACE_STRICT_PATCH", "1")
    report = DefaultPatcher().apply()
    assert report.strict is True
    assert getattr(module, ATTR).__name__ == "muspace_multi_scale_deformable_attn_strict"


def test_strict_wrapper_refuses_cpu_tensors(monkeypatch):
    module, _ = _install_fake_module(monkeypatch, TARGET)
    DefaultPatcher().apply(strict=True)
    value, shapes, _, loc, attn = reference_fixture()
    with pytest.raises(RuntimeError, match="requires a ROCm tensor"):
        getattr(module, ATTR)(value, shapes, loc, attn)


def test_missing_mmcv_is_a_patch_error(monkeypatch):
    monkeypatch.setitem(sys.modules, TARGET, None)
    with pytest.raises(PatchError, match="mmcv MSDeformAttn helper is unavailable"):
        DefaultPatcher().apply()


def test_restore_releases_legacy_extension_guard(monkeypatch):
    _install_fake_module(monkeypatch, TARGET)
    ext_loader, original_load_ext = _install_fake_ext_loader(monkeypatch)
    patcher = DefaultPatcher()
    patcher.apply()
    assert ext_loader.load_ext is not original_load_ext
    assert hasattr(ext_loader, "_muspace_original_load_ext")
    patcher.restore()
    assert ext_loader.load_ext is original_load_ext
    assert not hasattr(ext_loader, "_muspace_original_load_ext")
    patcher.restore()
    assert ext_loader.load_ext is original_load_ext


def test_legacy_extension_guard_returns_placeholder_for_failed_load(monkeypatch):
    _install_fake_module(monkeypatch, TARGET)
    ext_loader, _ = _install_fake_ext_loader(monkeypatch)
    patcher = DefaultPatcher()
    patcher.apply()
    placeholder = ext_loader.load_ext("_ext", ["nms"])
    assert isinstance(placeholder, _MissingLegacyExtension)
    assert hasattr(placeholder, "nms")
    assert placeholder.get_compiler_version() == "unavailable"
    with pytest.raises(PatchError, match="mmcv._ext is unavailable"):
        placeholder.nms()
    patcher.restore()


# ------------------------------------------------------------ Qwen-Drive ---

QW_ATTENTION = "qwen_drive_perception.attention"
QW_OPS = "qwen_drive_perception.ops"


def _install_fake_qwendrive(monkeypatch):
    package = types.ModuleType("qwen_drive_perception")
    attention = types.ModuleType(QW_ATTENTION)
    ops = types.ModuleType(QW_OPS)

    def msda(*args):
        return ("pytorch", args)

    def forward(*args):
        return ("cuda-forward", args)

    attention.multi_scale_deformable_attn_cuda = msda
    ops.ms_deform_attn_bf16_forward = forward
    monkeypatch.setitem(sys.modules, "qwen_drive_perception", package)
    monkeypatch.setitem(sys.modules, QW_ATTENTION, attention)
    monkeypatch.setitem(sys.modules, QW_OPS, ops)
    return attention, ops, msda, forward


def test_qwendrive_patcher_rebinds_and_restores(monkeypatch):
    attention, ops, msda, forward = _install_fake_qwendrive(monkeypatch)
    patcher = QwenDrivePatcher()
    report = patcher.apply()
    assert report.patched_modules == (QW_ATTENTION, QW_OPS)
    assert attention.multi_scale_deformable_attn_cuda is ops.ms_deform_attn_bf16_forward
    assert attention.multi_scale_deformable_attn_cuda.__name__ == "muspace_qwendrive_msda"
    patcher.apply()  # a second apply keeps the published fallback
    patcher.restore()
    assert attention.multi_scale_deformable_attn_cuda is msda
    assert ops.ms_deform_attn_bf16_forward is forward


def test_qwendrive_msda_wrapper_routes_by_device(monkeypatch):
    attention, ops, *_ = _install_fake_qwendrive(monkeypatch)
    captured = {}

    def fake_msda(*args, **kwargs):
        captured["args"] = args
        captured["kwargs"] = kwargs
        return "native"

    monkeypatch.setattr("muspace_amd.ops.multi_scale_deformable_attn", fake_msda)
    patcher = QwenDrivePatcher()
    patcher.apply()
    wrapper = attention.multi_scale_deformable_attn_cuda
    gpu = types.SimpleNamespace(dtype=torch.bfloat16, device=types.SimpleNamespace(type="cuda"),
                                is_cuda=True)
    assert wrapper(gpu, "shapes", "starts", "locations", "weights", 64) == "native"
    assert captured["kwargs"]["im2col_step"] == 64
    assert captured["kwargs"]["backend"] == "auto"
    assert captured["args"][1] == "shapes"
    with pytest.raises(TypeError, match="bfloat16"):
        wrapper(types.SimpleNamespace(dtype=torch.float32, device=types.SimpleNamespace(type="cuda"),
                                      is_cuda=True), None, None, None, None, 64)
    cpu = types.SimpleNamespace(dtype=torch.float32, device=types.SimpleNamespace(type="cpu"),
                                is_cuda=False)
    assert wrapper(cpu, "shapes", "starts", "locations", "weights", 64)[0] == "pytorch"
    assert ops.ms_deform_attn_bf16_forward is wrapper
    patcher.restore()


def test_qwendrive_missing_symbols_is_a_patch_error(monkeypatch):
    attention, *_ = _install_fake_qwendrive(monkeypatch)
    monkeypatch.delattr(attention, "multi_scale_deformable_attn_cuda")
    with pytest.raises(PatchError, match="missing the symbols"):
        QwenDrivePatcher().apply()


# ------------------------------------------------------------ SparseDrive ---


def test_sparsedrive_patcher(monkeypatch):
    """Reference tests/ops/test_deformable_aggregation.py:112-131."""
    from muspace_amd.patcher import SparseDrivePatcher

    ops = types.ModuleType("projects.mmdet3d_plugin.ops")
    blocks = types.ModuleType("projects.mmdet3d_plugin.models.blocks")

    def original(*args, **kwargs):
        return "original"

    ops.deformable_aggregation_function = original
    blocks.DAF = original
    blocks.DAF_VALID = False
    monkeypatch.setitem(sys.modules, ops.__name__, ops)
    monkeypatch.setitem(sys.modules, blocks.__name__, blocks)

    patcher = SparseDrivePatcher()
    report = patcher.apply()
    assert report.action == "applied"
    assert ops.deformable_aggregation_function is not original
    assert blocks.DAF is ops.deformable_aggregation_function
    assert blocks.DAF_VALID is True
    assert ops.deformable_aggregation_function.__name__ == "muspace_deformable_aggregation"
    assert patcher.restore().action == "restored"
    assert ops.deformable_aggregation_function is original and blocks.DAF is original
    assert blocks.DAF_VALID is False


def test_sparsedrive_patched_entry_computes_on_the_cpu(monkeypatch):
    from muspace_amd.patcher import SparseDrivePatcher
    from test_dfa_oracle import SMALL_EXPECTED, small_case

    ops = types.ModuleType("projects.mmdet3d_plugin.ops")
    ops.deformable_aggregation_function = lambda *a: None
    monkeypatch.setitem(sys.modules, ops.__name__, ops)
    patcher = SparseDrivePatcher()
    patcher.apply()
    mc, spatial, start, loc, weights = small_case()
    out = ops.deformable_aggregation_function(mc, spatial.long(), start.long(), loc, weights)
    torch.testing.assert_close(out, SMALL_EXPECTED)
    patcher.restore()


def test_sparsedrive_missing_ops_module_is_a_patch_error(monkeypatch):
    from muspace_amd.patcher import SparseDrivePatcher

    monkeypatch.setitem(sys.modules, "projects.mmdet3d_plugin.ops", None)
    with pytest.raises(PatchError, match="SparseDrive ops package import failed"):
        SparseDrivePatcher().apply()


def test_two_patchers_share_one_extension_guard(monkeypatch):
    """The guard belongs to the patcher that installed it: a second patcher
    neither stacks another guard nor removes the first one's."""
    _install_fake_module(monkeypatch, TARGET)
    ext_loader, original_load_ext = _install_fake_ext_loader(monkeypatch)
    first, second = DefaultPatcher(), DefaultPatcher()
    first.apply()
    guarded = ext_loader.load_ext
    second.apply()
    assert ext_loader.load_ext is guarded
    second.restore()
    assert ext_loader.load_ext is guarded
    first.restore()
    assert ext_loader.load_ext is original_load_ext
    assert not hasattr(ext_loader, "_muspace_original_load_ext")


def test_strict_then_compat_restores_the_original(monkeypatch):
    module, original = _install_fake_module(monkeypatch, TARGET)
    patcher = DefaultPatcher()
    assert patcher.apply(strict=True).action == "applied"
    assert patcher.apply(strict=False).action == "applied"
    assert getattr(module, ATTR).__name__ == "muspace_multi_scale_deformable_attn_compat"
    assert patcher.restore().patched_modules == (TARGET,)
    assert getattr(module, ATTR) is original
