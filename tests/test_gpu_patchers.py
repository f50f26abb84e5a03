"""The drop-in routes on ROCm tensors: the patched helpers reach the HIP kernels.

The CPU tests (test_runtime_patcher.py) check that the patchers rebind the right
symbols; these run the rebound callables on the GPU. They follow the callers
the reference patches: mmcv's 4-argument helper
(/root/reference/mu_space/patcher/runtime.py:398-439) and Qwen-Drive's
6-argument bf16 entry (runtime.py:285-337), whose published gate admits
bfloat16 device tensors only. Expected values come from the CPU oracle;
tolerances are the reference tests' (1e-5 fp32 forward and 1e-4 fp32
gradients, 2e-2 for bf16: tests/ops/test_multi_scale_deformable_attn.py:414).
"""

import sys
import types

import pytest
import torch

from conftest import gpu_available
from msda_testlib import reference_fixture
from muspace_amd import clear_dispatch_report, get_last_dispatch_report
from muspace_amd.patcher import DefaultPatcher, QwenDrivePatcher
from oracle import msda_torch

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not gpu_available(), reason="AMD GPU required"),
]

DEV = "cuda"
MMCV = "mmcv.ops.multi_scale_deform_attn"
MMCV_ATTR = "multi_scale_deformable_attn_pytorch"
QW_ATTENTION = "qwen_drive_perception.attention"
QW_OPS = "qwen_drive_perception.ops"


def _cpu_reference(tensors):
    """fp32 CPU leaves of the floating tensors (bf16 values are widened exactly)."""
    out = []
    for t in tensors:
        if t.dtype.is_floating_point:
            out.append(t.detach().cpu().float().requires_grad_(True))
        else:
            out.append(t.detach().cpu())
    return out


def _install_fake_mmcv(monkeypatch):
    module = types.ModuleType(MMCV)

    def original(*args):
        raise AssertionError("the patched helper must not call mmcv's own path for device tensors")

    setattr(module, MMCV_ATTR, original)
    monkeypatch.setitem(sys.modules, MMCV, module)
    return module


def _install_fake_qwendrive(monkeypatch):
    package = types.ModuleType("qwen_drive_perception")
    attention = types.ModuleType(QW_ATTENTION)
    ops = types.ModuleType(QW_OPS)

    def published(*args):
        raise AssertionError("bfloat16 device tensors must not reach the published fallback")

    attention.multi_scale_deformable_attn_cuda = published
    ops.ms_deform_attn_bf16_forward = published
    monkeypatch.setitem(sys.modules, "qwen_drive_perception", package)
    monkeypatch.setitem(sys.modules, QW_ATTENTION, attention)
    monkeypatch.setitem(sys.modules, QW_OPS, ops)
    return attention, ops


@pytest.mark.parametrize("strict", [False, True])
def test_mmcv_helper_runs_the_hip_kernels(monkeypatch, strict):
    module = _install_fake_mmcv(monkeypatch)
    patcher = DefaultPatcher()
    patcher.apply(strict=strict)
    try:
        clear_dispatch_report()
        value, shapes, _, loc, attn = reference_fixture(
            device=DEV, batch=2, queries=17, heads=8, embed_dims=32,
            levels=((7, 9), (4, 5), (2, 3)), points=4)
        ref = _cpu_reference((value, shapes, loc, attn))
        out = getattr(module, MMCV_ATTR)(value, shapes, loc, attn)
        report = get_last_dispatch_report()
        assert report.selected_backend == "hip"
        assert report.native_fallback is False
        expected = msda_torch.msda_forward(*ref)
        torch.testing.assert_close(out.detach().cpu(), expected.detach(), rtol=1e-5, atol=1e-5)
        g = torch.randn(out.shape, generator=torch.Generator().manual_seed(5))
        (out * g.to(DEV)).sum().backward()
        (expected * g).sum().backward()
        for native, cpu in ((value, ref[0]), (loc, ref[2]), (attn, ref[3])):
            torch.testing.assert_close(native.grad.cpu(), cpu.grad, rtol=1e-4, atol=1e-4)
    finally:
        patcher.restore()


@pytest.mark.parametrize("strict", [False, True])
def test_qwendrive_entry_runs_bf16_forward_and_backward_on_the_gpu(monkeypatch, strict):
    attention, ops = _install_fake_qwendrive(monkeypatch)
    patcher = QwenDrivePatcher()
    patcher.apply(strict=strict)
    try:
        clear_dispatch_report()
        value, shapes, starts, loc, attn = reference_fixture(
            device=DEV, dtype=torch.bfloat16, batch=1, queries=9, heads=4, embed_dims=32,
            levels=((5, 6), (3, 3)), points=4)
        ref = _cpu_reference((value, shapes, loc, attn))
        out = attention.multi_scale_deformable_attn_cuda(value, shapes, starts, loc, attn, 64)
        assert out.dtype == torch.bfloat16
        report = get_last_dispatch_report()
        assert report.selected_backend == "hip"
        assert report.native_fallback is False
        expected = msda_torch.msda_forward(*ref)
        grad = torch.linspace(0.1, 1.0, out.numel()).view(out.shape)
        (out.float() * grad.to(DEV)).sum().backward()
        (expected * grad).sum().backward()
        tolerance = 2e-2
        torch.testing.assert_close(out.float().cpu(), expected.detach(), rtol=tolerance,
                                   atol=tolerance)
        for native, cpu in ((value, ref[0]), (loc, ref[2]), (attn, ref[3])):
            torch.testing.assert_close(native.grad.float().cpu(), cpu.grad, rtol=tolerance,
                                       atol=tolerance)
        # The ops-module symbol is the same entry.
        again = ops.ms_deform_attn_bf16_forward(value.detach(), shapes, starts, loc.detach(),
                                                attn.detach(), 64)
        torch.testing.assert_close(again, out.detach(), rtol=0, atol=0)
    finally:
        patcher.restore()


def test_qwendrive_entry_rejects_float32_device_tensors(monkeypatch):
    attention, _ = _install_fake_qwendrive(monkeypatch)
    patcher = QwenDrivePatcher()
    patcher.apply()
    try:
        value, shapes, starts, loc, attn = reference_fixture(device=DEV, requires_grad=False)
        with pytest.raises(TypeError, match="bfloat16"):
            attention.multi_scale_deformable_attn_cuda(value, shapes, starts, loc, attn, 64)
    finally:
        patcher.restore()
