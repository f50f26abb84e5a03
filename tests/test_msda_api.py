"""CPU contract tests of the operator API.

Mirrors the CPU tests of /root/reference/tests/ops/test_multi_scale_deformable_attn.py
(:84-253, :471-481) with the native backend renamed from MUSA to HIP.
"""

from importlib import import_module

import pytest
import torch

from msda_testlib import reference_fixture as _fixture
from muspace_amd import (
    clear_dispatch_report,
    explain_dispatch,
    get_dispatch_reports,
    get_last_dispatch_report,
    multi_scale_deformable_attn,
)
from oracle import msda_torch

msda_module = import_module("muspace_amd.ops.multi_scale_deformable_attn")
dispatch_module = import_module("muspace_amd.runtime.kernel_dispatch")


def test_reference_forward_backward_on_cpu():
    clear_dispatch_report()
    value, spatial_shapes, level_start_index, sampling_locations, attention_weights = _fixture()
    output = multi_scale_deformable_attn(
        value, spatial_shapes, level_start_index, sampling_locations, attention_weights,
        backend="reference",
    )
    assert output.shape == (1, 5, 6)
    output.sum().backward()
    for t in (value, sampling_locations, attention_weights):
        assert t.grad is not None
        assert torch.isfinite(t.grad).all()
    report = get_last_dispatch_report()
    assert report is not None
    assert report.operator == "multi_scale_deformable_attn"
    assert report.requested_backend == "reference"
    assert report.selected_backend == "reference"
    assert report.native_fallback is False


def test_reference_path_equals_oracle_bitwise():
    """The product's reference backend is the reference path's op sequence."""
    value, shapes, starts, loc, attn = _fixture(batch=2, queries=6, heads=3, embed_dims=4,
                                                levels=((2, 3), (3, 1)), points=3)
    out = multi_scale_deformable_attn(value, shapes, starts, loc, attn, backend="reference")
    expect = msda_torch.msda_forward(value, shapes, loc, attn)
    assert torch.equal(out, expect)


def test_auto_cpu_dispatch_uses_reference():
    clear_dispatch_report()
    value, *_ = _fixture()
    decision = explain_dispatch(value, backend="auto")
    assert decision.backend == "reference"
    assert decision.device == "cpu"


@pytest.mark.parametrize(
    ("batch", "queries", "heads", "embed_dims", "levels", "points"),
    [
        (1, 5, 2, 3, ((2, 2),), 4),
        (2, 3, 4, 2, ((1, 3), (2, 1)), 2),
        (1, 7, 1, 8, ((1, 1), (1, 2), (2, 2)), 3),
    ],
)
def test_reference_shape_coverage_on_cpu(batch, queries, heads, embed_dims, levels, points):
    tensors = _fixture(batch=batch, queries=queries, heads=heads, embed_dims=embed_dims,
                       levels=levels, points=points)
    output = multi_scale_deformable_attn(*tensors, backend="reference")
    assert output.shape == (batch, queries, heads * embed_dims)
    output.square().mean().backward()
    value, _, _, sampling_locations, attention_weights = tensors
    for t in (value, sampling_locations, attention_weights):
        assert torch.isfinite(t.grad).all()


def test_reference_accepts_noncontiguous_inputs_on_cpu():
    tensors = _fixture(batch=2, queries=3, heads=2, embed_dims=4, levels=((1, 2), (2, 2)),
                       points=2, noncontiguous=True)
    value, _, _, sampling_locations, _ = tensors
    assert not value.is_contiguous()
    assert not sampling_locations.is_contiguous()
    output = multi_scale_deformable_attn(*tensors, backend="reference")
    assert output.shape == (2, 3, 8)


def test_sampling_and_attention_dtypes_follow_value_dtype():
    value, spatial_shapes, level_start_index, sampling_locations, attention_weights = _fixture()
    output = multi_scale_deformable_attn(
        value, spatial_shapes, level_start_index, sampling_locations.double(),
        attention_weights.double(), backend="reference",
    )
    assert output.dtype == value.dtype


def test_invalid_backend_fails_explicitly():
    clear_dispatch_report()
    tensors = _fixture()
    with pytest.raises(RuntimeError, match="unknown backend"):
        multi_scale_deformable_attn(*tensors, backend="unknown")
    report = get_last_dispatch_report()
    assert report is not None
    assert report.selected_backend == "error"
    assert report.reason == "unknown backend: unknown"


@pytest.mark.parametrize("backend", ["hip", "musa"])
def test_native_backend_on_cpu_tensor_is_an_error(backend):
    clear_dispatch_report()
    with pytest.raises(RuntimeError, match="requires a ROCm tensor"):
        multi_scale_deformable_attn(*_fixture(), backend=backend)
    assert get_last_dispatch_report().selected_backend == "error"


def test_dispatch_log_env_writes_stderr(monkeypatch, capsys):
    clear_dispatch_report()
    monkeypatch.setenv("MUSPACE_DISPATCH_LOG", "1")
    multi_scale_deformable_attn(*_fixture(), backend="reference")
    captured = capsys.readouterr()
    assert "muSPACE dispatch:" in captured.err
    assert '"selected_backend": "reference"' in captured.err


def test_dispatch_report_history_is_bounded(monkeypatch):
    clear_dispatch_report()
    monkeypatch.setattr(dispatch_module, "_dispatch_reports",
                        type(dispatch_module._dispatch_reports)(maxlen=3))
    tensors = _fixture()
    for _ in range(5):
        multi_scale_deformable_attn(*tensors, backend="reference")
    assert len(get_dispatch_reports()) == 3


def test_auto_native_failure_records_reference_fallback(monkeypatch):
    clear_dispatch_report()
    tensors = _fixture()
    monkeypatch.setattr(msda_module, "_native_extension", lambda: object())
    monkeypatch.setattr(msda_module, "_requires_native_backend", lambda *args: True)
    monkeypatch.setattr(
        msda_module,
        "_explain_dispatch",
        lambda value, *, backend, native_available: msda_module.DispatchDecision(
            "hip", value.device.type, "simulated ROCm tensor selects native backend"
        ),
    )

    def fail_native(*args, **kwargs):
        raise RuntimeError("simulated native failure")

    monkeypatch.setattr(msda_module._NativeMSDAFunction, "apply", fail_native)
    with pytest.warns(RuntimeWarning, match="simulated native failure"):
        output = multi_scale_deformable_attn(*tensors, backend="auto")
    assert output.shape == (1, 5, 6)
    report = get_last_dispatch_report()
    assert report.requested_backend == "auto"
    assert report.selected_backend == "reference"
    assert report.native_available is True
    assert report.native_fallback is True
    assert report.fallback_reason == "simulated native failure"


def test_forced_native_failure_is_reraised(monkeypatch):
    clear_dispatch_report()
    monkeypatch.setattr(msda_module, "_native_extension", lambda: object())
    monkeypatch.setattr(msda_module, "_requires_native_backend", lambda *args: True)
    monkeypatch.setattr(
        msda_module,
        "_explain_dispatch",
        lambda value, *, backend, native_available: msda_module.DispatchDecision(
            "hip", value.device.type, "forced HIP backend"
        ),
    )

    def fail_native(*args, **kwargs):
        raise RuntimeError("simulated native failure")

    monkeypatch.setattr(msda_module._NativeMSDAFunction, "apply", fail_native)
    with pytest.raises(RuntimeError, match="simulated native failure"):
        multi_scale_deformable_attn(*_fixture(), backend="hip")
    report = get_last_dispatch_report()
    assert report.selected_backend == "error"
    assert report.reason == "simulated native failure"


def test_rocm_tensor_without_library_is_an_error_not_a_fallback(monkeypatch):
    """auto on a ROCm tensor never silently leaves the HIP kernels."""
    monkeypatch.setattr(dispatch_module, "is_rocm_tensor", lambda tensor: True)
    decision = dispatch_module.explain_dispatch(torch.zeros(1), backend="auto",
                                                native_available=False)
    assert decision.backend == "error"
    assert "unavailable" in decision.reason
    forced = dispatch_module.explain_dispatch(torch.zeros(1), backend="musa",
                                              native_available=True)
    assert forced.backend == "hip"


def test_auto_fallback_env_restores_the_reference_policy(monkeypatch):
    """MUSPACE_AUTO_FALLBACK=1: auto on a ROCm tensor without the library takes
    the PyTorch path with the reason recorded (reference kernel_dispatch.py:94-100);
    a forced native backend still fails."""
    monkeypatch.setattr(dispatch_module, "is_rocm_tensor", lambda tensor: True)
    monkeypatch.setenv("MUSPACE_AUTO_FALLBACK", "1")
    decision = dispatch_module.explain_dispatch(torch.zeros(1), backend="auto",
                                                native_available=False)
    assert decision.backend == "reference"
    assert decision.reason == "HIP backend is unavailable; falling back to PyTorch reference"
    forced = dispatch_module.explain_dispatch(torch.zeros(1), backend="hip",
                                              native_available=False)
    assert forced.backend == "error"


def test_spatial_shape_dtype_is_validated():
    value, spatial_shapes, level_start_index, sampling_locations, attention_weights = _fixture()
    with pytest.raises(TypeError, match="spatial_shapes must be int64"):
        multi_scale_deformable_attn(value, spatial_shapes.to(torch.int32), level_start_index,
                                    sampling_locations, attention_weights, backend="reference")


def test_level_start_index_dtype_is_validated():
    value, spatial_shapes, level_start_index, sampling_locations, attention_weights = _fixture()
    with pytest.raises(TypeError, match="level_start_index must be int64"):
        multi_scale_deformable_attn(value, spatial_shapes, level_start_index.to(torch.int32),
                                    sampling_locations, attention_weights, backend="reference")


def test_reference_out_of_range_samples_are_zero_with_zero_gradients():
    tensors = list(_fixture(batch=1, queries=2, heads=1, embed_dims=2, levels=((2, 2),), points=2))
    with torch.no_grad():
        tensors[3].fill_(-1.0)
    output = multi_scale_deformable_attn(*tensors, backend="reference")
    torch.testing.assert_close(output, torch.zeros_like(output))
    output.sum().backward()
    for tensor in (tensors[0], tensors[3], tensors[4]):
        torch.testing.assert_close(tensor.grad, torch.zeros_like(tensor.grad))


def test_float64_value_is_rejected():
    value, spatial_shapes, level_start_index, sampling_locations, attention_weights = _fixture()
    with pytest.raises(TypeError, match="value must be float16, bfloat16 or float32"):
        multi_scale_deformable_attn(value.double(), spatial_shapes, level_start_index,
                                    sampling_locations.double(), attention_weights.double(),
                                    backend="reference")


def test_compat_signature_derives_level_start_index():
    from muspace_amd.ops import multi_scale_deformable_attn_pytorch_compat

    value, shapes, _, loc, attn = _fixture(levels=((1, 2), (2, 3), (1, 1)), points=2)
    out = multi_scale_deformable_attn_pytorch_compat(value, shapes, loc, attn)
    torch.testing.assert_close(out, msda_torch.msda_forward(value, shapes, loc, attn))


@pytest.mark.parametrize("which", ["msda", "softmax"])
def test_early_binning_reservation_returns_when_the_workspace_allocation_fails(
        which, monkeypatch):
    """A failed workspace allocation (out of memory) gives its early-binning
    reservation back at once; otherwise every such failure would shrink the
    device's budget for good, until early binning silently stopped."""
    msda_module = import_module("muspace_amd.ops.multi_scale_deformable_attn")
    softmax_module = import_module("muspace_amd.ops.msda_softmax")
    budget = msda_module.BinningBudget(limit_of=lambda index: 1 << 40)
    monkeypatch.setattr(msda_module, "binning_budget", budget)
    monkeypatch.setattr(msda_module, "_device_index", lambda device: 0)

    class FailingExtension:
        def backward_workspace_bytes(self, value, sampling):
            return 1 << 20

        backward_softmax_workspace_bytes = backward_workspace_bytes

        def backward_workspace(self, value, sampling):
            raise MemoryError("out of device memory")

        backward_softmax_workspace = backward_workspace

    value = torch.zeros(1, 4, 2, 8)
    sampling = torch.zeros(1, 3, 2, 1, 2, 2)
    attn = torch.zeros(1, 3, 2, 1, 2)
    with pytest.raises(MemoryError):
        if which == "msda":
            msda_module._binning_buffers(FailingExtension(), value, sampling, attn)
        else:
            softmax_module._binning_buffers(FailingExtension(), value, sampling, attn)
    assert budget.held(0) == 0
