"""Every tensor of an MSDA call is checked before anything is launched.

The reference checks device, dtype and contiguity of all of its tensors before
its first launch (/root/reference/csrc/ms_deformable_attn/ms_deform_attn_musa.mu:514-522,
/root/reference/csrc/ffi/tensor_utils.hpp:13-38), and under ``backend="auto"`` a
failed check falls back to the PyTorch path
(/root/reference/mu_space/ops/multi_scale_deformable_attn.py:311-338; its test
with a fake native module: tests/ops/test_multi_scale_deformable_attn.py:204-229).

Here the autograd function may start the backward's binning before the
forward's launch, so the checks must come before that too. These CPU tests use
the real argument checks of ``NativeLibrary`` on CPU tensors that stand in for
device tensors (the device predicate is patched; a tensor marked ``_host``
plays a host tensor next to device tensors) and record every launch instead
of running it.
"""

import warnings
from importlib import import_module

import pytest
import torch

from muspace_amd import clear_dispatch_report, get_last_dispatch_report
from muspace_amd.runtime import native

msda_module = import_module("muspace_amd.ops.multi_scale_deformable_attn")
softmax_module = import_module("muspace_amd.ops.msda_softmax")

LEVELS = ((6, 8), (3, 4))
BATCH, QUERIES, HEADS, CHANNELS, POINTS = 2, 10, 2, 4, 3


def _inputs(requires_grad=True):
    g = torch.Generator().manual_seed(7)
    nv = sum(h * w for h, w in LEVELS)
    value = torch.randn(BATCH, nv, HEADS, CHANNELS, generator=g)
    loc = torch.rand(BATCH, QUERIES, HEADS, len(LEVELS), POINTS, 2, generator=g)
    attn = torch.rand(BATCH, QUERIES, HEADS, len(LEVELS), POINTS, generator=g)
    shapes = torch.tensor(LEVELS, dtype=torch.int64)
    starts = torch.tensor([0, 48], dtype=torch.int64)
    for t in (value, loc, attn):
        t.requires_grad_(requires_grad)
    return value, shapes, starts, loc, attn


def _host(tensor):
    tensor._host = True
    return tensor


class _RecordingExtension:
    """The library's own argument checks; every launch is recorded instead."""

    def __init__(self, lib):
        self.lib = lib
        self.calls = []

    def check_forward(self, *args):
        self.calls.append("check_forward")
        return self.lib.check_forward(*args)

    def backward_workspace(self, *args):
        self.calls.append("backward_workspace")
        return torch.empty(1 << 12, dtype=torch.uint8)

    backward_softmax_workspace = backward_workspace

    def __getattr__(self, name):
        def launch(*args, **kwargs):
            self.calls.append(name)
            for arg in args:  # the forward's output is the only [bs, nq, M*C] tensor
                if isinstance(arg, torch.Tensor) and arg.shape == (BATCH, QUERIES,
                                                                   HEADS * CHANNELS):
                    arg.zero_()

        return launch


@pytest.fixture
def recording(monkeypatch, native_lib):
    """Native routing for CPU tensors, with launches recorded."""
    monkeypatch.setattr(native, "_is_device_tensor", lambda t: not getattr(t, "_host", False))
    ext = _RecordingExtension(native_lib)
    for module in (msda_module, softmax_module):
        monkeypatch.setattr(module, "_native_extension", lambda: ext)
        monkeypatch.setattr(module, "_requires_native_backend", lambda *args: True,
                            raising=False)
        monkeypatch.setattr(
            module, "_explain_dispatch",
            lambda value, *, backend, native_available: msda_module.DispatchDecision(
                "hip", value.device.type, "simulated ROCm tensor selects native HIP backend"),
        )

    def buffers(ext_, value, loc, attn):  # host stand-ins for the device buffers
        ext_.calls.append("backward_workspace")
        return (torch.empty(1 << 12, dtype=torch.uint8),
                (torch.empty(value.shape), torch.empty(loc.shape), torch.empty(attn.shape)))

    monkeypatch.setattr(msda_module, "_binning_buffers", buffers)
    monkeypatch.setattr(softmax_module, "_binning_buffers", buffers)
    monkeypatch.setenv("MUSPACE_EARLY_BINNING", "1")
    return ext


def test_valid_inputs_are_checked_then_binned_then_run(recording):
    clear_dispatch_report()
    out = msda_module.multi_scale_deformable_attn(*_inputs(), backend="auto")
    assert out.shape == (BATCH, QUERIES, HEADS * CHANNELS)
    assert recording.calls == ["check_forward", "backward_workspace",
                               "ms_deform_attn_forward_bin"]
    assert get_last_dispatch_report().selected_backend == "hip"


def test_softmax_operator_is_checked_then_binned_then_run(recording):
    """The softmax operator in training: one forward call that also bins."""
    clear_dispatch_report()
    out = softmax_module.multi_scale_deformable_attn_softmax(*_inputs(), backend="auto")
    assert out.shape == (BATCH, QUERIES, HEADS * CHANNELS)
    assert recording.calls == ["check_forward", "backward_workspace",
                               "ms_deform_attn_forward_softmax_bin"]


def _bad_host_spatial_shapes(t):
    t[1] = _host(t[1].clone())


def _bad_host_attention(t):
    t[4] = _host(t[4].detach().clone().requires_grad_())


def _bad_heads_in_locations(t):
    t[3] = t[3].detach()[:, :, :1].clone().requires_grad_()


def _bad_points_in_attention(t):
    t[4] = t[4].detach()[..., :2].clone().requires_grad_()


BAD = {
    "host spatial_shapes": (_bad_host_spatial_shapes, "spatial_shapes must be a ROCm device"),
    "host attention_weights": (_bad_host_attention, "attention_weights must be a ROCm device"),
    "sampling_locations with the wrong M": (_bad_heads_in_locations,
                                            "sampling_locations must have shape"),
    "attention_weights with the wrong P": (_bad_points_in_attention,
                                           "attention_weights must have shape"),
}


@pytest.mark.parametrize("case", sorted(BAD))
def test_bad_input_raises_before_any_launch(recording, case):
    spoil, message = BAD[case]
    tensors = list(_inputs())
    spoil(tensors)
    with pytest.raises(RuntimeError, match=message):
        msda_module.multi_scale_deformable_attn(*tensors, backend="hip")
    assert recording.calls == ["check_forward"]
    assert get_last_dispatch_report().selected_backend == "error"


@pytest.mark.parametrize("case", sorted(BAD))
def test_bad_input_under_auto_is_a_recorded_fallback(recording, case):
    spoil, message = BAD[case]
    tensors = list(_inputs())
    spoil(tensors)
    clear_dispatch_report()
    with warnings.catch_warnings():
        warnings.simplefilter("ignore", RuntimeWarning)
        try:
            msda_module.multi_scale_deformable_attn(*tensors, backend="auto")
        except RuntimeError:
            pass  # the reference path rejects mis-shaped inputs in its own way
    assert recording.calls == ["check_forward"]
    report = get_last_dispatch_report()
    assert report.native_fallback is True
    assert report.selected_backend == "reference"
    assert message.split(" must")[0] in report.fallback_reason


@pytest.mark.parametrize("case", sorted(BAD))
def test_softmax_operator_checks_before_binning(recording, case):
    spoil, message = BAD[case]
    tensors = list(_inputs())
    spoil(tensors)
    with pytest.raises(RuntimeError, match=message):
        softmax_module.multi_scale_deformable_attn_softmax(*tensors, backend="hip")
    assert recording.calls == ["check_forward"]


def _grads(value, loc, attn):
    return (torch.empty(value.shape), torch.empty(loc.shape), torch.empty(attn.shape))


@pytest.fixture
def raw_launches(monkeypatch, native_lib):
    """Every C entry point that launches is replaced by a recorder."""
    monkeypatch.setattr(native, "_is_device_tensor", lambda t: not getattr(t, "_host", False))
    launched = []
    for name in list(native_lib._raw):
        if name.startswith("ms_deform_attn_") and not name.endswith("_workspace_size"):
            monkeypatch.setitem(native_lib._raw, name,
                                lambda *args, _n=name: launched.append(_n) or 0)
    return launched


@pytest.mark.parametrize("part", ["ms_deform_attn_backward_bin",
                                  "ms_deform_attn_backward_softmax_bin"])
@pytest.mark.parametrize("case", sorted(BAD))
def test_binning_entry_checks_its_own_arguments(native_lib, raw_launches, part, case):
    spoil, message = BAD[case]
    tensors = [t.detach() if t.dtype.is_floating_point else t for t in _inputs(False)]
    spoil(tensors)
    value, shapes, starts, loc, attn = tensors
    workspace = torch.empty(1 << 20, dtype=torch.uint8)
    with pytest.raises(RuntimeError, match=message):
        getattr(native_lib, part)(value, shapes, starts, loc, attn, *_grads(value, loc, attn),
                                  64, workspace, stream=object())
    assert raw_launches == []


@pytest.mark.parametrize("entry", ["ms_deform_attn_forward_bin",
                                   "ms_deform_attn_forward_softmax_bin"])
@pytest.mark.parametrize("case", sorted(BAD))
def test_fused_forward_binning_entry_checks_its_own_arguments(native_lib, raw_launches, entry,
                                                               case):
    spoil, message = BAD[case]
    tensors = [t.detach() if t.dtype.is_floating_point else t for t in _inputs(False)]
    spoil(tensors)
    value, shapes, starts, loc, attn = tensors
    out = torch.empty(BATCH, QUERIES, HEADS * CHANNELS)
    workspace = torch.empty(1 << 20, dtype=torch.uint8)
    with pytest.raises(RuntimeError, match=message):
        getattr(native_lib, entry)(value, shapes, starts, loc, attn, out,
                                   *_grads(value, loc, attn), 64, workspace)
    assert raw_launches == []


def test_rest_rejects_a_workspace_smaller_than_the_shapes_need(native_lib, raw_launches):
    value, shapes, starts, loc, attn = (t.detach() for t in _inputs(False))
    # a shape the tile path covers (C = 32), so the workspace is not empty
    value = torch.randn(value.shape[0], value.shape[1], value.shape[2], 32)
    grad = torch.randn(BATCH, QUERIES, HEADS * 32)
    need = native_lib.raw("ms_deform_attn_backward_workspace_size")(
        0, BATCH, value.shape[1], HEADS, 32, len(LEVELS), QUERIES, POINTS)
    assert need > 1
    small = torch.empty(need - 1, dtype=torch.uint8)
    with pytest.raises(RuntimeError, match="workspace holds"):
        native_lib.ms_deform_attn_backward_rest(value, shapes, starts, loc, attn, grad,
                                                *_grads(value, loc, attn), 64, small)
    assert raw_launches == []


def test_gradient_buffer_on_another_device_is_rejected(native_lib, raw_launches):
    value, shapes, starts, loc, attn = (t.detach() for t in _inputs(False))
    gv, gl, ga = _grads(value, loc, attn)
    gl = gl.to("meta")  # a device other than the value's
    with pytest.raises(RuntimeError, match="grad_sampling_locations is on meta"):
        native_lib.check_backward(value, shapes, starts, loc, attn, None, gv, gl, ga)


# ------------------------------------------------- early-binning budget ---


def test_binning_budget_reserves_up_to_its_limit_and_releases():
    budget = msda_module.BinningBudget(limit_of=lambda index: 100)
    assert budget.try_reserve(0, 60)
    assert not budget.try_reserve(0, 50)  # 110 > 100: no early binning
    assert budget.try_reserve(1, 90)  # per device
    budget.release(0, 60)
    assert budget.try_reserve(0, 100)
    assert budget.held(0) == 100 and budget.held(1) == 90


def test_reservations_over_the_budget_are_refused(monkeypatch):
    """A forward whose buffers would exceed the budget gets no reservation
    (it then does not bin early); releasing one makes room again."""
    budget = msda_module.BinningBudget(limit_of=lambda index: 1 << 20)
    monkeypatch.setattr(msda_module, "binning_budget", budget)
    monkeypatch.setattr(msda_module, "_device_index", lambda device: 0)
    value, shapes, starts, loc, attn = _inputs()
    need = 4 * (value.numel() + loc.numel() + attn.numel()) + 4096
    assert budget.try_reserve(0, (1 << 20) - need + 1)
    assert msda_module._reserve_early_buffers(4096, value, loc, attn) is None
    budget.release(0, (1 << 20) - need + 1)
    release = msda_module._reserve_early_buffers(4096, value, loc, attn)
    assert release is not None and budget.held(0) == need
    release()
    assert budget.held(0) == 0
