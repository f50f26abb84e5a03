"""Fused spatial cross-attention scatter-average on the GPU, against the oracle.

The op (muspace_amd.ops.scatter_div) adds each camera's MSDA rows into the BEV
slots as ``slots[b, index[r]] += out / count[b, index[r]]``; the reference
sketches it as ms_deformable_im2col_scatter_div_* (/root/reference/csrc/
ms_deformable_attn/ms_deform_attn_musa_kernel.muh:419-486, forward only).
Expected values come from oracle/msda_scatter_div.py (forward) and its
autograd (backward). Tolerances: fp32 forward 1e-5 and gradients 1e-4;
16-bit value 2e-2 against the fp32 oracle on the same (rounded) inputs.
"""

import pytest
import torch

from conftest import gpu_available
from msda_testlib import scatter_div_case
from muspace_amd import multi_scale_deformable_attn, multi_scale_deformable_attn_scatter_div
from muspace_amd import workloads
from oracle import msda_scatter_div
from oracle.msda_torch import msda_forward

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not gpu_available(), reason="AMD GPU required"),
]

DEV = "cuda"


def _device_case(case, value_dtype, geometry_dtype):
    value, shapes, starts, loc, attn, indexes, count, slots = case
    return (value.to(value_dtype).to(DEV), shapes.to(DEV), starts.to(DEV),
            loc.to(geometry_dtype).to(DEV), attn.to(geometry_dtype).to(DEV),
            [i.to(DEV) for i in indexes], count.to(geometry_dtype).to(DEV),
            slots.to(value_dtype).to(DEV))


def _oracle_inputs(device_case):
    """fp32 CPU copies of exactly what the device received."""
    value, shapes, _, loc, attn, indexes, count, slots = device_case
    f = lambda t: t.detach().float().cpu()  # noqa: E731
    return (f(value), shapes.cpu(), f(loc), f(attn), [i.cpu() for i in indexes], f(count),
            f(slots))


@pytest.mark.parametrize(
    "value_dtype,geometry_dtype,channels",
    [
        (torch.float32, torch.float32, 32),
        (torch.float32, torch.float32, 16),
        (torch.float32, torch.float32, 64),
        (torch.float32, torch.float32, 3),
        (torch.bfloat16, torch.bfloat16, 32),
        (torch.bfloat16, torch.float32, 32),
        (torch.float16, torch.float16, 32),
        (torch.float16, torch.float32, 8),
    ],
)
def test_forward_and_backward_match_the_oracle(value_dtype, geometry_dtype, channels):
    case = scatter_div_case(11, batch=2, cams=4, max_len=13, num_query=40, heads=3,
                            channels=channels, levels=((5, 7), (3, 4), (2, 2)), points=4,
                            out_of_range=True)
    dev = _device_case(case, value_dtype, geometry_dtype)
    value, shapes, starts, loc, attn, indexes, count, slots = dev
    for t in (value, loc, attn, slots):
        t.requires_grad_(True)
    ref = [t.clone().requires_grad_(t.is_floating_point()) if i != 4 else t
           for i, t in enumerate(_oracle_inputs(dev))]
    # slots is a leaf that requires grad: the op adds in place into a copy of it
    out = multi_scale_deformable_attn_scatter_div(value, shapes, starts, loc, attn, indexes,
                                                  count, slots.clone())
    expected = msda_scatter_div.scatter_div(ref[0], ref[1], ref[2], ref[3], ref[4], ref[5],
                                            ref[6])
    fp32 = value_dtype == torch.float32
    tol_f, tol_b = (1e-5, 1e-4) if fp32 else (2e-2, 2e-2)
    assert out.dtype == value_dtype
    torch.testing.assert_close(out.detach().float().cpu(), expected.detach(), rtol=tol_f,
                               atol=tol_f)
    g = torch.randn(out.shape, generator=torch.Generator().manual_seed(3))
    (out.float() * g.to(DEV)).sum().backward()
    (expected * g).sum().backward()
    for native, cpu in ((value, ref[0]), (loc, ref[2]), (attn, ref[3]), (slots, ref[6])):
        assert native.grad.dtype == native.dtype
        torch.testing.assert_close(native.grad.float().cpu(), cpu.grad, rtol=tol_b, atol=tol_b)


def test_cameras_accumulate_in_place_and_repeat_calls_add_again():
    case = scatter_div_case(12, batch=1, cams=3, max_len=10, num_query=25, heads=8,
                            channels=32, levels=((6, 5), (3, 3)), points=4)
    value, shapes, starts, loc, attn, indexes, count, slots = _device_case(
        case, torch.float32, torch.float32)
    start = slots.clone()
    result = multi_scale_deformable_attn_scatter_div(value, shapes, starts, loc, attn, indexes,
                                                     count, slots)
    assert result is slots
    once = result.clone()
    multi_scale_deformable_attn_scatter_div(value, shapes, starts, loc, attn, indexes, count,
                                            slots)
    torch.testing.assert_close(slots - once, once - start, rtol=1e-5, atol=1e-5)
    fresh = multi_scale_deformable_attn_scatter_div(value, shapes, starts, loc, attn, indexes,
                                                    count)
    torch.testing.assert_close(fresh, once - start, rtol=1e-5, atol=1e-5)


def test_sca_c2_shape_matches_the_unfused_composition():
    """Full size: one BEVFormer sample, six cameras, c2's levels and points,
    a 200 x 200 BEV grid. The fused op equals the dense operator followed by
    BEVFormer's per-camera adds and the division (size-independent property),
    forward and backward."""
    inputs = workloads.make_sca_inputs(device=DEV)
    value = inputs["value"].requires_grad_(True)
    loc = inputs["sampling_locations"].requires_grad_(True)
    attn = inputs["attention_weights"].requires_grad_(True)
    shapes, starts = inputs["spatial_shapes"], inputs["level_start_index"]
    indexes, count = inputs["indexes"], inputs["count"]
    fused = multi_scale_deformable_attn_scatter_div(value, shapes, starts, loc, attn, indexes,
                                                    count)
    g = torch.randn(fused.shape, generator=torch.Generator().manual_seed(7)).to(DEV)
    (fused * g).sum().backward()
    grads = [t.grad.clone() for t in (value, loc, attn)]
    for t in (value, loc, attn):
        t.grad = None
    dense = multi_scale_deformable_attn(value, shapes, starts, loc, attn)
    cams = len(indexes)
    dense = dense.view(1, cams, dense.shape[1], dense.shape[2])
    slots = torch.zeros_like(fused)
    for cam, index in enumerate(indexes):
        slots[:, index] = slots[:, index] + dense[:, cam, : len(index)] / count[:, index, None]
    (slots * g).sum().backward()
    torch.testing.assert_close(fused.detach(), slots.detach(), rtol=1e-5, atol=1e-5)
    for a, e in zip(grads, (value.grad, loc.grad, attn.grad)):
        torch.testing.assert_close(a, e, rtol=1e-4, atol=1e-4)


def test_rejects_cpu_tensors_and_bad_indexes():
    case = scatter_div_case(13, dtype=torch.float32)
    value, shapes, starts, loc, attn, indexes, count, slots = case
    with pytest.raises(RuntimeError, match="ROCm tensors only"):
        multi_scale_deformable_attn_scatter_div(value, shapes, starts, loc, attn, indexes, count)
    value, shapes, starts, loc, attn, indexes, count, slots = _device_case(
        case, torch.float32, torch.float32)
    too_long = [torch.arange(loc.shape[1] + 1, device=DEV)] + indexes[1:]
    with pytest.raises(RuntimeError, match="more than max_len"):
        multi_scale_deformable_attn_scatter_div(value, shapes, starts, loc, attn, too_long, count)
    with pytest.raises(TypeError, match="int64"):
        multi_scale_deformable_attn_scatter_div(value, shapes, starts, loc, attn,
                                                [i.int() for i in indexes], count)
    with pytest.raises(RuntimeError, match="num_cams"):
        multi_scale_deformable_attn_scatter_div(value, shapes, starts, loc, attn,
                                                indexes + indexes[:1], count)


@pytest.mark.parametrize("value_dtype", [torch.float32, torch.bfloat16])
def test_per_camera_entry_point_matches_the_all_camera_call(value_dtype):
    """The reference's interface (one ordered launch per camera) against the
    all-camera call the operator uses."""
    from muspace_amd.runtime.native import load_native_module

    lib = load_native_module()
    case = scatter_div_case(14, batch=2, cams=5, max_len=11, num_query=30, heads=4,
                            channels=32, levels=((7, 6), (4, 3)), points=4, out_of_range=True)
    value, shapes, starts, loc, attn, indexes, count, slots = _device_case(
        case, value_dtype, value_dtype)
    per_camera = slots.clone()
    for cam, index in enumerate(indexes):
        lib.ms_deform_attn_forward_scatter_div(value, shapes, starts, loc, attn, index, count,
                                               per_camera, len(indexes), cam)
    together = slots.clone()
    lib.ms_deform_attn_forward_scatter_div_cams(value, shapes, starts, loc, attn,
                                                torch.cat(indexes), [len(i) for i in indexes],
                                                count, together)
    tol = 1e-5 if value_dtype == torch.float32 else 0.0
    torch.testing.assert_close(together, per_camera, rtol=tol, atol=tol)
    expected = msda_scatter_div.scatter_div(*_oracle_inputs(
        (value, shapes, starts, loc, attn, indexes, count, slots)))
    tol = 1e-5 if value_dtype == torch.float32 else 2e-2
    torch.testing.assert_close(together.float().cpu(), expected, rtol=tol, atol=tol)


def test_more_cameras_than_one_launch_holds():
    """17 cameras: the all-camera call splits them over two launches."""
    case = scatter_div_case(15, batch=1, cams=17, max_len=6, num_query=50, heads=2,
                            channels=16, levels=((5, 4),), points=2, dtype=torch.float32)
    dev = _device_case(case, torch.float32, torch.float32)
    value, shapes, starts, loc, attn, indexes, count, slots = dev
    for t in (value, loc, attn):
        t.requires_grad_(True)
    ref = [t.clone().requires_grad_(t.is_floating_point()) if i != 4 else t
           for i, t in enumerate(_oracle_inputs(dev))]
    out = multi_scale_deformable_attn_scatter_div(value, shapes, starts, loc, attn, indexes,
                                                  count, slots.clone())
    expected = msda_scatter_div.scatter_div(*ref)
    torch.testing.assert_close(out.detach().cpu(), expected.detach(), rtol=1e-5, atol=1e-5)
    g = torch.randn(out.shape, generator=torch.Generator().manual_seed(4))
    (out * g.to(DEV)).sum().backward()
    (expected * g).sum().backward()
    for native, cpu in ((value, ref[0]), (loc, ref[2]), (attn, ref[3])):
        torch.testing.assert_close(native.grad.cpu(), cpu.grad, rtol=1e-4, atol=1e-4)


_DTYPES = [(torch.float32, torch.float32), (torch.bfloat16, torch.float32),
           (torch.bfloat16, torch.bfloat16), (torch.float16, torch.float32),
           (torch.float16, torch.float16)]


def _oracle_grads(ref, g, value_dtype):
    """Oracle gradients for the grad rows the op hands the MSDA backward.

    The op's backward gathers ``grad_slots[b, bev] * (1 / count[b, bev])`` into
    per-camera rows stored in the value dtype (the rounding a 16-bit unfused
    composition makes too), so the oracle's MSDA autograd is fed exactly those
    rows; grad_slots passes through unchanged.
    """
    value, shapes, loc, attn, indexes, count, slots = ref
    gq, inv = g.to(value_dtype).float(), 1.0 / count.detach()
    rows, max_len = loc.shape[0], loc.shape[1]
    cams, num_query = len(indexes), gq.shape[1]
    grad_rows = torch.zeros(rows, max_len, gq.shape[-1])
    for cam, index in enumerate(indexes):
        keep = torch.nonzero((index >= 0) & (index < num_query)).flatten()
        bev = index[keep]
        for b in range(rows // cams):
            grad_rows[b * cams + cam, keep] = (gq[b, bev] * inv[b, bev, None]).to(
                value_dtype).float()
    (msda_forward(value, shapes, loc, attn) * grad_rows).sum().backward()
    return value.grad, loc.grad, attn.grad, gq


@pytest.mark.parametrize("seed", range(20))
def test_random_shapes_match_the_oracle(seed):
    """Seeded random cameras, lengths, BEV sizes, levels, heads, points and
    channels over every dtype combination; odd seeds turn 10% of the sampling
    locations into NaN, which drops those samples (the oracle is given an
    out-of-range location there instead)."""
    r = torch.Generator().manual_seed(9000 + seed)
    pick = lambda lo, hi: int(torch.randint(lo, hi + 1, (1,), generator=r))  # noqa: E731
    channels = (8, 16, 32, 64, 3, 32)[pick(0, 5)]
    levels = tuple((pick(1, 20), pick(1, 20)) for _ in range(pick(1, 4)))
    num_query = pick(4, 120)
    case = scatter_div_case(seed, batch=pick(1, 3), cams=pick(2, 7),
                            max_len=pick(2, num_query), num_query=num_query,
                            heads=pick(1, 8), channels=channels, levels=levels,
                            points=pick(1, 8), out_of_range=seed % 3 == 0)
    value_dtype, geometry_dtype = _DTYPES[seed % len(_DTYPES)]
    if seed % 2:
        loc = case[3].clone()
        drop = torch.rand(loc.shape[:-1], generator=r) < 0.1
        loc[..., 1] = torch.where(drop, torch.nan, loc[..., 1])
        case = case[:3] + (loc,) + case[4:]
    dev = _device_case(case, value_dtype, geometry_dtype)
    value, shapes, starts, loc, attn, indexes, count, slots = dev
    for t in (value, loc, attn, slots):
        t.requires_grad_(True)
    ref = list(_oracle_inputs(dev))
    ref[2] = torch.nan_to_num(ref[2], nan=-10.0)
    ref = [t.clone().requires_grad_(t.is_floating_point()) if i != 4 else t
           for i, t in enumerate(ref)]
    out = multi_scale_deformable_attn_scatter_div(value, shapes, starts, loc, attn, indexes,
                                                  count, slots.clone())
    expected = msda_scatter_div.scatter_div(*[t.detach() if i != 4 else t
                                              for i, t in enumerate(ref)])
    fp32 = value_dtype == torch.float32
    tol_f, tol_b = (1e-5, 1e-4) if fp32 else (2e-2, 2e-2)
    torch.testing.assert_close(out.detach().float().cpu(), expected, rtol=tol_f, atol=tol_f)
    g = torch.randn(out.shape, generator=torch.Generator().manual_seed(seed))
    (out.float() * g.to(DEV)).sum().backward()
    for name, native, cpu in zip(("value", "loc", "attn", "slots"), (value, loc, attn, slots),
                                 _oracle_grads(ref, g, value_dtype)):
        assert native.grad.dtype == native.dtype
        torch.testing.assert_close(native.grad.float().cpu(), cpu, rtol=tol_b, atol=tol_b,
                                   msg=lambda m, name=name: f"{name}: {m}")
