"""The backward entry that allocates nothing (ms_deform_attn_backward_noalloc),
called through the C-ABI, against ms_deform_attn_backward on the same inputs:
two calls in a row, the second smaller, each to the float32 backward
tolerance (1e-4; tile-boundary sums are added atomically, in no fixed order).
The first call has the c2 shape, whose six batch entries do not fit the fixed
scratch together, so it runs in several passes over the batch; the second is
small enough for one pass and must not see anything the first left behind.
A third case stores value, grad_output and the geometry in bfloat16 and has a
batch of five whose last pass holds fewer entries than the others, so the
per-pass offsets are checked at 16-bit element sizes and for a short last pass.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

from conftest import gpu_available
from muspace_amd.runtime.native import DTYPE_BF16, DTYPE_F16, DTYPE_F32
from muspace_amd.workloads import CONFIGS, make_inputs

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not gpu_available(), reason="AMD GPU required"),
]

DEV = "cuda"
SCRATCH = 64 << 20  # MUSPACE_NOALLOC_SCRATCH_BYTES


def _small_inputs():
    g = torch.Generator().manual_seed(11)
    levels = ((16, 24), (8, 12))
    nv = sum(h * w for h, w in levels)
    batch, queries, heads, channels, points = 2, 300, 4, 32, 4
    logits = torch.randn(batch, queries, heads, len(levels) * points, generator=g)
    return {
        "value": torch.randn(batch, nv, heads, channels, generator=g),
        "spatial_shapes": torch.tensor(levels, dtype=torch.int64),
        "level_start_index": torch.tensor([0, 16 * 24], dtype=torch.int64),
        "sampling_locations": torch.rand(batch, queries, heads, len(levels), points, 2,
                                         generator=g) * 1.1 - 0.05,
        "attention_weights": torch.softmax(logits, -1).view(batch, queries, heads, len(levels),
                                                            points),
        "grad_output": torch.randn(batch, queries, heads * channels, generator=g),
    }


def _device(t):
    return {k: v.to(DEV).contiguous() for k, v in t.items()}


_CODES = {torch.float32: DTYPE_F32, torch.float16: DTYPE_F16, torch.bfloat16: DTYPE_BF16}


def _raw_noalloc(lib, t, grads):
    """ms_deform_attn_backward_noalloc through the bare C entry point."""
    value, loc = t["value"], t["sampling_locations"]
    batch, spatial, heads, channels = value.shape
    _, queries, _, levels, points, _ = loc.shape
    fn = lib.raw("ms_deform_attn_backward_noalloc")
    rc = fn(value.data_ptr(), _CODES[value.dtype], t["spatial_shapes"].data_ptr(),
            t["level_start_index"].data_ptr(), loc.data_ptr(),
            t["attention_weights"].data_ptr(), _CODES[loc.dtype], t["grad_output"].data_ptr(),
            grads[0].data_ptr(), grads[1].data_ptr(), grads[2].data_ptr(),
            batch, spatial, heads, channels, levels, queries, points, 64,
            torch.cuda.current_stream().cuda_stream)
    assert rc == 0, lib.last_error()


def _poisoned(t):
    return tuple(torch.full(t[k].shape, float("nan"), device=DEV, dtype=torch.float32)
                 for k in ("value", "sampling_locations", "attention_weights"))


def _check(lib, t):
    ref = _poisoned(t)
    lib.ms_deform_attn_backward(t["value"], t["spatial_shapes"], t["level_start_index"],
                                t["sampling_locations"], t["attention_weights"],
                                t["grad_output"], *ref, 64)
    got = _poisoned(t)
    _raw_noalloc(lib, t, got)
    torch.cuda.synchronize()
    for name, a, b in zip(("grad_value", "grad_sampling_locations", "grad_attention_weights"),
                          got, ref):
        assert torch.isfinite(a).all(), f"{name}: elements left unwritten"
        torch.testing.assert_close(a, b, rtol=1e-4, atol=1e-4, msg=name)


def test_noalloc_backward_matches_the_allocating_entry_twice(native_lib):
    cfg = CONFIGS["c2"]
    size = native_lib.raw("ms_deform_attn_backward_workspace_size")
    full = size(0, cfg.batch, cfg.spatial_size, cfg.heads, cfg.channels, cfg.num_levels,
                cfg.queries, cfg.points)
    one = size(0, 1, cfg.spatial_size, cfg.heads, cfg.channels, cfg.num_levels, cfg.queries,
               cfg.points)
    assert one <= SCRATCH < full  # the first call runs in several passes
    print(f"[no-alloc] c2: {full} bytes of scratch for the batch, {one} per entry", flush=True)
    _check(native_lib, _device(make_inputs(cfg)))
    small = _device(_small_inputs())
    print("[no-alloc] second, smaller call", flush=True)
    _check(native_lib, small)


def test_noalloc_backward_16bit_storage_with_a_short_last_pass(native_lib):
    """bfloat16 value, grad_output, locations and weights; five batch entries
    of 4000 queries at the c2 levels: the passes hold as many entries as fit
    the scratch (two or more), and the last pass holds fewer."""
    cfg = CONFIGS["c2"]
    batch, queries = 5, 4000
    size = native_lib.raw("ms_deform_attn_backward_workspace_size")
    fit = max(n for n in range(1, batch + 1)
              if size(DTYPE_BF16, n, cfg.spatial_size, cfg.heads, cfg.channels, cfg.num_levels,
                       queries, cfg.points) <= SCRATCH)
    assert 2 <= fit < batch and batch % fit != 0, fit
    g = torch.Generator().manual_seed(5)
    levels = cfg.levels
    logits = torch.randn(batch, queries, cfg.heads, cfg.num_levels * cfg.points, generator=g)
    starts = [0]
    for h, w in levels[:-1]:
        starts.append(starts[-1] + h * w)
    t = {
        "value": torch.randn(batch, cfg.spatial_size, cfg.heads, cfg.channels, generator=g),
        "spatial_shapes": torch.tensor(levels, dtype=torch.int64),
        "level_start_index": torch.tensor(starts, dtype=torch.int64),
        "sampling_locations": torch.rand(batch, queries, cfg.heads, cfg.num_levels, cfg.points,
                                         2, generator=g),
        "attention_weights": torch.softmax(logits, -1).view(batch, queries, cfg.heads,
                                                            cfg.num_levels, cfg.points),
        "grad_output": torch.randn(batch, queries, cfg.heads * cfg.channels, generator=g),
    }
    t = {k: (v.to(torch.bfloat16) if v.is_floating_point() else v) for k, v in t.items()}
    print(f"[no-alloc] bf16: batch {batch} x {queries} queries, passes of up to {fit}", flush=True)
    _check(native_lib, _device(t))
