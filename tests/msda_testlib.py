"""Shared helpers of the MSDA tests: seeded small cases and comparisons."""

from __future__ import annotations

import numpy as np
import torch


def level_starts(levels) -> torch.Tensor:
    sizes = [h * w for h, w in levels]
    return torch.tensor([sum(sizes[:i]) for i in range(len(sizes))], dtype=torch.int64)


def reference_fixture(
    *,
    device="cpu",
    dtype=torch.float32,
    batch=1,
    queries=5,
    heads=2,
    embed_dims=3,
    levels=((2, 2),),
    points=4,
    noncontiguous=False,
    requires_grad=True,
):
    """The reference tests' fixture: same seed, draws and distributions.

    /root/reference/tests/ops/test_multi_scale_deformable_attn.py:16-64
    (value ~ N(0,1), locations ~ U(0,1), weights = softmax(U(0,1)) over points).
    """
    generator = torch.Generator(device="cpu").manual_seed(20260714)
    value_length = sum(h * w for h, w in levels)
    shape = (batch, value_length, heads, embed_dims)
    if noncontiguous:
        value = torch.randn(*shape, 2, generator=generator, dtype=dtype).to(device)[..., 0]
    else:
        value = torch.randn(*shape, generator=generator, dtype=dtype).to(device)
    spatial_shapes = torch.tensor(levels, dtype=torch.int64, device=device)
    level_start_index = level_starts(levels).to(device)
    sampling_shape = (batch, queries, heads, len(levels), points, 2)
    if noncontiguous:
        loc = torch.rand(*sampling_shape, 2, generator=generator, dtype=dtype).to(device)[..., 0]
    else:
        loc = torch.rand(*sampling_shape, generator=generator, dtype=dtype).to(device)
    attention_shape = (batch, queries, heads, len(levels), points)
    if noncontiguous:
        attn = torch.rand(*attention_shape, 2, generator=generator, dtype=dtype).to(device)[..., 0]
    else:
        attn = torch.rand(*attention_shape, generator=generator, dtype=dtype).to(device)
    attn = torch.softmax(attn, dim=-1)
    if requires_grad:
        value.requires_grad_(True)
        loc.requires_grad_(True)
        attn.requires_grad_(True)
    return value, spatial_shapes, level_start_index, loc, attn


def random_case(
    seed: int,
    *,
    batch=2,
    queries=7,
    heads=3,
    channels=5,
    levels=((3, 5), (2, 2), (1, 3)),
    points=3,
    loc_low=-0.1,
    loc_high=1.1,
    dtype=torch.float64,
):
    """Random inputs with some samples outside the image (zero padding)."""
    g = torch.Generator().manual_seed(seed)
    nv = sum(h * w for h, w in levels)
    L = len(levels)
    value = torch.randn(batch, nv, heads, channels, generator=g, dtype=dtype)
    loc = torch.rand(batch, queries, heads, L, points, 2, generator=g, dtype=dtype)
    loc = loc * (loc_high - loc_low) + loc_low
    logits = torch.randn(batch, queries, heads, L * points, generator=g, dtype=dtype)
    attn = torch.softmax(logits, -1).view(batch, queries, heads, L, points)
    grad = torch.randn(batch, queries, heads * channels, generator=g, dtype=dtype)
    shapes = torch.tensor(levels, dtype=torch.int64)
    return value, shapes, level_starts(levels), loc, attn, grad


def max_violation(actual, expected, rtol: float, atol: float) -> float:
    """max(|a-e| - atol - rtol*|e|): <= 0 iff torch.testing.assert_close would pass."""
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    if a.size == 0:
        return -1.0
    return float(np.max(np.abs(a - e) - atol - rtol * np.abs(e)))


def scatter_div_case(
    seed: int,
    *,
    batch=2,
    cams=3,
    max_len=9,
    num_query=20,
    heads=2,
    channels=4,
    levels=((3, 5), (2, 2)),
    points=3,
    lengths=None,
    out_of_range=False,
    dtype=torch.float64,
):
    """Camera-rebatched inputs of the fused scatter-average.

    Returns (value, shapes, starts, loc, attn, indexes, count, slots): value
    ``[batch*cams, nv, M, C]``, geometry ``[batch*cams, max_len, ...]``, one
    index tensor per camera (distinct BEV ids; ``lengths`` fixes how many),
    count ``[batch, num_query]`` = (b + 1) x cameras seeing each query (at
    least 1) and random initial slots.
    Default lengths: max_len for camera 0, 0 for camera 1 (an empty camera),
    random below max_len for the rest. ``out_of_range`` appends ids -1 and
    num_query to the last camera.
    """
    g = torch.Generator().manual_seed(seed)
    rows = batch * cams
    value, shapes, starts, loc, attn, _ = random_case(
        seed, batch=rows, queries=max_len, heads=heads, channels=channels, levels=levels,
        points=points, dtype=dtype)
    if lengths is None:
        lengths = [max_len, 0] + [
            int(torch.randint(1, max_len, (1,), generator=g)) for _ in range(cams - 2)]
    indexes = []
    seen = torch.zeros(num_query, dtype=dtype)
    for cam in range(cams):
        ids = torch.randperm(num_query, generator=g)[: lengths[cam]]
        seen[ids] += 1
        if out_of_range and cam == cams - 1:
            ids = torch.cat([ids, torch.tensor([-1, num_query])])[:max_len]
        indexes.append(ids.to(torch.int64))
    # cameras seeing each query, scaled by b + 1 so that batch entries differ
    count = torch.stack([seen.clamp(min=1) * (b + 1) for b in range(batch)])
    slots = torch.randn(batch, num_query, heads * channels, generator=g, dtype=dtype)
    return value, shapes, starts, loc, attn, indexes, count, slots
