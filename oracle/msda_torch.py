"""TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Op-for-op restatement, on the CPU, of the reference PyTorch path
``multi_scale_deformable_attn_pytorch``
(/root/reference/mu_space/ops/multi_scale_deformable_attn.py:26-58). Each line
below names the reference line it follows; the operation order is kept so that
float32 results equal the reference path's bit for bit on the same torch.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F


def msda_forward(
    value: torch.Tensor,
    value_spatial_shapes: torch.Tensor,
    sampling_locations: torch.Tensor,
    attention_weights: torch.Tensor,
) -> torch.Tensor:
    """MSDA output ``[bs, nq, M*C]`` (reference ops:26-58)."""
    bs, _, heads, channels = value.shape  # :32
    _, queries, _, levels, points, _ = sampling_locations.shape  # :33
    shapes = [(int(h), int(w)) for h, w in value_spatial_shapes.tolist()]
    per_level_values = value.split([h * w for h, w in shapes], dim=1)  # :34
    grids = 2 * sampling_locations - 1  # :35
    sampled = []
    for level, (h, w) in enumerate(shapes):  # :37
        image = (
            per_level_values[level].flatten(2).transpose(1, 2).reshape(bs * heads, channels, h, w)
        )  # :38-40
        grid = grids[:, :, :, level].transpose(1, 2).flatten(0, 1)  # :41
        sampled.append(
            F.grid_sample(
                image, grid, mode="bilinear", padding_mode="zeros", align_corners=False
            )
        )  # :42-49
    weights = attention_weights.transpose(1, 2).reshape(
        bs * heads, 1, queries, levels * points
    )  # :50-52
    output = (
        (torch.stack(sampled, dim=-2).flatten(-2) * weights)
        .sum(-1)
        .view(bs, heads * channels, queries)
    )  # :53-57
    return output.transpose(1, 2).contiguous()  # :58


def msda_forward_backward(
    value: torch.Tensor,
    value_spatial_shapes: torch.Tensor,
    sampling_locations: torch.Tensor,
    attention_weights: torch.Tensor,
    grad_output: torch.Tensor,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """(output, grad_value, grad_sampling_locations, grad_attention_weights).

    Gradients are those autograd gives the reference path for the upstream
    gradient ``grad_output`` (what the reference's device tests compare the
    native backward against, tests/ops/test_multi_scale_deformable_attn.py:286-306).
    """
    v = value.detach().clone().requires_grad_(True)
    loc = sampling_locations.detach().clone().requires_grad_(True)
    attn = attention_weights.detach().clone().requires_grad_(True)
    out = msda_forward(v, value_spatial_shapes, loc, attn)
    out.backward(grad_output)
    return out.detach(), v.grad, loc.grad, attn.grad
