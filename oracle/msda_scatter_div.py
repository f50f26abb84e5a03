"""TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

CPU restatement of BEVFormer's spatial cross-attention scatter-average fused
into MSDA, as the reference's unexported kernel
``ms_deformable_im2col_scatter_div_gpu_kernel_channels32_runtime``
(/root/reference/csrc/ms_deformable_attn/ms_deform_attn_musa_kernel.muh:419-486)
and its per-camera host loop (ms_deform_attn_musa.mu:455-505) compute it:

  * value and geometry row ``b*num_cams + cam`` is camera ``cam`` of batch
    entry ``b`` (``sample_id = b_col * num_cams + cam_id``, .muh:439);
  * row ``r < valid_len`` of a camera adds to BEV query ``index[r]``
    (``bev_query = data_index[q_col]``, .muh:438);
  * the MSDA sum of the row is scaled by ``inv_count = 1 / count[b, bev]``
    and then added to the slot (.muh:483-484);
  * cameras are added one after another (one launch each, .mu:455-505).

The MSDA sum itself is the grid_sample restatement of msda_torch.py. Indices
outside ``[0, num_query)`` add nothing (the operator's documented rule; the
reference would write out of bounds). Built from differentiable torch ops, so
autograd of this function is the backward oracle.

``scatter_div_direct`` is an independent float64 formulation for pinning:
explicit loops over (b, cam, r) on msda_direct's closed-form sums, with each
slot's camera contributions summed first and divided once.
"""

from __future__ import annotations

from typing import Sequence

import numpy as np
import torch

from . import msda_direct
from .msda_torch import msda_forward


def scatter_div(
    value: torch.Tensor,
    spatial_shapes: torch.Tensor,
    sampling_locations: torch.Tensor,
    attention_weights: torch.Tensor,
    indexes: Sequence[torch.Tensor],
    count: torch.Tensor,
    slots: torch.Tensor,
) -> torch.Tensor:
    """slots after every camera's ``slots[b, index[r]] += out[b, cam, r] / count[b, index[r]]``."""
    rows = value.shape[0]
    num_cams = len(indexes)
    batch = rows // num_cams
    num_query = slots.shape[1]
    out = msda_forward(value, spatial_shapes, sampling_locations, attention_weights)
    out = out.view(batch, num_cams, out.shape[1], out.shape[2])  # row b*num_cams + cam
    inv = 1.0 / count  # inv_count, .muh:483
    result = slots.clone()
    for cam, index in enumerate(indexes):  # one launch per camera, in order
        rows_kept = torch.nonzero((index >= 0) & (index < num_query)).flatten()
        bev = index[rows_kept]
        result[:, bev] = result[:, bev] + out[:, cam, rows_kept] * inv[:, bev].unsqueeze(-1)
    return result


def scatter_div_direct(value, spatial_shapes, sampling_locations, attention_weights, indexes,
                       count, slots) -> np.ndarray:
    """Float64 loops: slot + (sum over cameras of the MSDA row) / count."""
    value = np.asarray(value, dtype=np.float64)
    loc = np.asarray(sampling_locations, dtype=np.float64)
    attn = np.asarray(attention_weights, dtype=np.float64)
    count = np.asarray(count, dtype=np.float64)
    result = np.array(slots, dtype=np.float64)
    num_cams = len(indexes)
    batch = value.shape[0] // num_cams
    num_query = result.shape[1]
    total = np.zeros_like(result)
    for b in range(batch):
        for cam in range(num_cams):
            row = b * num_cams + cam
            out = msda_direct.forward(value[row:row + 1], spatial_shapes, loc[row:row + 1],
                                      attn[row:row + 1])[0]
            for r, bev in enumerate(np.asarray(indexes[cam]).tolist()):
                if 0 <= bev < num_query:
                    total[b, bev] += out[r]
    return result + total / count[..., None]
