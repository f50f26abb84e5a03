"""TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

CPU restatements of deformable aggregation (SparseDrive's multi-camera,
multi-scale feature aggregation) as the reference defines it:

* ``aggregate_loops`` follows the reference's PyTorch reference
  ``deformable_aggregation_reference`` and its ``_bilinear_sample``
  (/root/reference/mu_space/ops/deformable_aggregation.py:88-158) sample by
  sample: skip (pt, cam) unless 0 < x < 1 and 0 < y < 1 (:127-130), per scale
  h = y*H - 0.5, w = x*W - 0.5 (:136-137), corners outside the map dropped
  (:104-111), group weight repeated over the group's channels (:138-142).
  Scalar torch ops, so autograd gives its gradients; for tiny shapes only.
* ``aggregate_batched`` computes the same sum with one index_select per
  (camera, scale, corner) over every (batch, anchor, point), written
  independently of the loop form, for shapes the loop cannot reach. It runs on
  whatever device its inputs live on. Skipped points (NaN included) get a
  finite stand-in location before any arithmetic, so their zero mask is exact
  in the output and in every gradient, as the loop form's `continue` is.

Both are differentiable; the backward oracle is autograd of either.
"""

from __future__ import annotations

import torch


def aggregate_loops(mc_ms_feat, spatial_shape, scale_start_index, sampling_location, weights):
    batch, _, channels = mc_ms_feat.shape
    cams, scales, _ = spatial_shape.shape
    anchors, pts = sampling_location.shape[1], sampling_location.shape[2]
    groups = weights.shape[-1]
    per_group = channels // groups
    shapes = spatial_shape.tolist()
    starts = scale_start_index.tolist()
    rows = []
    for b in range(batch):
        for a in range(anchors):
            acc = mc_ms_feat.new_zeros(channels)
            for p in range(pts):
                for c in range(cams):
                    x = sampling_location[b, a, p, c, 0]
                    y = sampling_location[b, a, p, c, 1]
                    if not (0 < float(x.detach()) < 1 and 0 < float(y.detach()) < 1):
                        continue
                    for s in range(scales):
                        height, width = shapes[c][s]
                        fmap = mc_ms_feat[b, starts[c][s]: starts[c][s] + height * width]
                        fmap = fmap.view(height, width, channels)
                        h_im = y * height - 0.5
                        w_im = x * width - 0.5
                        h0 = int(torch.floor(h_im.detach()))
                        w0 = int(torch.floor(w_im.detach()))
                        lh, lw = h_im - h0, w_im - w0
                        hh, hw = 1 - lh, 1 - lw
                        value = mc_ms_feat.new_zeros(channels)
                        if h0 >= 0 and w0 >= 0:
                            value = value + hh * hw * fmap[h0, w0]
                        if h0 >= 0 and w0 + 1 <= width - 1:
                            value = value + hh * lw * fmap[h0, w0 + 1]
                        if h0 + 1 <= height - 1 and w0 >= 0:
                            value = value + lh * hw * fmap[h0 + 1, w0]
                        if h0 + 1 <= height - 1 and w0 + 1 <= width - 1:
                            value = value + lh * lw * fmap[h0 + 1, w0 + 1]
                        acc = acc + value * weights[b, a, p, c, s].repeat_interleave(per_group)
            rows.append(acc)
    return torch.stack(rows).view(batch, anchors, channels)


def aggregate_batched(mc_ms_feat, spatial_shape, scale_start_index, sampling_location, weights):
    batch, num_feat, channels = mc_ms_feat.shape
    cams, scales, _ = spatial_shape.shape
    anchors, pts = sampling_location.shape[1], sampling_location.shape[2]
    groups = weights.shape[-1]
    flat = mc_ms_feat.reshape(batch * num_feat, channels)
    b_base = (torch.arange(batch, device=mc_ms_feat.device) * num_feat).view(batch, 1, 1)
    total = mc_ms_feat.new_zeros((batch, anchors, channels))
    for c in range(cams):
        x = sampling_location[:, :, :, c, 0]
        y = sampling_location[:, :, :, c, 1]
        inside = (x > 0) & (x < 1) & (y > 0) & (y < 1)
        # skipped points (NaN included) take a finite stand-in, so that no NaN
        # reaches a product with a zero mask in the output or the gradients
        x = torch.where(inside, x, torch.full_like(x, 0.5))
        y = torch.where(inside, y, torch.full_like(y, 0.5))
        for s in range(scales):
            height, width = (int(v) for v in spatial_shape[c, s].tolist())
            start = int(scale_start_index[c, s])
            h_im = y * height - 0.5
            w_im = x * width - 0.5
            hl = torch.floor(h_im)
            wl = torch.floor(w_im)
            fh = h_im - hl
            fw = w_im - wl
            hl = hl.long()
            wl = wl.long()
            acc = mc_ms_feat.new_zeros((batch, anchors, pts, channels))
            for dy in (0, 1):
                for dx in (0, 1):
                    yy, xx = hl + dy, wl + dx
                    ok = inside & (yy >= 0) & (yy < height) & (xx >= 0) & (xx < width)
                    coef = (fh if dy else 1 - fh) * (fw if dx else 1 - fw)
                    idx = b_base + start + yy.clamp(0, height - 1) * width + xx.clamp(0, width - 1)
                    rows = flat.index_select(0, idx.reshape(-1)).view(batch, anchors, pts, channels)
                    acc = acc + (coef * ok)[..., None] * rows
            w = weights[:, :, :, c, s, :]  # [B, A, P, G]
            acc = acc.view(batch, anchors, pts, groups, channels // groups) * w[..., None]
            total = total + acc.sum(dim=2).reshape(batch, anchors, channels)
    return total
