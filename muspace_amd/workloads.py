"""Seeded MSDA workloads: the benchmark configurations and their byte model.

Plays the role of the reference's benchmark case module
(/root/reference/benchmarks/msda/msda_single_level_case.py:41-82) for the
configurations this build is measured on:

  c0  forward only, 4 levels (32,32),(16,16),(8,8),(4,4), bs 1, nq 1000, P 4
  c1  Deformable-DETR encoder, 4 levels (100,167)...(13,21), bs 2, nq 22223, P 4
  c2  BEVFormer spatial cross-attention, 4 levels (116,200)...(15,25), bs 6, nq 10000, P 8
  c3  BEVFormer temporal self-attention, 1 level (200,200), bs 2, nq 40000, P 4
  c4  c2's levels at bs 12, nq 15000, 16-bit value with float32 geometry
  bevformer-1l  the reference's own published case (value scale 1.38,
      attention weights 0.25, locations U(-0.0175, 1.0175); the reference
      draws a separate backward set, here one set serves both directions)

All have 8 heads of 32 channels. Tensors are drawn on the CPU in float32 from
``torch.Generator("cpu").manual_seed(seed)`` in the order value, locations,
attention logits (softmax over the L*P samples of each query and head),
grad_output, then cast and moved.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

DEFAULT_SEED = 2333
HBM_PEAK_GBPS = 8000.0  # MI355X HBM3E

_SCA_LEVELS = ((116, 200), (58, 100), (29, 50), (15, 25))


@dataclass(frozen=True)
class MSDAConfig:
    name: str
    batch: int
    queries: int
    levels: tuple[tuple[int, int], ...]
    points: int
    loc_low: float
    loc_high: float
    heads: int = 8
    channels: int = 32
    grid_locations: bool = False  # c3: query grid position + N(0, 0.02)
    backward: bool = True
    value_scale: float = 1.0
    constant_attention: float | None = None
    description: str = ""

    @property
    def spatial_size(self) -> int:
        return sum(h * w for h, w in self.levels)

    @property
    def num_levels(self) -> int:
        return len(self.levels)

    def with_queries(self, queries: int) -> "MSDAConfig":
        return MSDAConfig(**{**self.__dict__, "queries": queries})

    def with_batch(self, batch: int) -> "MSDAConfig":
        return MSDAConfig(**{**self.__dict__, "batch": batch})


CONFIGS: dict[str, MSDAConfig] = {
    "c0": MSDAConfig(
        "c0", 1, 1000, ((32, 32), (16, 16), (8, 8), (4, 4)), 4, -0.05, 1.05,
        backward=False, description="forward only, CPU-runnable",
    ),
    "c1": MSDAConfig(
        "c1", 2, 22223, ((100, 167), (50, 84), (25, 42), (13, 21)), 4, -0.05, 1.05,
        description="Deformable-DETR encoder",
    ),
    "c2": MSDAConfig(
        "c2", 6, 10000, _SCA_LEVELS, 8, 0.0, 1.0,
        description="BEVFormer spatial cross-attention",
    ),
    "c3": MSDAConfig(
        "c3", 2, 40000, ((200, 200),), 4, -0.05, 1.05, grid_locations=True,
        description="BEVFormer temporal self-attention",
    ),
    "c4": MSDAConfig(
        "c4", 12, 15000, _SCA_LEVELS, 8, 0.0, 1.0,
        description="BEVFormer spatial cross-attention, 16-bit value, fp32 geometry",
    ),
    "bevformer-1l": MSDAConfig(
        "bevformer-1l", 2, 40000, ((200, 200),), 4, -0.0175, 1.0175,
        value_scale=1.38, constant_attention=0.25,
        description="the reference's published single-level case",
    ),
}


def level_start_index(levels) -> torch.Tensor:
    sizes = [h * w for h, w in levels]
    starts = [0]
    for s in sizes[:-1]:
        starts.append(starts[-1] + s)
    return torch.tensor(starts[: len(sizes)], dtype=torch.int64)


def make_inputs(
    cfg: MSDAConfig,
    *,
    seed: int = DEFAULT_SEED,
    value_dtype: torch.dtype = torch.float32,
    geometry_dtype: torch.dtype = torch.float32,
    device: str | torch.device = "cpu",
    with_grad_output: bool = True,
) -> dict[str, torch.Tensor]:
    """Seeded inputs of ``cfg`` (see module docstring for the draw order)."""
    gen = torch.Generator(device="cpu").manual_seed(seed)
    bs, nq, M, C, P, L = cfg.batch, cfg.queries, cfg.heads, cfg.channels, cfg.points, cfg.num_levels
    value = torch.randn((bs, cfg.spatial_size, M, C), generator=gen) * cfg.value_scale
    if cfg.grid_locations:
        (h, w), = cfg.levels
        idx = torch.arange(nq)
        centre = torch.stack([(idx % w + 0.5) / w, (idx // w + 0.5) / h], dim=-1)
        noise = torch.randn((bs, nq, M, L, P, 2), generator=gen) * 0.02
        loc = (centre.view(1, nq, 1, 1, 1, 2) + noise).clamp_(cfg.loc_low, cfg.loc_high)
    else:
        loc = torch.rand((bs, nq, M, L, P, 2), generator=gen)
        loc = loc * (cfg.loc_high - cfg.loc_low) + cfg.loc_low
    if cfg.constant_attention is not None:
        attn = torch.full((bs, nq, M, L, P), cfg.constant_attention)
    else:
        logits = torch.randn((bs, nq, M, L * P), generator=gen)
        attn = torch.softmax(logits, dim=-1).view(bs, nq, M, L, P)
    out = {
        "value": value.to(value_dtype).to(device),
        "spatial_shapes": torch.tensor(cfg.levels, dtype=torch.int64).to(device),
        "level_start_index": level_start_index(cfg.levels).to(device),
        "sampling_locations": loc.to(geometry_dtype).to(device),
        "attention_weights": attn.to(geometry_dtype).to(device),
    }
    if with_grad_output:
        grad = torch.randn((bs, nq, M * C), generator=gen)
        out["grad_output"] = grad.to(value_dtype).to(device)
    return out


def algorithmic_bytes(
    cfg: MSDAConfig,
    value_dtype: torch.dtype = torch.float32,
    geometry_dtype: torch.dtype = torch.float32,
) -> tuple[int, int]:
    """(forward, backward) algorithmic bytes: every tensor once at its storage width.

    fwd = |value| + |loc| + |attn| + |out|
    bwd = |value| + |loc| + |attn| + |grad_out| + |grad_value f32| + |grad_loc f32| + |grad_attn f32|
    Zero-fills, dtype casts and repeated gathers of the same value rows are
    not counted.
    """
    vb = torch.empty((), dtype=value_dtype).element_size()
    gb = torch.empty((), dtype=geometry_dtype).element_size()
    n_value = cfg.batch * cfg.spatial_size * cfg.heads * cfg.channels
    n_attn = cfg.batch * cfg.queries * cfg.heads * cfg.num_levels * cfg.points
    n_loc = 2 * n_attn
    n_out = cfg.batch * cfg.queries * cfg.heads * cfg.channels
    fwd = n_value * vb + n_loc * gb + n_attn * gb + n_out * vb
    bwd = n_value * vb + n_loc * gb + n_attn * gb + n_out * vb + 4 * (n_value + n_loc + n_attn)
    return fwd, bwd


def backward_rest_bytes(cfg: MSDAConfig, value_dtype: torch.dtype = torch.float32) -> int:
    """Algorithmic bytes of the backward's second part (the tile kernel,
    ms_deform_attn_backward_rest): the tensors it reads or writes, once --
    value, grad_output and the three float32 gradients. Its binned records are
    scratch derived from the locations and weights, which the binning read."""
    vb = torch.empty((), dtype=value_dtype).element_size()
    n_value = cfg.batch * cfg.spatial_size * cfg.heads * cfg.channels
    n_attn = cfg.batch * cfg.queries * cfg.heads * cfg.num_levels * cfg.points
    n_out = cfg.batch * cfg.queries * cfg.heads * cfg.channels
    return n_value * vb + n_out * vb + 4 * (n_value + 2 * n_attn + n_attn)


# ------------------------------------------- the reference's published case ---


def make_published_case(
    *,
    seed: int = DEFAULT_SEED,
    dtype: torch.dtype = torch.float32,
    device: str | torch.device = "cpu",
) -> dict[str, dict[str, torch.Tensor]]:
    """The reference's published MSDA case ``bevformer-1l``, as its benchmark
    draws it (/root/reference/benchmarks/msda/msda_single_level_case.py:41-82):
    separate forward and backward input sets from generators seeded ``seed``
    and ``seed + 1`` (value scale 1.38 and 1.25), one 200x200 level, 40000
    queries of 8 heads x 32 channels and 4 points, locations
    ``U(0, 1) * 1.035 - 0.0175``, attention weights 0.25, every tensor in
    ``dtype`` (geometry included), and a non-contiguous grad_output: a
    ``[40000, 256, 2]`` draw scaled by 6.3e-6 and permuted to
    ``[2, 40000, 256]`` (strides (1, 512, 2)), so the timed region keeps the
    reference's ``grad_output.contiguous()`` copy."""
    batch, queries, heads, channels, points = 2, 40000, 8, 32, 4

    def draw(gen, scale):
        value = torch.randn((batch, 40000, heads, channels), generator=gen) * scale
        loc = torch.rand((batch, queries, heads, 1, points, 2), generator=gen) * 1.035 - 0.0175
        return {
            "value": value.to(dtype).to(device),
            "spatial_shapes": torch.tensor([[200, 200]], dtype=torch.int64).to(device),
            "level_start_index": torch.tensor([0], dtype=torch.int64).to(device),
            "sampling_locations": loc.to(dtype).to(device),
            "attention_weights": torch.full((batch, queries, heads, 1, points), 0.25,
                                            dtype=dtype).to(device),
        }

    forward_gen = torch.Generator(device="cpu").manual_seed(seed)
    backward_gen = torch.Generator(device="cpu").manual_seed(seed + 1)
    forward_inputs = draw(forward_gen, 1.38)
    backward_inputs = draw(backward_gen, 1.25)
    grad = torch.randn((queries, heads * channels, batch), generator=backward_gen) * 6.3e-6
    backward_inputs["grad_output"] = grad.to(dtype).to(device).permute(2, 0, 1)
    return {"forward_inputs": forward_inputs, "backward_inputs": backward_inputs}


# ------------------------------------------------ spatial cross-attention ---

SCA_BEV = (200, 200)  # BEVFormer-base BEV grid: 40000 queries
SCA_CAMERAS = 6
SCA_FOV_DEG = 90.0


def sca_camera_indexes(
    bev_h: int = SCA_BEV[0],
    bev_w: int = SCA_BEV[1],
    num_cams: int = SCA_CAMERAS,
    fov_deg: float = SCA_FOV_DEG,
) -> tuple[list[torch.Tensor], torch.Tensor]:
    """(indexes, count) of a synthetic camera ring, on the CPU.

    num_cams cameras sit at the centre of the BEV grid; camera i looks along
    360*i/num_cams degrees and sees the cells whose centre lies within fov_deg/2
    of that direction. ``indexes[i]`` lists those cells (row-major BEV ids, in
    increasing order, as ``nonzero`` gives them) and ``count`` ``[bev_h*bev_w]``
    is the number of cameras that see each cell, at least 1 (BEVFormer's
    ``count.clamp(min=1)``). At the defaults each camera sees 9900 or 10000 of
    the 40000 cells and about half of the cells are seen by two cameras.
    """
    ys, xs = torch.meshgrid(torch.arange(bev_h, dtype=torch.float64),
                            torch.arange(bev_w, dtype=torch.float64), indexing="ij")
    angle = torch.rad2deg(torch.atan2(ys + 0.5 - bev_h / 2, xs + 0.5 - bev_w / 2)).flatten()
    indexes = []
    count = torch.zeros(bev_h * bev_w, dtype=torch.float32)
    for cam in range(num_cams):
        off = (angle - 360.0 * cam / num_cams + 180.0) % 360.0 - 180.0
        seen = off.abs() < fov_deg / 2
        indexes.append(torch.nonzero(seen).flatten())
        count += seen.float()
    return indexes, count.clamp_(min=1.0)


def make_sca_inputs(
    *,
    seed: int = DEFAULT_SEED,
    device: str | torch.device = "cpu",
) -> dict[str, object]:
    """c2's tensors as one BEVFormer sample's six rebatched cameras, plus the
    camera ring of :func:`sca_camera_indexes` (max valid rows 10000 = c2's nq)."""
    cfg = CONFIGS["c2"]
    assert cfg.batch == SCA_CAMERAS
    inputs = make_inputs(cfg, seed=seed, device=device, with_grad_output=False)
    indexes, count = sca_camera_indexes()
    assert max(len(i) for i in indexes) <= cfg.queries
    inputs["indexes"] = [i.to(device) for i in indexes]
    inputs["count"] = count.view(1, -1).to(device)
    return inputs


def sca_algorithmic_bytes(valid_rows: int, cameras: int, num_query: int,
                          cfg: MSDAConfig | None = None) -> int:
    """Algorithmic bytes of the fused scatter-average forward (fp32).

    Every tensor once at its storage width: the cameras' value, the geometry
    of the valid rows (loc, attn), their int64 index and float32 count
    entries, and the slots read once and written once. Padding rows are not
    read.
    """
    cfg = cfg or CONFIGS["c2"]
    n_value = cfg.batch * cfg.spatial_size * cfg.heads * cfg.channels
    per_row = cfg.heads * cfg.num_levels * cfg.points  # attention weights per row
    row = cfg.heads * cfg.channels
    slots = (cfg.batch // cameras) * num_query * row
    return 4 * n_value + valid_rows * (4 * 3 * per_row + 8 + 4) + 2 * 4 * slots


# --------------------------------------------------- deformable aggregation ---

# SparseDrive's production shape, as the reference's benchmark case defines it
# (/root/reference/benchmarks/deformable_aggregation/deformable_aggregation_case.py:30-54):
# 8 samples, 6 cameras x 4 scales of (64,176)..(8,22) maps, 256 channels in 8
# groups, 900 anchors x 13 points, 18.6% of (anchor, point, camera) inside (0, 1).
DFA_BATCH, DFA_CAMS, DFA_ANCHORS, DFA_PTS, DFA_GROUPS, DFA_CHANNELS = 8, 6, 900, 13, 8, 256
DFA_SCALES = ((64, 176), (32, 88), (16, 44), (8, 22))
DFA_ACTIVE_FRAC = 0.18635328114032745
DFA_WEIGHT_SCALE = 0.004


def make_dfa_inputs(
    *,
    seed: int = DEFAULT_SEED,
    device: str | torch.device = "cpu",
    active_frac: float = DFA_ACTIVE_FRAC,
) -> dict[str, torch.Tensor]:
    """Seeded SparseDrive-shaped inputs. Drawn on the CPU in the order feature
    maps ~ N(0,1), active mask, outside points ~ 10*N(0,1), inside points
    ~ U(0.01, 0.99), weights ~ 0.004*U(0,1), then grad_output ~ N(0,1)."""
    gen = torch.Generator(device="cpu").manual_seed(seed)
    per_cam = sum(h * w for h, w in DFA_SCALES)
    num_feat = DFA_CAMS * per_cam
    starts, offset = [], 0
    for _ in range(DFA_CAMS):
        row = []
        for h, w in DFA_SCALES:
            row.append(offset)
            offset += h * w
        starts.append(row)
    point_shape = (DFA_BATCH, DFA_ANCHORS, DFA_PTS, DFA_CAMS)
    feat = torch.randn((DFA_BATCH, num_feat, DFA_CHANNELS), generator=gen)
    active = torch.rand(point_shape, generator=gen) < active_frac
    outside = torch.randn(*point_shape, 2, generator=gen) * 10.0
    inside = torch.rand(*point_shape, 2, generator=gen) * 0.98 + 0.01
    loc = torch.where(active.unsqueeze(-1), inside, outside)
    weights = torch.rand((*point_shape, len(DFA_SCALES), DFA_GROUPS), generator=gen)
    weights = weights * DFA_WEIGHT_SCALE
    grad = torch.randn((DFA_BATCH, DFA_ANCHORS, DFA_CHANNELS), generator=gen)
    return {
        "mc_ms_feat": feat.to(device),
        "spatial_shape": torch.tensor([list(map(list, DFA_SCALES))] * DFA_CAMS,
                                      dtype=torch.int32).to(device),
        "scale_start_index": torch.tensor(starts, dtype=torch.int32).to(device),
        "sampling_location": loc.to(device),
        "weights": weights.to(device),
        "grad_output": grad.to(device),
    }


def dfa_algorithmic_bytes() -> tuple[int, int]:
    """(forward, backward) bytes of the SparseDrive shape, every tensor once:
    fwd = |feat| + |loc| + |weights| + |out|; bwd adds |grad_out| and the three
    gradients (float32) to the inputs."""
    per_cam = sum(h * w for h, w in DFA_SCALES)
    n_feat = DFA_BATCH * DFA_CAMS * per_cam * DFA_CHANNELS
    n_pts = DFA_BATCH * DFA_ANCHORS * DFA_PTS * DFA_CAMS
    n_loc = 2 * n_pts
    n_w = n_pts * len(DFA_SCALES) * DFA_GROUPS
    n_out = DFA_BATCH * DFA_ANCHORS * DFA_CHANNELS
    fwd = 4 * (n_feat + n_loc + n_w + n_out)
    bwd = 4 * (n_feat + n_loc + n_w + n_out + n_feat + n_loc + n_w)
    return fwd, bwd
