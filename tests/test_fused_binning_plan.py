"""Which shapes ms_deform_attn_forward_bin runs as the forward kernel with the
backward's record stores fused in (host-side planning only, no launch).

Every BASELINE training config (c1-c4, fp32 and 16-bit values) writes its
location and weight gradients straight to sample order (slab span at most
8 MB), so the fused path must apply there; a span above 8 MB takes the
records-plus-gather backward and the unfused binning, and channel counts
without a row kernel take the atomic backward (nothing to bin).
"""

import pytest
import torch

from muspace_amd.workloads import CONFIGS


def _meta(cfg, value_dtype):
    value = torch.empty((cfg.batch, cfg.spatial_size, cfg.heads, cfg.channels),
                        dtype=value_dtype, device="meta")
    loc = torch.empty((cfg.batch, cfg.queries, cfg.heads, cfg.num_levels, cfg.points, 2),
                      device="meta")
    return value, loc


@pytest.mark.parametrize("name,value_dtype", [
    ("c1", torch.float32), ("c2", torch.float32), ("c3", torch.float32),
    ("c4", torch.bfloat16), ("c4", torch.float16), ("bevformer-1l", torch.float32),
])
def test_baseline_training_configs_fuse(native_lib, name, value_dtype):
    value, loc = _meta(CONFIGS[name], value_dtype)
    assert native_lib.forward_bin_fuses(value, loc)


def test_span_above_8mb_takes_the_binning_kernels(native_lib):
    # one slab of 22000 queries x 32 samples x 12 bytes = 8.4 MB
    value = torch.empty((1, 600, 2, 32), device="meta")
    loc = torch.empty((1, 22000, 2, 1, 32, 2), device="meta")
    assert not native_lib.forward_bin_fuses(value, loc)
    small = torch.empty((1, 10000, 2, 1, 32, 2), device="meta")
    assert native_lib.forward_bin_fuses(value, small)


@pytest.mark.parametrize("channels", [3, 8, 12])
def test_channels_without_a_tile_path_do_not_fuse(native_lib, channels):
    value = torch.empty((2, 300, 4, channels), device="meta")
    loc = torch.empty((2, 200, 4, 2, 4, 2), device="meta")
    assert not native_lib.forward_bin_fuses(value, loc)
