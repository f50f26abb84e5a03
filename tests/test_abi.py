"""The C-ABI library loads on the CPU host and exports every declared symbol.

No kernel is launched: only symbol resolution, the ABI version and the
host-side argument validation (which fails before any device call).
"""

import ctypes
import re
from pathlib import Path

import pytest

from muspace_amd.runtime import native

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "muspace_msda.h"
HEADERS = sorted((ROOT / "include").glob("*.h"))


def declared_symbols() -> list[str]:
    names = []
    for header in HEADERS:
        names += re.findall(r"^MUSPACE_API\s+(?:const\s+)?\w+\s*\*?\s*(\w+)\s*\(",
                            header.read_text(), re.M)
    return names


def test_header_declares_the_reference_entry_points():
    names = declared_symbols()
    assert {"ms_deform_attn_forward", "ms_deform_attn_backward", "add_one",
            "muspace_last_error", "muspace_abi_version",
            "deformable_aggregation_forward_opt", "deformable_aggregation_backward_opt",
            "deformable_aggregation_forward_base", "deformable_aggregation_backward_base"} <= set(names)


def test_library_exports_every_declared_symbol(native_lib):
    handle = ctypes.CDLL(str(native_lib.path))
    for name in declared_symbols():
        assert hasattr(handle, name), f"{native_lib.path.name} does not export {name}"


def test_loader_binds_every_declared_symbol(native_lib):
    assert set(declared_symbols()) <= set(native._EXPORTS)


def test_abi_version_matches_header(native_lib):
    version = int(re.search(r"#define MUSPACE_MSDA_ABI_VERSION (\d+)", HEADER.read_text()).group(1))
    assert native_lib.raw("muspace_abi_version")() == version == native.ABI_VERSION


def _forward_args(**overrides):
    args = dict(value=None, value_dtype=0, shapes=None, starts=None, loc=None, attn=None,
                geometry_dtype=0, out=None, batch=2, spatial=4, heads=1, channels=32,
                levels=1, queries=3, points=4, im2col_step=64, stream=None)
    args.update(overrides)
    return list(args.values())


@pytest.mark.parametrize(
    ("overrides", "message"),
    [
        ({"value_dtype": 7}, "value must be float32, float16 or bfloat16"),
        ({"value_dtype": 2, "geometry_dtype": 1}, "must be float32 or bfloat16"),
        ({"im2col_step": 0}, "im2col_step must be positive"),
        ({"batch": 3, "im2col_step": 2}, "not divisible by im2col_step"),
        ({"heads": 0}, "invalid dims"),
        ({"levels": 65}, "at most 64 levels"),
        ({"spatial": 1 << 28}, "32-bit"),
        ({}, "null tensor pointer"),
    ],
)
@pytest.mark.parametrize("entry", ["ms_deform_attn_forward", "ms_deform_attn_forward_softmax"])
def test_forward_validation_fails_before_any_launch(native_lib, overrides, message, entry):
    fn = native_lib.raw(entry)
    rc = fn(*_forward_args(**overrides))
    assert rc != 0
    assert message in native_lib.last_error()


def test_empty_problem_is_a_no_op(native_lib):
    fn = native_lib.raw("ms_deform_attn_forward")
    assert fn(*_forward_args(queries=0)) == 0
    assert native_lib.last_error() == ""


def test_backward_validation_fails_before_any_launch(native_lib):
    fn = native_lib.raw("ms_deform_attn_backward")
    args = [None, 0, None, None, None, None, 0, None, None, None, None,
            3, 4, 1, 32, 1, 3, 4, 2, None]
    assert fn(*args) != 0
    assert "not divisible by im2col_step" in native_lib.last_error()
    args[-2] = 64
    assert fn(*args) != 0
    assert "null tensor pointer" in native_lib.last_error()


def test_noalloc_backward_rejects_an_entry_larger_than_its_scratch(native_lib):
    """One batch entry of 8 heads x 100000 queries x 32 samples needs about
    630 MB of tile scratch, more than the 64 MiB array: MUSPACE_ERANGE before
    anything runs (the pointers are stand-ins; nothing may read them)."""
    fn = native_lib.raw("ms_deform_attn_backward_noalloc")
    args = [1, 0, 1, 1, 1, 1, 0, 1, 1, 1, 1,
            2, 30825, 8, 32, 4, 100000, 8, 64, None]
    assert fn(*args) == 2  # MUSPACE_ERANGE
    msg = native_lib.last_error()
    assert "needs" in msg and "scratch" in msg
    # two entries' workspace is far past the array, so the planner steps down
    # to one entry, and reports that entry's real size
    needed = int(re.search(r"needs (\d+) bytes", msg).group(1))
    size = native_lib.raw("ms_deform_attn_backward_workspace_size")
    assert needed == size(0, 1, 30825, 8, 32, 4, 100000, 8) > (64 << 20), msg
    args[1:2] = [9]  # a bad dtype is still MUSPACE_EINVAL, first
    assert fn(*args) == 1


def _backward_ws_args(**overrides):
    args = dict(value=1, value_dtype=0, shapes=1, starts=1, loc=1, attn=1, geometry_dtype=0,
                grad=1, grad_value=1, grad_loc=1, grad_attn=1, batch=2, spatial=4, heads=1,
                channels=32, levels=1, queries=3, points=4, im2col_step=2, workspace=None,
                workspace_bytes=0, stream=None)
    args.update(overrides)
    return list(args.values())


@pytest.mark.parametrize("entry", ["ms_deform_attn_backward_softmax_bin",
                                   "ms_deform_attn_backward_softmax_rest"])
def test_softmax_backward_parts_require_a_workspace(native_lib, entry):
    """The probabilities live at the head of the workspace: no or too small a
    workspace is MUSPACE_EINVAL, checked before anything is launched (the plain
    backward would fall back to atomics instead)."""
    fn = native_lib.raw(entry)
    assert fn(*_backward_ws_args()) == 1
    assert "workspace" in native_lib.last_error()


def test_softmax_workspace_size(native_lib):
    size = native_lib.raw("ms_deform_attn_backward_softmax_workspace_size")
    plain = native_lib.raw("ms_deform_attn_backward_workspace_size")
    dims = (2, 4, 1, 32, 1, 3, 4)  # batch, spatial, heads, channels, levels, queries, points
    probs = 2 * 3 * 1 * 4 * 4  # units * L*P * fp32, padded below to 256 bytes
    assert size(0, 0, *dims) == 256 + plain(0, *dims)
    assert size(0, 0, 2, 4, 1, 3, 1, 3, 4) == 256  # C = 3: no tile path, probabilities only
    assert size(0, 0, 2, 4, 0, 32, 1, 3, 4) == 0  # invalid dims
    assert size(0, 0, 2, 4, 1, 32, 1, 0, 4) == 0  # nothing sampled
    assert probs < 256


def _dfa_forward_args(**overrides):
    args = dict(feat=1, shape=1, start=1, loc=1, weights=1, out=1, batch=1, cams=2, feat_n=10,
                embeds=64, scales=2, anchors=3, pts=4, groups=8, stream=None)
    args.update(overrides)
    return list(args.values())


@pytest.mark.parametrize(
    ("overrides", "message"),
    [
        ({"groups": 9}, "num_groups must be in [1, 8]"),
        ({"groups": 0}, "num_groups must be in [1, 8]"),
        ({"embeds": 60}, "must be divisible by num_groups"),
        ({"cams": 100, "scales": 3}, "num_cams * num_scale must be at most 256"),
        ({"anchors": -1}, "invalid dims"),
        ({"out": None}, "null tensor pointer"),
    ],
)
@pytest.mark.parametrize("entry", ["deformable_aggregation_forward_opt",
                                   "deformable_aggregation_forward_base"])
def test_dfa_forward_validation_fails_before_any_launch(native_lib, overrides, message, entry):
    fn = native_lib.raw(entry)
    assert fn(*_dfa_forward_args(**overrides)) != 0
    assert message in native_lib.last_error()


@pytest.mark.parametrize("entry", ["deformable_aggregation_backward_opt",
                                   "deformable_aggregation_backward_base"])
def test_dfa_backward_validation_fails_before_any_launch(native_lib, entry):
    fn = native_lib.raw(entry)
    args = [1] * 9 + [1, 2, 10, 64, 2, 3, 4, 9, None]  # 9 groups
    assert fn(*args) != 0
    assert "num_groups must be in [1, 8]" in native_lib.last_error()
    args = [1] * 5 + [None] + [1] * 3 + [1, 2, 10, 64, 2, 3, 4, 8, None]  # grad_output NULL
    assert fn(*args) != 0
    assert "null tensor pointer" in native_lib.last_error()
