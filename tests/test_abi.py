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
def test_forward_validation_fails_before_any_launch(native_lib, overrides, message):
    fn = native_lib.raw("ms_deform_attn_forward")
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
