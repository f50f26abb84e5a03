"""Loader for the MI355X C-ABI library ``libmuspace_msda.so``.

Replaces the reference's TVM-FFI loader
(/root/reference/mu_space/runtime/native.py:20-77). The public names are kept
(``load_native_module``, ``native_function``, ``native_module_proxy``,
``native_available``, ``native_error``, ``NativeModuleUnavailable``), but the
library is a plain C-ABI shared object opened with :mod:`ctypes`, and every
export is resolved once at load time instead of on every call.

The callables returned for ``ms_deform_attn_forward`` / ``ms_deform_attn_backward``
take torch tensors with the argument order of the reference exports
(/root/reference/csrc/ms_deformable_attn/ms_deform_attn_musa.mu:507-628), check
device, dtype, contiguity and shapes the way ``check_musa_contiguous``
(/root/reference/csrc/ffi/tensor_utils.hpp:13-38) does, and launch on the
caller's current HIP stream. A non-zero return code becomes ``RuntimeError``
carrying the library's message.
"""

from __future__ import annotations

import ctypes
from functools import lru_cache
from importlib.resources import files
from pathlib import Path
from typing import Any, Callable

LIBRARY_RELPATH = "native/libmuspace_msda.so"
ABI_VERSION = 6

DTYPE_F32, DTYPE_F16, DTYPE_BF16 = 0, 1, 2

_c_int64 = ctypes.c_int64
_c_int = ctypes.c_int
_c_ptr = ctypes.c_void_p

# name -> (restype, argtypes); mirrors include/muspace_msda.h
_EXPORTS: dict[str, tuple[Any, list[Any]]] = {
    "muspace_abi_version": (_c_int, []),
    "muspace_last_error": (ctypes.c_char_p, []),
    "add_one": (_c_int, [_c_ptr, _c_ptr, _c_int64, _c_ptr]),
    "ms_deform_attn_forward": (
        _c_int,
        [_c_ptr, _c_int, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_int, _c_ptr]
        + [_c_int64] * 8
        + [_c_ptr],
    ),
    "ms_deform_attn_backward": (
        _c_int,
        [_c_ptr, _c_int, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_int, _c_ptr, _c_ptr, _c_ptr, _c_ptr]
        + [_c_int64] * 8
        + [_c_ptr],
    ),
    "ms_deform_attn_backward_ws": (
        _c_int,
        [_c_ptr, _c_int, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_int, _c_ptr, _c_ptr, _c_ptr, _c_ptr]
        + [_c_int64] * 8
        + [_c_ptr, ctypes.c_size_t, _c_ptr],
    ),
    "ms_deform_attn_backward_noalloc": (
        _c_int,
        [_c_ptr, _c_int, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_int, _c_ptr, _c_ptr, _c_ptr, _c_ptr]
        + [_c_int64] * 8
        + [_c_ptr],
    ),
    "ms_deform_attn_backward_workspace_size": (ctypes.c_size_t, [_c_int] + [_c_int64] * 7),
    "ms_deform_attn_forward_bin_fused": (_c_int, [_c_int] + [_c_int64] * 7),
    "ms_deform_attn_backward_bin": (
        _c_int,
        [_c_ptr, _c_int, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_int, _c_ptr, _c_ptr, _c_ptr, _c_ptr]
        + [_c_int64] * 8
        + [_c_ptr, ctypes.c_size_t, _c_ptr],
    ),
    "ms_deform_attn_backward_rest": (
        _c_int,
        [_c_ptr, _c_int, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_int, _c_ptr, _c_ptr, _c_ptr, _c_ptr]
        + [_c_int64] * 8
        + [_c_ptr, ctypes.c_size_t, _c_ptr],
    ),
    "ms_deform_attn_forward_bin": (
        _c_int,
        [_c_ptr, _c_int, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_int, _c_ptr, _c_ptr, _c_ptr, _c_ptr]
        + [_c_int64] * 8
        + [_c_ptr, ctypes.c_size_t, _c_ptr],
    ),
    "ms_deform_attn_forward_softmax": (
        _c_int,
        [_c_ptr, _c_int, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_int, _c_ptr]
        + [_c_int64] * 8
        + [_c_ptr],
    ),
    "ms_deform_attn_backward_softmax_workspace_size": (
        ctypes.c_size_t, [_c_int, _c_int] + [_c_int64] * 7
    ),
    "ms_deform_attn_backward_softmax_bin": (
        _c_int,
        [_c_ptr, _c_int, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_int, _c_ptr, _c_ptr, _c_ptr, _c_ptr]
        + [_c_int64] * 8
        + [_c_ptr, ctypes.c_size_t, _c_ptr],
    ),
    "ms_deform_attn_backward_softmax_rest": (
        _c_int,
        [_c_ptr, _c_int, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_int, _c_ptr, _c_ptr, _c_ptr, _c_ptr]
        + [_c_int64] * 8
        + [_c_ptr, ctypes.c_size_t, _c_ptr],
    ),
    "ms_deform_attn_forward_softmax_bin": (
        _c_int,
        [_c_ptr, _c_int, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_int, _c_ptr, _c_ptr, _c_ptr, _c_ptr]
        + [_c_int64] * 8
        + [_c_ptr, ctypes.c_size_t, _c_ptr],
    ),
    "ms_deform_attn_forward_softmax_bin_fused": (_c_int, [_c_int] + [_c_int64] * 7),
    "ms_deform_attn_backward_softmax": (
        _c_int,
        [_c_ptr, _c_int, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_int, _c_ptr, _c_ptr, _c_ptr, _c_ptr]
        + [_c_int64] * 8
        + [_c_ptr],
    ),
    "ms_deform_attn_forward_scatter_div": (
        _c_int,
        [_c_ptr, _c_int, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_int, _c_ptr, _c_ptr, _c_ptr]
        + [_c_int64] * 11
        + [_c_ptr],
    ),
    "ms_deform_attn_forward_scatter_div_cams": (
        _c_int,
        [_c_ptr, _c_int, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_int, _c_ptr, _c_ptr, _c_ptr, _c_ptr]
        + [_c_int64] * 9
        + [_c_ptr],
    ),
    "ms_deform_attn_scatter_div_grad": (
        _c_int,
        [_c_ptr, _c_int, _c_ptr, _c_ptr, _c_ptr, _c_int, _c_ptr] + [_c_int64] * 5 + [_c_ptr],
    ),
    # include/muspace_dfa.h
    "deformable_aggregation_forward_opt": (_c_int, [_c_ptr] * 6 + [_c_int64] * 8 + [_c_ptr]),
    "deformable_aggregation_forward_base": (_c_int, [_c_ptr] * 6 + [_c_int64] * 8 + [_c_ptr]),
    "deformable_aggregation_backward_opt": (_c_int, [_c_ptr] * 9 + [_c_int64] * 8 + [_c_ptr]),
    "deformable_aggregation_backward_base": (_c_int, [_c_ptr] * 9 + [_c_int64] * 8 + [_c_ptr]),
}


class NativeModuleUnavailable(RuntimeError):
    """The package does not contain a usable libmuspace_msda.so."""


def library_path() -> Path:
    return Path(files("muspace_amd").joinpath(LIBRARY_RELPATH))


def _dtype_code(dtype) -> int:
    import torch

    codes = {torch.float32: DTYPE_F32, torch.float16: DTYPE_F16, torch.bfloat16: DTYPE_BF16}
    try:
        return codes[dtype]
    except KeyError:
        raise RuntimeError(f"unsupported dtype {dtype}") from None


def _is_device_tensor(tensor) -> bool:
    """A tensor in GPU memory (torch's ``cuda`` device type on a ROCm build)."""
    return bool(getattr(tensor, "is_cuda", False))


def _check(tensor, name: str, dtypes, device=None) -> None:
    """Device, dtype and contiguity of one tensor argument (the reference's
    ``check_musa_contiguous``, csrc/ffi/tensor_utils.hpp:13-38); ``device``,
    when given, is the device every argument of the call must share."""
    if tensor is None:
        raise RuntimeError(f"{name} is required")
    if not _is_device_tensor(tensor):
        raise RuntimeError(f"{name} must be a ROCm device tensor, got device {tensor.device}")
    if device is not None and tensor.device != device:
        raise RuntimeError(f"{name} is on {tensor.device}, expected {device} (the value's device)")
    if tensor.dtype not in dtypes:
        allowed = ", ".join(str(d).replace("torch.", "") for d in dtypes)
        raise RuntimeError(f"{name} must be {allowed}, got {str(tensor.dtype).replace('torch.', '')}")
    if not tensor.is_contiguous():
        raise RuntimeError(f"{name} must be contiguous")


def _check_shape(tensor, name: str, shape: tuple[int, ...]) -> None:
    if tuple(tensor.shape) != shape:
        raise RuntimeError(f"{name} must have shape {list(shape)}, got {list(tensor.shape)}")


class NativeLibrary:
    """The loaded library with its exports bound once."""

    def __init__(self, handle: ctypes.CDLL, path: Path) -> None:
        self.path = path
        self._raw: dict[str, Any] = {}
        for name, (restype, argtypes) in _EXPORTS.items():
            try:
                fn = getattr(handle, name)
            except AttributeError:
                raise NativeModuleUnavailable(
                    f"muSPACE native library {path.name} does not export {name!r}"
                ) from None
            fn.restype = restype
            fn.argtypes = argtypes
            self._raw[name] = fn
        version = self._raw["muspace_abi_version"]()
        if version != ABI_VERSION:
            raise NativeModuleUnavailable(
                f"muSPACE native library {path} has ABI version {version}, expected {ABI_VERSION}; "
                "rebuild it with `python -m muspace_amd.build`"
            )
        self._bound: dict[str, Callable[..., Any]] = {
            "check_forward": self.check_forward,
            "check_backward": self.check_backward,
            "ms_deform_attn_forward": self.ms_deform_attn_forward,
            "ms_deform_attn_backward": self.ms_deform_attn_backward,
            "ms_deform_attn_backward_noalloc": self.ms_deform_attn_backward_noalloc,
            "backward_workspace": self.backward_workspace,
            "backward_workspace_bytes": self.backward_workspace_bytes,
            "backward_softmax_workspace_bytes": self.backward_softmax_workspace_bytes,
            "ms_deform_attn_backward_bin": self.ms_deform_attn_backward_bin,
            "ms_deform_attn_backward_rest": self.ms_deform_attn_backward_rest,
            "ms_deform_attn_forward_bin": self.ms_deform_attn_forward_bin,
            "forward_bin_fuses": self.forward_bin_fuses,
            "ms_deform_attn_forward_softmax": self.ms_deform_attn_forward_softmax,
            "ms_deform_attn_backward_softmax": self.ms_deform_attn_backward_softmax,
            "backward_softmax_workspace": self.backward_softmax_workspace,
            "ms_deform_attn_backward_softmax_bin": self.ms_deform_attn_backward_softmax_bin,
            "ms_deform_attn_backward_softmax_rest": self.ms_deform_attn_backward_softmax_rest,
            "ms_deform_attn_forward_softmax_bin": self.ms_deform_attn_forward_softmax_bin,
            "forward_softmax_bin_fuses": self.forward_softmax_bin_fuses,
            "ms_deform_attn_forward_scatter_div": self.ms_deform_attn_forward_scatter_div,
            "ms_deform_attn_forward_scatter_div_cams": self.ms_deform_attn_forward_scatter_div_cams,
            "deformable_aggregation_forward_opt": self.deformable_aggregation_forward_opt,
            "deformable_aggregation_forward_base": self.deformable_aggregation_forward_base,
            "deformable_aggregation_backward_opt": self.deformable_aggregation_backward_opt,
            "deformable_aggregation_backward_base": self.deformable_aggregation_backward_base,
            "ms_deform_attn_scatter_div_grad": self.ms_deform_attn_scatter_div_grad,
            "add_one": self.add_one,
        }

    # ----------------------------------------------------------- helpers ---
    def raw(self, name: str) -> Any:
        """The bare ctypes function for ``name`` (pointer-level C-ABI)."""
        try:
            return self._raw[name]
        except KeyError:
            raise NativeModuleUnavailable(
                f"muSPACE native library does not export {name!r}"
            ) from None

    def function(self, name: str) -> Callable[..., Any]:
        try:
            return self._bound[name]
        except KeyError:
            pass
        return self.raw(name)

    def last_error(self) -> str:
        msg = self._raw["muspace_last_error"]()
        return msg.decode("utf-8", "replace") if msg else ""

    def _raise_on(self, rc: int, name: str) -> None:
        if rc != 0:
            raise RuntimeError(self.last_error() or f"{name} failed with code {rc}")

    @staticmethod
    def _stream(tensor) -> int:
        import torch

        return torch.cuda.current_stream(tensor.device).cuda_stream

    # ------------------------------------------------------ tensor entry ---
    def ms_deform_attn_forward(
        self, value, spatial_shapes, level_start_index, sampling_locations,
        attention_weights, output, im2col_step: int,
    ) -> None:
        """Tensor-level forward with the reference export's argument order."""
        self._forward_call("ms_deform_attn_forward", value, spatial_shapes, level_start_index,
                           sampling_locations, attention_weights, output, im2col_step)

    def ms_deform_attn_forward_softmax(
        self, value, spatial_shapes, level_start_index, sampling_locations,
        attention_logits, output, im2col_step: int,
    ) -> None:
        """Forward with the attention weights given as logits: each (b, q, m)
        unit's weights are the softmax of its L*P logits (fused)."""
        self._forward_call("ms_deform_attn_forward_softmax", value, spatial_shapes,
                           level_start_index, sampling_locations, attention_logits, output,
                           im2col_step)

    def check_forward(self, value, spatial_shapes, level_start_index, sampling_locations,
                      attention_weights, output=None) -> tuple[int, ...]:
        """Validate the forward's tensors without launching anything.

        Every tensor must be a contiguous ROCm tensor on the value's device
        with the dtype the kernels read, and the shapes must agree with
        ``value`` and ``spatial_shapes`` -- the reference checks all of them
        before its first launch (ms_deform_attn_musa.mu:514-522,
        csrc/ffi/tensor_utils.hpp:13-38). ``output`` may be None (the binning
        part of the backward has none). Raises RuntimeError; returns
        (batch, spatial, heads, channels, levels, queries, points).
        """
        import torch

        _check(value, "value", (torch.float32, torch.float16, torch.bfloat16))
        dev = value.device
        _check(spatial_shapes, "spatial_shapes", (torch.int64,), dev)
        _check(level_start_index, "level_start_index", (torch.int64,), dev)
        geom = (torch.float32,) if value.dtype == torch.float32 else (torch.float32, value.dtype)
        _check(sampling_locations, "sampling_locations", geom, dev)
        _check(attention_weights, "attention_weights", (sampling_locations.dtype,), dev)
        if value.dim() != 4 or sampling_locations.dim() != 6:
            raise RuntimeError("value must be 4-D and sampling_locations 6-D")
        if spatial_shapes.dim() != 2:
            raise RuntimeError("spatial_shapes must be 2-D [num_levels, 2]")
        batch, spatial, heads, channels = value.shape
        levels = spatial_shapes.shape[0]
        queries, points = sampling_locations.shape[1], sampling_locations.shape[4]
        _check_shape(spatial_shapes, "spatial_shapes", (levels, 2))
        _check_shape(level_start_index, "level_start_index", (levels,))
        _check_shape(sampling_locations, "sampling_locations",
                     (batch, queries, heads, levels, points, 2))
        _check_shape(attention_weights, "attention_weights", (batch, queries, heads, levels, points))
        if output is not None:
            _check(output, "out", (value.dtype,), dev)
            _check_shape(output, "out", (batch, queries, heads * channels))
        return batch, spatial, heads, channels, levels, queries, points

    def check_backward(self, value, spatial_shapes, level_start_index, sampling_locations,
                       attention_weights, grad_output, grad_value, grad_sampling_locations,
                       grad_attention_weights) -> tuple[int, ...]:
        """Validate the backward's tensors (as :meth:`check_forward`, plus
        grad_output in the value's dtype and three float32 gradients of the
        inputs' shapes). ``grad_output`` is None for the binning part, which
        does not read it. Raises RuntimeError; returns the dims."""
        import torch

        dims = self.check_forward(value, spatial_shapes, level_start_index, sampling_locations,
                                  attention_weights)
        batch, _, heads, channels, _, queries, _ = dims
        dev = value.device
        if grad_output is not None:
            _check(grad_output, "grad", (value.dtype,), dev)
            _check_shape(grad_output, "grad", (batch, queries, heads * channels))
        for tensor, name, like in ((grad_value, "grad_value", value),
                                   (grad_sampling_locations, "grad_sampling_locations",
                                    sampling_locations),
                                   (grad_attention_weights, "grad_attention_weights",
                                    attention_weights)):
            _check(tensor, name, (torch.float32,), dev)
            _check_shape(tensor, name, tuple(like.shape))
        return dims

    def _forward_call(self, name, value, spatial_shapes, level_start_index, sampling_locations,
                      attention_weights, output, im2col_step) -> None:
        import torch

        batch, spatial, heads, channels, levels, queries, points = self.check_forward(
            value, spatial_shapes, level_start_index, sampling_locations, attention_weights,
            output)
        with torch.cuda.device(value.device):
            rc = self._raw[name](
                value.data_ptr(), _dtype_code(value.dtype), spatial_shapes.data_ptr(),
                level_start_index.data_ptr(), sampling_locations.data_ptr(),
                attention_weights.data_ptr(), _dtype_code(sampling_locations.dtype),
                output.data_ptr(), batch, spatial, heads, channels, levels, queries, points,
                int(im2col_step), self._stream(value),
            )
        self._raise_on(rc, name)

    def ms_deform_attn_backward(
        self, value, spatial_shapes, level_start_index, sampling_locations,
        attention_weights, grad_output, grad_value, grad_sampling_locations,
        grad_attention_weights, im2col_step: int,
    ) -> None:
        """Tensor-level backward with the reference export's argument order.

        All three gradient buffers are overwritten (none needs zero-filling).
        The tile-owned kernels' scratch comes from torch's caching allocator
        on the value's device.
        """
        import torch

        self.check_backward(value, spatial_shapes, level_start_index, sampling_locations,
                            attention_weights, grad_output, grad_value, grad_sampling_locations,
                            grad_attention_weights)
        with torch.cuda.device(value.device):
            workspace = self.backward_workspace(value, sampling_locations)
            self._backward_call("ms_deform_attn_backward_ws", value, spatial_shapes,
                                level_start_index, sampling_locations, attention_weights,
                                grad_output, grad_value, grad_sampling_locations,
                                grad_attention_weights, im2col_step, workspace,
                                self._stream(value))

    def ms_deform_attn_backward_noalloc(
        self, value, spatial_shapes, level_start_index, sampling_locations,
        attention_weights, grad_output, grad_value, grad_sampling_locations,
        grad_attention_weights, im2col_step: int,
    ) -> None:
        """:meth:`ms_deform_attn_backward` through the C entry that allocates
        nothing: its scratch is the library's fixed per-GPU array
        (MUSPACE_NOALLOC_SCRATCH_BYTES), the batch processed in passes that fit
        it. Calls that overlap on one GPU race on that array."""
        import torch

        dims = self.check_backward(value, spatial_shapes, level_start_index, sampling_locations,
                                   attention_weights, grad_output, grad_value,
                                   grad_sampling_locations, grad_attention_weights)
        with torch.cuda.device(value.device):
            rc = self._raw["ms_deform_attn_backward_noalloc"](
                value.data_ptr(), _dtype_code(value.dtype), spatial_shapes.data_ptr(),
                level_start_index.data_ptr(), sampling_locations.data_ptr(),
                attention_weights.data_ptr(), _dtype_code(sampling_locations.dtype),
                grad_output.data_ptr(), grad_value.data_ptr(),
                grad_sampling_locations.data_ptr(), grad_attention_weights.data_ptr(),
                *dims, int(im2col_step), self._stream(value),
            )
        self._raise_on(rc, "ms_deform_attn_backward_noalloc")

    def ms_deform_attn_backward_softmax(
        self, value, spatial_shapes, level_start_index, sampling_locations,
        attention_logits, grad_output, grad_value, grad_sampling_locations,
        grad_attention_logits, im2col_step: int,
    ) -> None:
        """Backward of :meth:`ms_deform_attn_forward_softmax`: the value,
        location and logit gradients, all overwritten. Scratch (the softmax
        probabilities and the binning) comes from torch's caching allocator."""
        import torch

        self.check_backward(value, spatial_shapes, level_start_index, sampling_locations,
                            attention_logits, grad_output, grad_value, grad_sampling_locations,
                            grad_attention_logits)
        with torch.cuda.device(value.device):
            workspace = self.backward_softmax_workspace(value, sampling_locations)
            stream = self._stream(value)
            for name in ("ms_deform_attn_backward_softmax_bin",
                         "ms_deform_attn_backward_softmax_rest"):
                self._backward_call(name, value, spatial_shapes, level_start_index,
                                    sampling_locations, attention_logits, grad_output,
                                    grad_value, grad_sampling_locations, grad_attention_logits,
                                    im2col_step, workspace, stream)

    def _workspace_bytes(self, value, sampling_locations, softmax: bool) -> int:
        batch, spatial, heads, channels = value.shape
        queries, levels, points = (sampling_locations.shape[1], sampling_locations.shape[3],
                                   sampling_locations.shape[4])
        if softmax:
            return int(self._raw["ms_deform_attn_backward_softmax_workspace_size"](
                _dtype_code(value.dtype), _dtype_code(sampling_locations.dtype), batch, spatial,
                heads, channels, levels, queries, points))
        return int(self._raw["ms_deform_attn_backward_workspace_size"](
            _dtype_code(value.dtype), batch, spatial, heads, channels, levels, queries, points))

    def backward_workspace_bytes(self, value, sampling_locations) -> int:
        """Scratch bytes of the tile-owned backward for these shapes (0: the
        shape takes the atomic fallback)."""
        return self._workspace_bytes(value, sampling_locations, softmax=False)

    def backward_softmax_workspace_bytes(self, value, sampling_locations) -> int:
        """Scratch bytes of the softmax backward for these shapes."""
        return self._workspace_bytes(value, sampling_locations, softmax=True)

    def forward_bin_fuses(self, value, sampling_locations) -> bool:
        """Whether :meth:`ms_deform_attn_forward_bin` stores the backward's
        records from the forward kernel for these shapes (else it runs the
        plain forward and the binning kernels; same results)."""
        batch, spatial, heads, channels = value.shape
        _, queries, _, levels, points, _ = sampling_locations.shape
        return bool(self._raw["ms_deform_attn_forward_bin_fused"](
            _dtype_code(value.dtype), batch, spatial, heads, channels, levels, queries, points))

    def forward_softmax_bin_fuses(self, value, sampling_locations) -> bool:
        """Whether :meth:`ms_deform_attn_forward_softmax_bin` writes the
        probabilities and stores the backward's records from the softmax-fused
        forward kernel for these shapes (else it runs the softmax forward and
        the softmax binning; same results)."""
        batch, spatial, heads, channels = value.shape
        _, queries, _, levels, points, _ = sampling_locations.shape
        return bool(self._raw["ms_deform_attn_forward_softmax_bin_fused"](
            _dtype_code(value.dtype), batch, spatial, heads, channels, levels, queries, points))

    def backward_workspace(self, value, sampling_locations):
        """Scratch of the tile-owned backward for these shapes (1 byte when the
        shape takes the atomic fallback)."""
        import torch

        nbytes = self._workspace_bytes(value, sampling_locations, softmax=False)
        return torch.empty(max(nbytes, 1), dtype=torch.uint8, device=value.device)

    def backward_softmax_workspace(self, value, sampling_locations):
        """Scratch of the softmax backward for these shapes: the probabilities,
        then the tile-owned kernels' scratch when the tile path applies."""
        import torch

        nbytes = self._workspace_bytes(value, sampling_locations, softmax=True)
        return torch.empty(max(nbytes, 1), dtype=torch.uint8, device=value.device)

    def _check_split(self, value, spatial_shapes, level_start_index, sampling_locations,
                     attention_weights, grad_output, grad_value, grad_sampling_locations,
                     grad_attention_weights, workspace, softmax: bool) -> None:
        """Checks of one part of a backward split in two (binning, rest): every
        tensor as :meth:`check_backward`, and a workspace of at least the size
        the shapes need, so both parts take the same path (a smaller one
        would make the binning skip the tile path while the rest expects it)."""
        import torch

        self.check_backward(value, spatial_shapes, level_start_index, sampling_locations,
                            attention_weights, grad_output, grad_value, grad_sampling_locations,
                            grad_attention_weights)
        _check(workspace, "workspace", (torch.uint8,), value.device)
        need = self._workspace_bytes(value, sampling_locations, softmax)
        if workspace.numel() < need:
            raise RuntimeError(f"workspace holds {workspace.numel()} bytes, these shapes need "
                               f"{need}")

    def _backward_call(self, name, value, spatial_shapes, level_start_index, sampling_locations,
                       attention_weights, grad_output, grad_value, grad_sampling_locations,
                       grad_attention_weights, im2col_step, workspace, stream) -> None:
        batch, spatial, heads, channels = value.shape
        levels = spatial_shapes.shape[0]
        queries, points = sampling_locations.shape[1], sampling_locations.shape[4]
        rc = self._raw[name](
            value.data_ptr(), _dtype_code(value.dtype), spatial_shapes.data_ptr(),
            level_start_index.data_ptr(), sampling_locations.data_ptr(),
            attention_weights.data_ptr(), _dtype_code(sampling_locations.dtype),
            None if grad_output is None else grad_output.data_ptr(), grad_value.data_ptr(),
            grad_sampling_locations.data_ptr(), grad_attention_weights.data_ptr(),
            batch, spatial, heads, channels, levels, queries, points,
            int(im2col_step), workspace.data_ptr(), workspace.numel(), stream,
        )
        self._raise_on(rc, name)

    def _split_part(self, name, softmax, value, spatial_shapes, level_start_index,
                    sampling_locations, attention_weights, grad_output, grad_value,
                    grad_sampling_locations, grad_attention_weights, im2col_step, workspace,
                    stream) -> None:
        import torch

        self._check_split(value, spatial_shapes, level_start_index, sampling_locations,
                          attention_weights, grad_output, grad_value, grad_sampling_locations,
                          grad_attention_weights, workspace, softmax)
        st = stream if stream is not None else torch.cuda.current_stream(value.device)
        with torch.cuda.device(value.device):
            self._backward_call(name, value, spatial_shapes, level_start_index,
                                sampling_locations, attention_weights, grad_output, grad_value,
                                grad_sampling_locations, grad_attention_weights, im2col_step,
                                workspace, st.cuda_stream)

    def ms_deform_attn_backward_bin(
        self, value, spatial_shapes, level_start_index, sampling_locations, attention_weights,
        grad_value, grad_sampling_locations, grad_attention_weights, im2col_step, workspace,
        stream=None,
    ) -> None:
        """First part of the backward (binning; geometry only) on ``stream``
        (default: the current stream). Every tensor is checked before the
        launch; :meth:`ms_deform_attn_backward_rest` on the same workspace and
        gradients must follow it on a stream ordered after this one."""
        self._split_part("ms_deform_attn_backward_bin", False, value, spatial_shapes,
                         level_start_index, sampling_locations, attention_weights, None,
                         grad_value, grad_sampling_locations, grad_attention_weights,
                         im2col_step, workspace, stream)

    def ms_deform_attn_backward_rest(
        self, value, spatial_shapes, level_start_index, sampling_locations, attention_weights,
        grad_output, grad_value, grad_sampling_locations, grad_attention_weights, im2col_step,
        workspace,
    ) -> None:
        """Second part of the backward on the current stream, after the binning
        of the same workspace (ordered by the caller)."""
        self._split_part("ms_deform_attn_backward_rest", False, value, spatial_shapes,
                         level_start_index, sampling_locations, attention_weights, grad_output,
                         grad_value, grad_sampling_locations, grad_attention_weights,
                         im2col_step, workspace, None)

    def ms_deform_attn_forward_bin(
        self, value, spatial_shapes, level_start_index, sampling_locations, attention_weights,
        output, grad_value, grad_sampling_locations, grad_attention_weights, im2col_step,
        workspace,
    ) -> None:
        """The forward and the first part of the backward (binning) in one call
        on the current stream: writes ``output`` and bins into ``workspace``,
        as :meth:`ms_deform_attn_forward` followed by
        :meth:`ms_deform_attn_backward_bin` would. Where the tile path applies
        the forward kernel stores the backward's records itself. Every tensor
        is checked before the first launch;
        :meth:`ms_deform_attn_backward_rest` on the same workspace and
        gradients must follow it on a stream ordered after this one."""
        self._forward_bin_call("ms_deform_attn_forward_bin", False, value, spatial_shapes,
                               level_start_index, sampling_locations, attention_weights, output,
                               grad_value, grad_sampling_locations, grad_attention_weights,
                               im2col_step, workspace)

    def ms_deform_attn_forward_softmax_bin(
        self, value, spatial_shapes, level_start_index, sampling_locations, attention_logits,
        output, grad_value, grad_sampling_locations, grad_attention_logits, im2col_step,
        workspace,
    ) -> None:
        """:meth:`ms_deform_attn_forward_softmax` and the first part of its
        backward (:meth:`ms_deform_attn_backward_softmax_bin`) in one call on the
        current stream, on a workspace of :meth:`backward_softmax_workspace`'s
        size; :meth:`ms_deform_attn_backward_softmax_rest` on the same workspace
        and gradients follows it. Where it applies the softmax-fused forward
        kernel writes the probabilities and stores the backward's records itself."""
        self._forward_bin_call("ms_deform_attn_forward_softmax_bin", True, value, spatial_shapes,
                               level_start_index, sampling_locations, attention_logits, output,
                               grad_value, grad_sampling_locations, grad_attention_logits,
                               im2col_step, workspace)

    def _forward_bin_call(
        self, name, softmax, value, spatial_shapes, level_start_index, sampling_locations,
        attention_weights, output, grad_value, grad_sampling_locations, grad_attention_weights,
        im2col_step, workspace,
    ) -> None:
        """One of the forward + binning calls, every tensor and the workspace
        size checked before the launch."""
        import torch

        self.check_forward(value, spatial_shapes, level_start_index, sampling_locations,
                           attention_weights, output)
        self._check_split(value, spatial_shapes, level_start_index, sampling_locations,
                          attention_weights, None, grad_value, grad_sampling_locations,
                          grad_attention_weights, workspace, softmax)
        batch, spatial, heads, channels = value.shape
        levels = spatial_shapes.shape[0]
        queries, points = sampling_locations.shape[1], sampling_locations.shape[4]
        with torch.cuda.device(value.device):
            rc = self._raw[name](
                value.data_ptr(), _dtype_code(value.dtype), spatial_shapes.data_ptr(),
                level_start_index.data_ptr(), sampling_locations.data_ptr(),
                attention_weights.data_ptr(), _dtype_code(sampling_locations.dtype),
                output.data_ptr(), grad_value.data_ptr(), grad_sampling_locations.data_ptr(),
                grad_attention_weights.data_ptr(), batch, spatial, heads, channels, levels,
                queries, points, int(im2col_step), workspace.data_ptr(), workspace.numel(),
                self._stream(value),
            )
        self._raise_on(rc, name)

    def ms_deform_attn_backward_softmax_bin(
        self, value, spatial_shapes, level_start_index, sampling_locations, attention_logits,
        grad_value, grad_sampling_locations, grad_attention_logits, im2col_step, workspace,
        stream=None,
    ) -> None:
        """First part of the softmax backward (probabilities and binning; geometry
        and logits only) on ``stream`` (default: the current stream)."""
        self._split_part("ms_deform_attn_backward_softmax_bin", True, value, spatial_shapes,
                         level_start_index, sampling_locations, attention_logits, None,
                         grad_value, grad_sampling_locations, grad_attention_logits,
                         im2col_step, workspace, stream)

    def ms_deform_attn_backward_softmax_rest(
        self, value, spatial_shapes, level_start_index, sampling_locations, attention_logits,
        grad_output, grad_value, grad_sampling_locations, grad_attention_logits, im2col_step,
        workspace,
    ) -> None:
        """Second part of the softmax backward on the current stream."""
        self._split_part("ms_deform_attn_backward_softmax_rest", True, value, spatial_shapes,
                         level_start_index, sampling_locations, attention_logits, grad_output,
                         grad_value, grad_sampling_locations, grad_attention_logits,
                         im2col_step, workspace, None)

    def ms_deform_attn_forward_scatter_div(
        self, value, spatial_shapes, level_start_index, sampling_locations,
        attention_weights, index, count, slots, num_cams: int, cam_id: int,
    ) -> None:
        """One camera of the spatial cross-attention, added into ``slots`` in place.

        value ``[bs*num_cams, nv, M, C]``, sampling_locations
        ``[bs*num_cams, max_len, M, L, P, 2]``, attention_weights
        ``[bs*num_cams, max_len, M, L, P]``, index ``[valid_len]`` int64 (the BEV
        query of each of the camera's first valid_len rows), count
        ``[bs, num_query]`` and slots ``[bs, num_query, M*C]``. Argument order of
        the reference's ``ms_deformable_im2col_scatter_div_musa``
        (/root/reference/csrc/ms_deformable_attn/ms_deform_attn_musa.mu:455-505).
        """
        import torch

        half = (torch.float32, torch.float16, torch.bfloat16)
        _check(value, "value", half)
        _check(spatial_shapes, "spatial_shapes", (torch.int64,))
        _check(level_start_index, "level_start_index", (torch.int64,))
        geom = (torch.float32,) if value.dtype == torch.float32 else (torch.float32, value.dtype)
        _check(sampling_locations, "sampling_locations", geom)
        _check(attention_weights, "attention_weights", (sampling_locations.dtype,))
        _check(index, "index", (torch.int64,))
        _check(count, "count", (sampling_locations.dtype,))
        _check(slots, "slots", (value.dtype,))
        if value.dim() != 4 or sampling_locations.dim() != 6 or index.dim() != 1:
            raise RuntimeError("value must be 4-D, sampling_locations 6-D and index 1-D")
        if slots.dim() != 3:
            raise RuntimeError("slots must be 3-D [batch, num_query, num_heads*channels]")
        rows, spatial, heads, channels = value.shape
        if num_cams <= 0 or rows % num_cams != 0:
            raise RuntimeError(f"value rows {rows} are not a multiple of num_cams {num_cams}")
        batch, num_query = rows // num_cams, slots.shape[1]
        levels = spatial_shapes.shape[0]
        max_len, points = sampling_locations.shape[1], sampling_locations.shape[4]
        valid_len = index.shape[0]
        _check_shape(spatial_shapes, "spatial_shapes", (levels, 2))
        _check_shape(level_start_index, "level_start_index", (levels,))
        _check_shape(sampling_locations, "sampling_locations",
                     (rows, max_len, heads, levels, points, 2))
        _check_shape(attention_weights, "attention_weights", (rows, max_len, heads, levels, points))
        _check_shape(count, "count", (batch, num_query))
        _check_shape(slots, "slots", (batch, num_query, heads * channels))
        with torch.cuda.device(value.device):
            rc = self._raw["ms_deform_attn_forward_scatter_div"](
                value.data_ptr(), _dtype_code(value.dtype), spatial_shapes.data_ptr(),
                level_start_index.data_ptr(), sampling_locations.data_ptr(),
                attention_weights.data_ptr(), _dtype_code(sampling_locations.dtype),
                index.data_ptr(), count.data_ptr(), slots.data_ptr(), batch, num_cams,
                int(cam_id), valid_len, spatial, heads, channels, levels, max_len, points,
                num_query, self._stream(value),
            )
        self._raise_on(rc, "ms_deform_attn_forward_scatter_div")

    def ms_deform_attn_forward_scatter_div_cams(
        self, value, spatial_shapes, level_start_index, sampling_locations,
        attention_weights, index, valid_lens, count, slots,
    ) -> None:
        """Every camera of the spatial cross-attention added into ``slots`` in place.

        As :meth:`ms_deform_attn_forward_scatter_div` for cameras 0..num_cams-1,
        with ``index`` the cameras' BEV ids concatenated and ``valid_lens`` (a
        sequence of ints, one per camera) their lengths.
        """
        import torch

        half = (torch.float32, torch.float16, torch.bfloat16)
        _check(value, "value", half)
        _check(spatial_shapes, "spatial_shapes", (torch.int64,))
        _check(level_start_index, "level_start_index", (torch.int64,))
        geom = (torch.float32,) if value.dtype == torch.float32 else (torch.float32, value.dtype)
        _check(sampling_locations, "sampling_locations", geom)
        _check(attention_weights, "attention_weights", (sampling_locations.dtype,))
        _check(index, "index", (torch.int64,))
        _check(count, "count", (sampling_locations.dtype,))
        _check(slots, "slots", (value.dtype,))
        if value.dim() != 4 or sampling_locations.dim() != 6 or index.dim() != 1:
            raise RuntimeError("value must be 4-D, sampling_locations 6-D and index 1-D")
        if slots.dim() != 3:
            raise RuntimeError("slots must be 3-D [batch, num_query, num_heads*channels]")
        lens = [int(n) for n in valid_lens]
        num_cams = len(lens)
        rows, spatial, heads, channels = value.shape
        if num_cams <= 0 or rows % num_cams != 0:
            raise RuntimeError(f"value rows {rows} are not a multiple of num_cams {num_cams}")
        if sum(lens) != index.shape[0]:
            raise RuntimeError(
                f"index has {index.shape[0]} entries, valid_lens sum to {sum(lens)}")
        batch, num_query = rows // num_cams, slots.shape[1]
        levels = spatial_shapes.shape[0]
        max_len, points = sampling_locations.shape[1], sampling_locations.shape[4]
        _check_shape(spatial_shapes, "spatial_shapes", (levels, 2))
        _check_shape(level_start_index, "level_start_index", (levels,))
        _check_shape(sampling_locations, "sampling_locations",
                     (rows, max_len, heads, levels, points, 2))
        _check_shape(attention_weights, "attention_weights", (rows, max_len, heads, levels, points))
        _check_shape(count, "count", (batch, num_query))
        _check_shape(slots, "slots", (batch, num_query, heads * channels))
        host_lens = (ctypes.c_int64 * num_cams)(*lens)
        with torch.cuda.device(value.device):
            rc = self._raw["ms_deform_attn_forward_scatter_div_cams"](
                value.data_ptr(), _dtype_code(value.dtype), spatial_shapes.data_ptr(),
                level_start_index.data_ptr(), sampling_locations.data_ptr(),
                attention_weights.data_ptr(), _dtype_code(sampling_locations.dtype),
                index.data_ptr(), ctypes.cast(host_lens, ctypes.c_void_p), count.data_ptr(),
                slots.data_ptr(), batch, num_cams, spatial, heads, channels, levels, max_len,
                points, num_query, self._stream(value),
            )
        self._raise_on(rc, "ms_deform_attn_forward_scatter_div_cams")

    def ms_deform_attn_scatter_div_grad(
        self, grad_slots, index, valid_lens, count, grad_output,
    ) -> None:
        """grad_output ``[bs*num_cams, max_len, row]`` from grad_slots ``[bs,
        num_query, row]``: camera c's row r gets ``grad_slots[b, q] / count[b, q]``
        (q its BEV id in the concatenated ``index``) for r < valid_lens[c], zero
        past it."""
        import torch

        half = (torch.float32, torch.float16, torch.bfloat16)
        _check(grad_slots, "grad_slots", half)
        _check(index, "index", (torch.int64,))
        geom = (torch.float32,) if grad_slots.dtype == torch.float32 else (
            torch.float32, grad_slots.dtype)
        _check(count, "count", geom)
        _check(grad_output, "grad_output", (grad_slots.dtype,))
        if grad_slots.dim() != 3 or grad_output.dim() != 3 or index.dim() != 1:
            raise RuntimeError("grad_slots and grad_output must be 3-D and index 1-D")
        lens = [int(n) for n in valid_lens]
        num_cams = len(lens)
        if num_cams <= 0 or sum(lens) != index.shape[0]:
            raise RuntimeError(
                f"index has {index.shape[0]} entries, valid_lens sum to {sum(lens)}")
        batch, num_query, row = grad_slots.shape
        max_len = grad_output.shape[1]
        _check_shape(grad_output, "grad_output", (batch * num_cams, max_len, row))
        _check_shape(count, "count", (batch, num_query))
        host_lens = (ctypes.c_int64 * num_cams)(*lens)
        with torch.cuda.device(grad_slots.device):
            rc = self._raw["ms_deform_attn_scatter_div_grad"](
                grad_slots.data_ptr(), _dtype_code(grad_slots.dtype), index.data_ptr(),
                ctypes.cast(host_lens, ctypes.c_void_p), count.data_ptr(),
                _dtype_code(count.dtype), grad_output.data_ptr(), batch, num_cams, max_len,
                num_query, row, self._stream(grad_slots),
            )
        self._raise_on(rc, "ms_deform_attn_scatter_div_grad")

    # ------------------------------------------------ deformable aggregation ---
    @staticmethod
    def _dfa_dims(mc_ms_feat, spatial_shape, scale_start_index, sampling_location, weights):
        """Checks of the reference's validate() (deformable_aggregation_musa.mu:669-679)
        and the dims its launchers read (:660-668)."""
        import torch

        _check(mc_ms_feat, "mc_ms_feat", (torch.float32,))
        _check(spatial_shape, "spatial_shape", (torch.int32,))
        _check(scale_start_index, "scale_start_index", (torch.int32,))
        _check(sampling_location, "sampling_location", (torch.float32,))
        _check(weights, "weights", (torch.float32,))
        if (mc_ms_feat.dim() != 3 or spatial_shape.dim() != 3 or sampling_location.dim() != 5
                or weights.dim() != 6):
            raise RuntimeError("mc_ms_feat must be 3-D, spatial_shape 3-D, sampling_location "
                               "5-D and weights 6-D")
        batch, num_feat, num_embeds = mc_ms_feat.shape
        num_cams, num_scale = spatial_shape.shape[0], spatial_shape.shape[1]
        num_anchors, num_pts = sampling_location.shape[1], sampling_location.shape[2]
        num_groups = weights.shape[5]
        _check_shape(spatial_shape, "spatial_shape", (num_cams, num_scale, 2))
        _check_shape(scale_start_index, "scale_start_index", (num_cams, num_scale))
        _check_shape(sampling_location, "sampling_location",
                     (batch, num_anchors, num_pts, num_cams, 2))
        _check_shape(weights, "weights",
                     (batch, num_anchors, num_pts, num_cams, num_scale, num_groups))
        return (batch, num_cams, num_feat, num_embeds, num_scale, num_anchors, num_pts,
                num_groups)

    def _dfa_forward(self, name, mc_ms_feat, spatial_shape, scale_start_index,
                     sampling_location, weights, output) -> None:
        import torch

        dims = self._dfa_dims(mc_ms_feat, spatial_shape, scale_start_index, sampling_location,
                              weights)
        _check(output, "out", (torch.float32,))
        _check_shape(output, "out", (dims[0], dims[5], dims[3]))
        with torch.cuda.device(mc_ms_feat.device):
            rc = self._raw[name](
                mc_ms_feat.data_ptr(), spatial_shape.data_ptr(), scale_start_index.data_ptr(),
                sampling_location.data_ptr(), weights.data_ptr(), output.data_ptr(), *dims,
                self._stream(mc_ms_feat),
            )
        self._raise_on(rc, name)

    def _dfa_backward(self, name, mc_ms_feat, spatial_shape, scale_start_index,
                      sampling_location, weights, grad_output, grad_mc_ms_feat,
                      grad_sampling_location, grad_weights) -> None:
        import torch

        dims = self._dfa_dims(mc_ms_feat, spatial_shape, scale_start_index, sampling_location,
                              weights)
        for tensor, label, like in (
            (grad_output, "grad_output", (dims[0], dims[5], dims[3])),
            (grad_mc_ms_feat, "grad_mc_ms_feat", tuple(mc_ms_feat.shape)),
            (grad_sampling_location, "grad_sampling_location", tuple(sampling_location.shape)),
            (grad_weights, "grad_weights", tuple(weights.shape)),
        ):
            _check(tensor, label, (torch.float32,))
            _check_shape(tensor, label, like)
        with torch.cuda.device(mc_ms_feat.device):
            rc = self._raw[name](
                mc_ms_feat.data_ptr(), spatial_shape.data_ptr(), scale_start_index.data_ptr(),
                sampling_location.data_ptr(), weights.data_ptr(), grad_output.data_ptr(),
                grad_mc_ms_feat.data_ptr(), grad_sampling_location.data_ptr(),
                grad_weights.data_ptr(), *dims, self._stream(mc_ms_feat),
            )
        self._raise_on(rc, name)

    def deformable_aggregation_forward_opt(self, mc_ms_feat, spatial_shape, scale_start_index,
                                           sampling_location, weights, output) -> None:
        """output += aggregation (reference argument order, deformable_aggregation_musa.mu:717)."""
        self._dfa_forward("deformable_aggregation_forward_opt", mc_ms_feat, spatial_shape,
                          scale_start_index, sampling_location, weights, output)

    def deformable_aggregation_forward_base(self, mc_ms_feat, spatial_shape, scale_start_index,
                                            sampling_location, weights, output) -> None:
        self._dfa_forward("deformable_aggregation_forward_base", mc_ms_feat, spatial_shape,
                          scale_start_index, sampling_location, weights, output)

    def deformable_aggregation_backward_opt(self, mc_ms_feat, spatial_shape, scale_start_index,
                                            sampling_location, weights, grad_output,
                                            grad_mc_ms_feat, grad_sampling_location,
                                            grad_weights) -> None:
        """grad_mc_ms_feat += ...; location and weight gradients written
        (reference argument order, deformable_aggregation_musa.mu:725)."""
        self._dfa_backward("deformable_aggregation_backward_opt", mc_ms_feat, spatial_shape,
                           scale_start_index, sampling_location, weights, grad_output,
                           grad_mc_ms_feat, grad_sampling_location, grad_weights)

    def deformable_aggregation_backward_base(self, mc_ms_feat, spatial_shape,
                                             scale_start_index, sampling_location, weights,
                                             grad_output, grad_mc_ms_feat,
                                             grad_sampling_location, grad_weights) -> None:
        self._dfa_backward("deformable_aggregation_backward_base", mc_ms_feat, spatial_shape,
                           scale_start_index, sampling_location, weights, grad_output,
                           grad_mc_ms_feat, grad_sampling_location, grad_weights)

    def add_one(self, value, actual) -> None:
        """Build smoke: actual = value + 1 (float32 device tensors)."""
        import torch

        _check(value, "value", (torch.float32,))
        _check(actual, "actual", (torch.float32,))
        if value.numel() != actual.numel():
            raise RuntimeError("value and actual must have the same number of elements")
        with torch.cuda.device(value.device):
            rc = self._raw["add_one"](
                value.data_ptr(), actual.data_ptr(), value.numel(), self._stream(value)
            )
        self._raise_on(rc, "add_one")


@lru_cache(maxsize=1)
def load_native_module() -> NativeLibrary:
    # torch first: its bundled HIP runtime then satisfies the library's
    # libamdhip64.so.7 dependency, so both share one runtime, device context
    # and stream namespace.
    import torch  # noqa: F401

    library = library_path()
    if not library.is_file():
        raise NativeModuleUnavailable(
            f"muSPACE native library is missing from this installation ({library}); "
            "build it with `python -m muspace_amd.build`."
        )
    try:
        handle = ctypes.CDLL(str(library))
    except OSError as exc:
        raise NativeModuleUnavailable(
            f"unable to load muSPACE native library {library}: {exc}"
        ) from exc
    return NativeLibrary(handle, library)


def native_function(name: str) -> Callable[..., Any]:
    return load_native_module().function(name)


class NativeModuleProxy:
    """Attribute-compatible view used by the operator wrappers."""

    def __getattr__(self, name: str) -> Any:
        if name.startswith("__"):
            raise AttributeError(name)
        return native_function(name)


@lru_cache(maxsize=1)
def native_module_proxy() -> NativeModuleProxy:
    load_native_module()
    return NativeModuleProxy()


def native_available() -> bool:
    try:
        load_native_module()
    except NativeModuleUnavailable:
        return False
    return True


def native_error() -> str | None:
    try:
        load_native_module()
    except NativeModuleUnavailable as exc:
        return str(exc)
    return None
