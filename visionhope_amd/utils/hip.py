"""ctypes binding of ``libvisionhope_hip.so`` (C ABI in ``include/visionhope_hip.h``).

The Python modules of this package pass ``tensor.data_ptr()`` and the current
HIP stream of the tensor's device to the library; the library never allocates,
so every output and workspace below is a torch tensor from the caching
allocator.  If the library is missing, every GPU entry point raises: there is
no CPU or PyTorch fallback for GPU tensors.
"""

from __future__ import annotations

import contextlib
import ctypes
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parents[1] / "_lib" / "libvisionhope_hip.so"

VH_OK = 0
VH_ERR_SHAPE, VH_ERR_DTYPE, VH_ERR_HEAD_DIM, VH_ERR_WORKSPACE, VH_ERR_ARG, VH_ERR_LAUNCH = range(1, 7)
VH_DTYPE_F32, VH_DTYPE_BF16, VH_DTYPE_F16 = 0, 1, 2

_DTYPE_CODES = {torch.float32: VH_DTYPE_F32, torch.bfloat16: VH_DTYPE_BF16, torch.float16: VH_DTYPE_F16}

# Symbols declared in include/visionhope_hip.h (tests check the library exports all of them).
EXPORTED_SYMBOLS = (
    "vh_abi_version", "vh_last_error", "vh_set_dispatch_override", "vh_clear_dispatch_overrides",
    "vh_grn_workspace_fallbacks", "vh_stream_capture_id", "vh_srnl_workspace_bytes", "vh_srnl_spatial_forward",
    "vh_srnl_spatial_forward_noalloc",
    "vh_srnl_spatial_scan", "vh_srnl_spatial_readout", "vh_srnl_spatial_readout_lepe",
    "vh_srnl_line_forward_seq_noatomic", "vh_srnl_sequence_forward", "vh_srnl_forward",
    "vh_postprocess_scale_forward", "vh_grn_workspace_bytes", "vh_grn_forward",
    "vh_layernorm2d_forward", "vh_add_layernorm2d_forward", "vh_qnorm_forward", "vh_residual_add_forward",
    "vh_dwconv2d_nhwc_forward", "vh_dwconv2d_add_layernorm2d_forward", "vh_grn_scale_forward", "vh_pointwise_add_layernorm_nhwc_forward", "vh_pointwise_chain_nhwc_forward", "vh_pointwise_conv_nhwc_forward",
    "vh_bias_act_nhwc_forward", "vh_dwconv2d_gelu_grn_workspace_bytes", "vh_dwconv2d_gelu_grn_forward",
    "vh_conv3x3_nhwc_forward", "vh_srnl_backward_workspace_bytes", "vh_srnl_backward",
    "vh_postprocess_scale_backward_workspace_bytes", "vh_postprocess_scale_backward",
    "vh_grn_backward_workspace_bytes", "vh_grn_backward", "vh_layernorm2d_backward_workspace_bytes",
    "vh_layernorm2d_backward", "vh_qnorm_backward", "vh_residual_add_backward_workspace_bytes",
    "vh_residual_add_backward",
)


class SRNLConsts(ctypes.Structure):
    """``vh_srnl_consts``."""

    _fields_ = [
        ("step_scale", ctypes.c_float),
        ("min_retention", ctypes.c_float),
        ("retention_bias", ctypes.c_float),
        ("injection_margin", ctypes.c_float),
        ("spectral_clamp", ctypes.c_int32),
        ("spectral_factor", ctypes.c_float),
    ]


_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32
_f32 = ctypes.c_float
_sz = ctypes.c_size_t
_I64P = ctypes.POINTER(ctypes.c_int64)
_CP = ctypes.POINTER(SRNLConsts)

_SIGNATURES = {
    "vh_abi_version": (ctypes.c_int, []),
    "vh_last_error": (ctypes.c_char_p, []),
    "vh_set_dispatch_override": (ctypes.c_int, [ctypes.c_char_p, ctypes.c_char_p]),
    "vh_clear_dispatch_overrides": (None, []),
    "vh_grn_workspace_fallbacks": (ctypes.c_int, [_vp, _sz, _vp, ctypes.POINTER(ctypes.c_int64)]),
    "vh_stream_capture_id": (ctypes.c_int, [_vp, ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(ctypes.c_uint64)]),
    "vh_srnl_workspace_bytes": (_sz, [_i64, _i64, _i32]),
    "vh_srnl_spatial_forward": (ctypes.c_int, [
        _vp, _vp, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _vp, _vp,
        _i64, _i64, _i64, _i64, _i32, _I64P, _CP, _vp, _sz, _vp]),
    "vh_srnl_spatial_forward_noalloc": (ctypes.c_int, [
        _vp, _vp, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _vp, _vp,
        _i64, _i64, _i64, _i64, _i32, _I64P, _CP, _vp]),
    "vh_srnl_spatial_scan": (ctypes.c_int, [
        _vp, _i32, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i32, _I64P, _CP, _vp, _sz, _vp]),
    "vh_srnl_spatial_readout": (ctypes.c_int, [
        _vp, _vp, _i32, _vp, _i32, _vp, _vp, _vp, _i32, _i64, _i64, _i64, _i64, _i32, _I64P, _vp, _sz, _vp]),
    "vh_srnl_spatial_readout_lepe": (ctypes.c_int, [
        _vp, _vp, _i32, _vp, _i32, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i32, _I64P, _vp, _sz, _vp]),
    "vh_srnl_backward_workspace_bytes": (_sz, [_i64, _i64, _i64, _i64, _i32, _I64P]),
    "vh_srnl_backward": (ctypes.c_int, [
        _vp, _vp, _i32, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
        _i64, _i64, _i64, _i64, _i32, _I64P, _CP, _vp, _sz, _vp]),
    "vh_postprocess_scale_backward_workspace_bytes": (_sz, [_i64, _i64, _i64, _i64, _i32, _i32]),
    "vh_postprocess_scale_backward": (ctypes.c_int, [
        _vp, _i32, _vp, _vp, _i32, _vp, _i32, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i32, _vp, _sz, _vp]),
    "vh_grn_backward_workspace_bytes": (_sz, [_i64, _i64, _i64, _i64]),
    "vh_grn_backward": (ctypes.c_int, [
        _vp, _vp, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _vp, _sz, _vp]),
    "vh_layernorm2d_backward_workspace_bytes": (_sz, [_i64, _i64, _i64, _i64]),
    "vh_layernorm2d_backward": (ctypes.c_int, [
        _vp, _vp, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _vp, _sz, _vp]),
    "vh_residual_add_backward_workspace_bytes": (_sz, [_i64, _i64]),
    "vh_residual_add_backward": (ctypes.c_int, [
        _vp, _vp, _i32, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp, _sz, _vp]),
    "vh_qnorm_backward": (ctypes.c_int, [_vp, _vp, _vp, _vp, _i32, _i64, _i64, _i64, _i64, _i32, _vp]),
    "vh_srnl_line_forward_seq_noatomic": (ctypes.c_int, [
        _vp, _vp, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _vp, _vp,
        _i64, _i64, _i64, _i64, _i32, _CP, _vp, _sz, _vp]),
    "vh_srnl_sequence_forward": (ctypes.c_int, [
        _vp, _vp, _i32, _vp, _vp, _vp, _vp, _vp, _i32, _vp,
        _i64, _i64, _i64, _i64, _i32, _I64P, _CP, _vp, _sz, _vp]),
    "vh_srnl_forward": (ctypes.c_int, [
        _vp, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _vp,
        _i64, _i64, _i64, _i64, _i32, _I64P, _CP, _vp, _sz, _vp]),
    "vh_postprocess_scale_forward": (ctypes.c_int, [
        _vp, _vp, _i32, _vp, _i32, _vp, _vp, _i64, _i64, _i64, _i64, _i32, _i32, _vp]),
    "vh_grn_workspace_bytes": (_sz, [_i64, _i64, _i64, _i64]),
    "vh_grn_forward": (ctypes.c_int, [
        _vp, _i32, _vp, _vp, _vp, _i32, _vp, _vp, _i64, _i64, _i64, _i64, _f32, _vp, _sz, _vp]),
    "vh_layernorm2d_forward": (ctypes.c_int, [
        _vp, _i32, _vp, _vp, _vp, _i32, _vp, _vp, _i64, _i64, _i64, _i64, _f32, _i32, _vp]),
    "vh_add_layernorm2d_forward": (ctypes.c_int, [
        _vp, _vp, _i32, _vp, _vp, _vp, _vp, _i32, _i64, _i64, _i64, _i64, _f32, _vp]),
    "vh_dwconv2d_nhwc_forward": (ctypes.c_int, [
        _vp, _i32, _vp, _vp, _i32, _i32, _vp, _vp, _i64, _i64, _i64, _i64, _vp]),
    "vh_dwconv2d_add_layernorm2d_forward": (ctypes.c_int, [
        _vp, _i32, _vp, _vp, _i32, _vp, _vp, _f32, _vp, _vp, _i64, _i64, _i64, _i64, _vp]),
    "vh_grn_scale_forward": (ctypes.c_int, [
        _vp, _i32, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _f32, _vp, _sz, _vp]),
    "vh_pointwise_conv_nhwc_forward": (ctypes.c_int, [
        _vp, _i32, _vp, _vp, _i32, _vp, _vp, _vp, _i64, _vp, _i64, _i64, _i64, _vp]),
    "vh_pointwise_chain_nhwc_forward": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp]),
    "vh_pointwise_add_layernorm_nhwc_forward": (ctypes.c_int, [
        _vp, _vp, _vp, _vp, _vp, _vp, ctypes.c_float, _vp, _vp, _i64, _i64, _i64, _vp]),
    "vh_bias_act_nhwc_forward": (ctypes.c_int, [_vp, _i32, _vp, _i32, _vp, _i64, _i64, _vp]),
    "vh_conv3x3_nhwc_forward": (ctypes.c_int, [
        _vp, _i32, _vp, _vp, _i32, _vp, _i64, _i64, _i64, _i64, _i64, _i32, _vp]),
    "vh_dwconv2d_gelu_grn_workspace_bytes": (_sz, [_i64, _i64, _i64, _i64, _i32]),
    "vh_dwconv2d_gelu_grn_forward": (ctypes.c_int, [
        _vp, _i32, _vp, _vp, _i32, _vp, _f32, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _vp, _sz, _vp]),
    "vh_qnorm_forward": (ctypes.c_int, [_vp, _i32, _vp, _vp, _i64, _i64, _i64, _i64, _i32, _vp]),
    "vh_residual_add_forward": (ctypes.c_int, [
        _vp, _i32, _vp, _i32, _vp, _vp, _vp, _i64, _i64, _i64, _vp]),
}

_LIB = None


class NativeLibraryMissing(RuntimeError):
    """Raised when a GPU entry point is used but libvisionhope_hip.so is not built."""


def load_library(path: Path | str | None = None):
    """Load (once) and return the ctypes handle with argument types installed."""
    global _LIB
    if _LIB is not None and path is None:
        return _LIB
    lib_path = Path(path) if path is not None else LIB_PATH
    if not lib_path.exists():
        raise NativeLibraryMissing(
            f"{lib_path} is not built; run `python -c 'import __graft_entry__ as g; g.build()'` "
            "(hipcc, gfx950). VisionHOPE GPU kernels have no fallback.")
    lib = ctypes.CDLL(str(lib_path))
    for name, (restype, argtypes) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    if path is None:
        _LIB = lib
    return lib


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_CODES[dtype]
    except KeyError:
        raise TypeError(f"VisionHOPE kernels support FP16, BF16 and FP32 tensors, got {dtype}") from None


def stream_of(tensor: torch.Tensor):
    """Current HIP stream of the tensor's device, as a void*."""
    return ctypes.c_void_p(torch.cuda.current_stream(tensor.device).cuda_stream)


def ptr(tensor):
    return ctypes.c_void_p(tensor.data_ptr()) if tensor is not None else None


def check(rc: int, what: str):
    if rc != VH_OK:
        message = load_library().vh_last_error().decode(errors="replace")
        if rc == VH_ERR_DTYPE:
            raise TypeError(f"{what}: {message}")
        raise RuntimeError(f"{what}: {message} (status {rc})")


def int64_array(values):
    arr = (ctypes.c_int64 * len(values))(*[int(v) for v in values])
    return ctypes.cast(arr, _I64P), arr


def make_consts(step_scale, min_retention, retention_bias, injection_margin, spectral_clamp,
                spectral_margin) -> SRNLConsts:
    return SRNLConsts(float(step_scale), float(min_retention), float(retention_bias),
                      float(injection_margin), int(bool(spectral_clamp)), float(2.0 * spectral_margin))


def workspace(nbytes: int, device) -> torch.Tensor:
    """Workspace tensor of at least ``nbytes`` (fp32 elements, 256-byte granule)."""
    return torch.empty(max(1, (int(nbytes) + 255) // 256 * 64), dtype=torch.float32, device=device)


@contextlib.contextmanager
def dispatch_override(**values):
    """Force kernel choices of the library for the calls inside the block, e.g.
    ``with dispatch_override(scan_pack="2x2"): ...`` (names and values: the
    ``vh_set_dispatch_override`` comment of ``include/visionhope_hip.h``).  For tests and
    measurements: by default every entry point chooses from its arguments alone.  The
    overrides are process-wide and are cleared on exit."""
    lib = load_library()
    try:
        for name, value in values.items():
            check(lib.vh_set_dispatch_override(name.encode(), str(value).encode()), "vh_set_dispatch_override")
        yield
    finally:
        for name in values:
            lib.vh_set_dispatch_override(name.encode(), None)
