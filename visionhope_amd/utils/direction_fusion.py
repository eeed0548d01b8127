"""Restore and fuse directional SRNL outputs (mirrors ``utils/direction_fusion.py``).

    out = sum_d scale[d] * (y[d] + d_skip[d] * x[d])

y and x are the packed serialized scans ``[B, 4, heads, H*W, head_dim]``; the
native kernel restores each scan to image order and writes FP32
``[B, C, H, W]`` (NCHW or channels-last storage).
"""
import torch

from . import hip
from .autograd import backward_unavailable
from .cuda import on_tensor_device


class VisionHOPEPostprocessScaleFunction(torch.autograd.Function):
    @staticmethod
    @on_tensor_device
    def forward(ctx, y, x, d_skip, direction_scale, height, width, channels_last):
        if not y.is_cuda:
            raise RuntimeError("Fused SRNL postprocess requires CUDA tensors.")
        y_c = y.contiguous()
        x_c = x.contiguous()
        batch, _, heads, length, head_dim = y_c.shape
        channels = heads * head_dim
        skip = d_skip.detach().float().contiguous()
        scale = direction_scale.detach().float().contiguous()
        if skip.numel() not in (channels, 4 * channels):
            raise RuntimeError("d_skip must contain C or 4*C values")
        if int(height) * int(width) != length or scale.shape != (4, channels) or x_c.shape != y_c.shape:
            raise RuntimeError("Invalid shape for visionhope_postprocess_scale_forward.")
        if channels_last:
            out = torch.empty_strided((batch, channels, height, width),
                                      (height * width * channels, 1, width * channels, channels),
                                      device=y.device, dtype=torch.float32)
        else:
            out = torch.empty((batch, channels, height, width), device=y.device, dtype=torch.float32)
        lib = hip.load_library()
        hip.check(lib.vh_postprocess_scale_forward(
            hip.ptr(y_c), hip.ptr(x_c), hip.dtype_code(y_c.dtype), hip.ptr(skip),
            int(skip.numel() == 4 * channels), hip.ptr(scale), hip.ptr(out), batch, heads,
            int(height), int(width), head_dim, int(bool(channels_last)), hip.stream_of(y_c)),
            "vh_postprocess_scale_forward")
        return out

    @staticmethod
    def backward(ctx, d_out):
        backward_unavailable("direction fusion")


def can_fuse_scale_postprocess(y, x, d_skip, direction_scale, height, width):
    """Reference eligibility test (``utils/direction_fusion.py:122-139``)."""
    if direction_scale is None:
        return False
    if not (y.is_cuda and x.is_cuda and d_skip.is_cuda and direction_scale.is_cuda):
        return False
    if any(tensor.device != y.device for tensor in (x, d_skip, direction_scale)):
        return False
    if y.dtype not in (torch.float16, torch.bfloat16, torch.float32) or x.dtype != y.dtype:
        return False
    if d_skip.dtype != torch.float32 or direction_scale.dtype != torch.float32:
        return False
    if y.dim() != 5 or x.shape != y.shape or y.shape[1] != 4:
        return False
    if tuple(d_skip.shape) not in ((y.shape[2], y.shape[4]), (4, y.shape[2], y.shape[4])):
        return False
    if tuple(direction_scale.shape) != (4, y.shape[2] * y.shape[4]):
        return False
    return int(height) * int(width) == int(y.shape[3])


def visionhope_postprocess_scale(y, x, d_skip, direction_scale, height, width, channels_last=False):
    return VisionHOPEPostprocessScaleFunction.apply(
        y, x, d_skip, direction_scale, int(height), int(width), bool(channels_last))
