"""Restore and fuse directional SRNL outputs (mirrors ``utils/direction_fusion.py``).

    out = sum_d scale[d] * (y[d] + d_skip[d] * x[d])

y and x are the packed serialized scans ``[B, 4, heads, H*W, head_dim]``; the
native kernel restores each scan to image order and writes FP32
``[B, C, H, W]`` (NCHW or channels-last storage).
"""
import torch

from . import hip
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
        ctx.save_for_backward(y_c, x_c, skip, scale)
        ctx.dims = (batch, heads, int(height), int(width), head_dim)
        ctx.shapes = (d_skip.shape, direction_scale.shape)
        return out

    @staticmethod
    @on_tensor_device
    def backward(ctx, d_out):
        """Reference ``utils/direction_fusion.py:108-120``: dy, dx in the dtype of y, x;
        FP32 gradients of d_skip and direction_scale in their shapes."""
        y, x, skip, scale = ctx.saved_tensors
        batch, heads, height, width, head_dim = ctx.dims
        g = d_out.float()
        channels_last = g.is_contiguous(memory_format=torch.channels_last) and not g.is_contiguous()
        g = g.contiguous(memory_format=torch.channels_last) if channels_last else g.contiguous()
        per_dir = int(skip.numel() == 4 * heads * head_dim)
        dy = torch.empty_like(y)
        dx = torch.empty_like(x)
        d_skip = torch.empty(skip.shape, device=y.device, dtype=torch.float32)
        d_scale = torch.empty(scale.shape, device=y.device, dtype=torch.float32)
        lib = hip.load_library()
        ws = hip.workspace(lib.vh_postprocess_scale_backward_workspace_bytes(batch, heads, height, width, head_dim,
                                                                             per_dir), y.device)
        hip.check(lib.vh_postprocess_scale_backward(
            hip.ptr(g), int(channels_last), hip.ptr(y), hip.ptr(x), hip.dtype_code(y.dtype), hip.ptr(skip), per_dir,
            hip.ptr(scale), hip.ptr(dy), hip.ptr(dx), hip.ptr(d_skip), hip.ptr(d_scale), batch, heads, height, width,
            head_dim, hip.ptr(ws), ws.numel() * 4, hip.stream_of(y)), "vh_postprocess_scale_backward")
        skip_shape, scale_shape = ctx.shapes
        return dy, dx, d_skip.view(skip_shape), d_scale.view(scale_shape), None, None, None


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
