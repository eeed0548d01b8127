"""Native LayerNorm over channels for NCHW feature maps (replaces the Triton kernel of
``utils/layer_norm_cuda.py``).

Per pixel: mean, biased centred variance, ``y = (x - mean) * rstd * w + b``, FP32
output in the input's storage order (channels-last or NCHW).
"""
import torch
from torch.autograd import Function

from . import hip
from .cuda import on_tensor_device


class _VisionHOPELayerNorm2dFunction(Function):
    @staticmethod
    @on_tensor_device
    def forward(ctx, x, weight, bias, eps, force_channels_last=False, out_dtype=torch.float32):
        batch, channels, height, width = x.shape
        channels_last = x.is_contiguous(memory_format=torch.channels_last)
        if force_channels_last and not channels_last:
            x = x.contiguous(memory_format=torch.channels_last)
            channels_last = True
        elif not channels_last and not x.is_contiguous():
            x = x.contiguous()
        fmt = torch.channels_last if channels_last else torch.contiguous_format
        weight_shape, bias_shape = weight.shape, bias.shape
        weight = weight.detach().reshape(-1).float().contiguous()
        bias = bias.detach().reshape(-1).float().contiguous()
        y = torch.empty_like(x, dtype=out_dtype, memory_format=fmt)
        keep = ctx.needs_input_grad[0] or ctx.needs_input_grad[1] or ctx.needs_input_grad[2]
        rows = batch * height * width
        mean = torch.empty(rows, device=x.device, dtype=torch.float32) if keep else None
        rstd = torch.empty(rows, device=x.device, dtype=torch.float32) if keep else None
        lib = hip.load_library()
        hip.check(lib.vh_layernorm2d_forward(
            hip.ptr(x), hip.dtype_code(x.dtype), hip.ptr(weight), hip.ptr(bias), hip.ptr(y),
            hip.dtype_code(out_dtype), hip.ptr(mean), hip.ptr(rstd), batch, channels, height, width, float(eps),
            int(channels_last),
            hip.stream_of(x)), "vh_layernorm2d_forward")
        if keep:
            ctx.save_for_backward(x, weight, mean, rstd)
            ctx.param_shapes = (weight_shape, bias_shape)
        return y

    @staticmethod
    @on_tensor_device
    def backward(ctx, dy):
        """Reference ``utils/layer_norm_cuda.py:148-192``: dx in x's dtype (channels-last),
        FP32 dweight and dbias.  The statistics (mean and rstd per pixel, pixel order) are
        those the forward wrote; an NCHW input is re-laid out once here."""
        x, weight, mean, rstd = ctx.saved_tensors
        batch, channels, height, width = x.shape
        if not x.is_contiguous(memory_format=torch.channels_last):
            # NCHW forward: its statistics are in (b, h, w) order as well
            x = x.contiguous(memory_format=torch.channels_last)
        g = dy.to(dtype=torch.float32, memory_format=torch.channels_last)
        dx = torch.empty_like(x, memory_format=torch.channels_last)
        dweight = torch.empty(channels, device=x.device, dtype=torch.float32)
        dbias = torch.empty(channels, device=x.device, dtype=torch.float32)
        lib = hip.load_library()
        ws = hip.workspace(lib.vh_layernorm2d_backward_workspace_bytes(batch, channels, height, width), x.device)
        hip.check(lib.vh_layernorm2d_backward(
            hip.ptr(g), hip.ptr(x), hip.dtype_code(x.dtype), hip.ptr(weight), hip.ptr(mean), hip.ptr(rstd),
            hip.ptr(dx), hip.ptr(dweight), hip.ptr(dbias), batch, channels, height, width, hip.ptr(ws),
            ws.numel() * 4, hip.stream_of(x)), "vh_layernorm2d_backward")
        weight_shape, bias_shape = ctx.param_shapes
        return dx, dweight.view(weight_shape), dbias.view(bias_shape), None, None, None


def can_fuse_layernorm2d(x, weight, bias):
    """Eligibility of the native kernel (``utils/layer_norm_cuda.py:195-213``, minus Triton)."""
    if x.ndim != 4 or not x.is_cuda:
        return False
    if x.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        return False
    channels = x.shape[1]
    if channels < 1 or channels > 4096:
        return False
    if weight is None or bias is None:
        return False
    return (weight.device == x.device and bias.device == x.device
            and weight.is_floating_point() and bias.is_floating_point()
            and weight.numel() == channels and bias.numel() == channels)


def visionhope_layernorm2d(x, weight, bias, eps, force_channels_last=False, out_dtype=torch.float32):
    """FP32 output (the reference's contract); ``out_dtype`` stores the same values rounded
    to a 16-bit type when the consumer casts them anyway (autocast)."""
    return _VisionHOPELayerNorm2dFunction.apply(x, weight, bias, eps, force_channels_last, out_dtype)


def can_fuse_add_layernorm2d(x, r, weight, bias):
    """x + r followed by LayerNorm2d in one pass: channels-last CUDA tensors of one dtype,
    C % 8 == 0 with at most 8 groups of 8 channels per lane, 16-byte aligned."""
    if x.ndim != 4 or not x.is_cuda or r.shape != x.shape or r.dtype != x.dtype:
        return False
    if x.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        return False
    fmt = torch.channels_last
    if not (x.is_contiguous(memory_format=fmt) and r.is_contiguous(memory_format=fmt)):
        return False
    channels = x.shape[1]
    if channels % 8 or channels > 4096:
        return False
    groups, lanes = channels // 8, 1
    while lanes < 32 and groups % (2 * lanes) == 0:   # lanes per pixel row, as the kernel picks
        lanes *= 2
    if groups // lanes > 8:
        return False
    tensors = (x, r, weight, bias)
    return (all(t.data_ptr() % 16 == 0 for t in tensors) and weight.dtype == torch.float32
            and bias.dtype == torch.float32 and weight.is_contiguous() and bias.is_contiguous()
            and weight.numel() == channels and bias.numel() == channels)


@on_tensor_device
def visionhope_add_layernorm2d(x, r, weight, bias, eps, out_dtype=torch.float32):
    """``s = x + r`` (rounded to x's dtype) and ``LayerNorm2d(s)`` in one pass on
    channels-last maps; returns ``(s, y)`` with y stored as ``out_dtype``."""
    batch, channels, height, width = x.shape
    x_sum = torch.empty_like(x, memory_format=torch.channels_last)
    y = torch.empty_like(x, dtype=out_dtype, memory_format=torch.channels_last)
    lib = hip.load_library()
    hip.check(lib.vh_add_layernorm2d_forward(
        hip.ptr(x), hip.ptr(r), hip.dtype_code(x.dtype), hip.ptr(weight), hip.ptr(bias), hip.ptr(x_sum),
        hip.ptr(y), hip.dtype_code(out_dtype), batch, channels, height, width, float(eps), hip.stream_of(x)),
        "vh_add_layernorm2d_forward")
    return x_sum, y
