"""Native LayerNorm over channels for NCHW feature maps (replaces the Triton kernel of
``utils/layer_norm_cuda.py``).

Per pixel: mean, biased centred variance, ``y = (x - mean) * rstd * w + b``, FP32
output in the input's storage order (channels-last or NCHW).
"""
import torch
from torch.autograd import Function

from . import hip
from .autograd import backward_unavailable
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
        weight = weight.detach().reshape(-1).float().contiguous()
        bias = bias.detach().reshape(-1).float().contiguous()
        y = torch.empty_like(x, dtype=out_dtype, memory_format=fmt)
        lib = hip.load_library()
        hip.check(lib.vh_layernorm2d_forward(
            hip.ptr(x), hip.dtype_code(x.dtype), hip.ptr(weight), hip.ptr(bias), hip.ptr(y),
            hip.dtype_code(out_dtype), None, None, batch, channels, height, width, float(eps),
            int(channels_last),
            hip.stream_of(x)), "vh_layernorm2d_forward")
        return y

    @staticmethod
    def backward(ctx, dy):
        backward_unavailable("LayerNorm2d")


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
