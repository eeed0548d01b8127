"""Convolution + BatchNorm (+ GELU) of the stem and downsample layers with the BatchNorm
folded into the convolution (inference only).

In eval mode ``bn(conv(x)) = conv(x; W s) + ((b - mean) s + beta)`` with
``s = gamma / sqrt(var + eps)`` per output channel (``models/layers.py:85-119``). The
folded weight goes to the library convolution (cast by autocast as the original would be);
the folded bias and the activation run in one native channels-last pass
(``vh_bias_act_nhwc_forward``), which rounds the BatchNorm output and the activation output
to the activation dtype, as the unfolded modules do.
"""

import torch
from torch import nn
from torch.nn import functional as F

from . import hip
from .cached_params import _key
from .cuda import on_tensor_device

ACT_NONE, ACT_GELU = 0, 1


def foldable(conv, bn):
    """A Conv2d followed by an eval-mode affine BatchNorm2d with running statistics."""
    return (isinstance(conv, nn.Conv2d) and type(bn) is nn.BatchNorm2d and not bn.training
            and bn.track_running_stats and bn.running_mean is not None and bn.affine
            and bn.num_features == conv.out_channels and conv.out_channels % 8 == 0
            and conv.padding_mode == "zeros")


def folded_weights(conv, bn):
    """``(weight, bias)`` FP32 of the folded convolution, cached on the conv while every
    contributing parameter and statistic is unchanged."""
    parts = (conv.weight, conv.bias, bn.weight, bn.bias, bn.running_mean, bn.running_var)
    key = tuple(None if t is None else _key(t) for t in parts) + (float(bn.eps),)
    cached = getattr(conv, "_vh_folded_bn", None)
    if cached is None or cached[0] != key:
        with torch.no_grad():
            scale = bn.weight.float() / torch.sqrt(bn.running_var.float() + bn.eps)
            weight = conv.weight.float() * scale.view(-1, 1, 1, 1)
            bias = conv.bias.float() if conv.bias is not None else torch.zeros_like(scale)
            bias = ((bias - bn.running_mean.float()) * scale + bn.bias.float()).contiguous()
            weight = weight.contiguous(memory_format=torch.channels_last)
        object.__setattr__(conv, "_vh_folded_bn", (key, weight, bias))
        cached = conv._vh_folded_bn
    return cached[1], cached[2]


@on_tensor_device
def bias_act(x, bias, act=ACT_NONE):
    """``act(round(x + bias))`` per channel on the channels-last map ``x``, in place."""
    if not x.is_contiguous(memory_format=torch.channels_last) or x.data_ptr() % 16:
        raise ValueError("bias_act expects a 16-byte aligned channels-last map")
    lib = hip.load_library()
    hip.check(lib.vh_bias_act_nhwc_forward(
        hip.ptr(x), hip.dtype_code(x.dtype), hip.ptr(bias), int(act), hip.ptr(x), x.numel(), x.shape[1],
        hip.stream_of(x)), "vh_bias_act_nhwc_forward")
    return x


def conv_bn_act(x, conv, bn, act=ACT_NONE):
    """``act(bn(conv(x)))`` for an eval-mode BatchNorm, folded (module docstring)."""
    weight, bias = folded_weights(conv, bn)
    y = F.conv2d(x, weight, None, conv.stride, conv.padding, conv.dilation, conv.groups)
    if not y.is_contiguous(memory_format=torch.channels_last) or y.data_ptr() % 16:
        y = y.contiguous(memory_format=torch.channels_last)
    return bias_act(y, bias, act)
