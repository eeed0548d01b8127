"""Convolution + BatchNorm (+ GELU) of the stem and downsample layers with the BatchNorm
folded into the convolution (inference only).

In eval mode ``bn(conv(x)) = conv(x; W s) + ((b - mean) s + beta)`` with
``s = gamma / sqrt(var + eps)`` per output channel (``models/layers.py:85-119``). The
3x3 convolutions of the stem and downsample layers (every width that is a multiple of 32:
Tiny, Small and Base) run as one native implicit GEMM
with the folded bias and the GELU in its epilogue (``vh_conv3x3_nhwc_forward``: the
folded weight rounded to bf16 as autocast rounds it, the sum and the activation each
rounded to bf16). Other shapes go to the library convolution with the folded weight,
followed by one native channels-last pass for the bias and activation
(``vh_bias_act_nhwc_forward``), which rounds the BatchNorm output and the activation
output to the activation dtype, as the unfolded modules do.
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


def _bf16_compute(x, conv):
    """The convolution computes in bf16: a bf16 map, or the fp32 image under bf16 autocast
    (which the reference's autocast conv would round to bf16)."""
    if x.dtype == torch.bfloat16:
        return True
    return (x.dtype == torch.float32 and conv.in_channels == 3 and torch.is_autocast_enabled("cuda")
            and torch.get_autocast_dtype("cuda") == torch.bfloat16)


def native_conv3x3_ok(x, conv):
    """Whether ``vh_conv3x3_nhwc_forward`` takes ``conv`` on the channels-last map ``x``."""
    n, c = conv.out_channels, conv.in_channels
    return (x.is_cuda and x.dim() == 4 and x.shape[1] == c and conv.kernel_size == (3, 3)
            and conv.padding == (1, 1) and conv.dilation == (1, 1) and conv.groups == 1
            and conv.stride in ((1, 1), (2, 2)) and conv.padding_mode == "zeros"
            and x.is_contiguous(memory_format=torch.channels_last) and (c == 3 or c % 32 == 0)
            and n % 32 == 0 and _bf16_compute(x, conv))


def gemm_weight(conv, weight):
    """The folded weight as the implicit-GEMM operand ``[N, K]`` bf16 (layout in
    ``include/visionhope_hip.h``: channels-last taps, and for 3 input channels the taps
    padded to 4 channels and 16 taps), cached next to the folded weight it comes from."""
    cached = getattr(conv, "_vh_conv_gemm", None)
    if cached is None or cached[0] is not weight:
        with torch.no_grad():
            n, c = weight.shape[0], weight.shape[1]
            taps = weight.permute(0, 2, 3, 1).reshape(n, 9, c)
            if c == 3:
                padded = torch.zeros(n, 16, 4, device=weight.device, dtype=weight.dtype)
                padded[:, :9, :3] = taps
                taps = padded
            gemm = taps.reshape(n, -1).to(torch.bfloat16).contiguous()
        object.__setattr__(conv, "_vh_conv_gemm", (weight, gemm))
        cached = conv._vh_conv_gemm
    return cached[1]


@on_tensor_device
def conv3x3_bias_act(x, conv, weight, bias, act=ACT_NONE):
    """``act(conv(x; weight) + bias)`` for a 3x3, padding-1 ``conv`` on the channels-last
    map ``x`` through the native implicit GEMM; bf16 channels-last output."""
    gemm = gemm_weight(conv, weight)
    b, c, h, w = x.shape
    s = conv.stride[0]
    n = weight.shape[0]
    out = torch.empty((b, n, (h - 1) // s + 1, (w - 1) // s + 1), device=x.device, dtype=torch.bfloat16,
                      memory_format=torch.channels_last)
    lib = hip.load_library()
    hip.check(lib.vh_conv3x3_nhwc_forward(
        hip.ptr(x), hip.dtype_code(x.dtype), hip.ptr(gemm), hip.ptr(bias), int(act), hip.ptr(out),
        b, h, w, c, n, s, hip.stream_of(x)), "vh_conv3x3_nhwc_forward")
    return out


def _round32(n):
    return (n + 31) // 32 * 32


def padded_native_ok(x, conv):
    """Whether ``conv_bn_act_padded`` can run ``conv`` natively on ``x`` (whose channels may
    already carry zero padding beyond ``conv.in_channels``)."""
    c = x.shape[1]
    return (x.is_cuda and x.dim() == 4 and c >= conv.in_channels and (c == 3 or c % 32 == 0)
            and conv.kernel_size == (3, 3) and conv.padding == (1, 1) and conv.dilation == (1, 1)
            and conv.groups == 1 and conv.stride in ((1, 1), (2, 2)) and conv.padding_mode == "zeros"
            and x.is_contiguous(memory_format=torch.channels_last) and _bf16_compute(x, conv)
            and (c == conv.in_channels or c % 32 == 0))


def conv_bn_act_padded(x, conv, bn, act=ACT_NONE, pad_out=False):
    """``conv_bn_act`` for widths the implicit GEMM does not take (not a multiple of 32): the
    folded weight gets zero rows up to the next multiple of 32 outputs (``pad_out``) and zero
    columns for the zero channels ``x`` already carries; the padded bias is 0.  A padded
    output channel is then exactly act(0) = 0 (GELU or none), so the next convolution's zero
    weight columns see zeros and the real channels are unchanged.  Returns the map with
    ``round32(out_channels)`` channels when ``pad_out``, else with ``out_channels``."""
    weight, bias = folded_weights(conv, bn)
    n, cin = weight.shape[0], weight.shape[1]
    c = x.shape[1]
    n_pad = _round32(n) if pad_out else n
    key = (id(weight), c, n_pad)
    cached = getattr(conv, "_vh_padded", None)
    if cached is None or cached[0] != key or cached[1] is not weight:
        with torch.no_grad():
            w = torch.zeros(n_pad, c, 3, 3, device=weight.device, dtype=weight.dtype)
            w[:n, :cin] = weight
            w = w.contiguous(memory_format=torch.channels_last)
            b = torch.zeros(n_pad, device=bias.device, dtype=bias.dtype)
            b[:n] = bias
        object.__setattr__(conv, "_vh_padded", (key, weight, w, b))
        cached = conv._vh_padded
    w, b = cached[2], cached[3]
    return conv3x3_bias_act(x, conv, w, b, act)


def conv_bn_act(x, conv, bn, act=ACT_NONE):
    """``act(bn(conv(x)))`` for an eval-mode BatchNorm, folded (module docstring)."""
    weight, bias = folded_weights(conv, bn)
    if native_conv3x3_ok(x, conv):
        return conv3x3_bias_act(x, conv, weight, bias, act)
    y = F.conv2d(x, weight, None, conv.stride, conv.padding, conv.dilation, conv.groups)
    if not y.is_contiguous(memory_format=torch.channels_last) or y.data_ptr() % 16:
        y = y.contiguous(memory_format=torch.channels_last)
    return bias_act(y, bias, act)
