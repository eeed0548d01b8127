"""Fused depthwise convolutions of the VisionHOPE block on channels-last maps.

``depthwise_conv(x, conv, epilogue)`` runs a depthwise ``nn.Conv2d`` (K in {3, 5, 7},
stride 1, padding K//2) through ``vh_dwconv2d_nhwc_forward`` with the surrounding
elementwise work of the block fused into the same pass:

=================  =====================================  ==========================
epilogue           result                                 reference expression
=================  =====================================  ==========================
``EPI_PLAIN``      conv(x) + b                            ``conv(x)``
``EPI_ADD_INPUT``  x + conv(x) + b                        ``x + self.cpe(x)``
``EPI_GATE``       x + sigmoid(aux) * (conv(x) + b)       ``_local_features``
``EPI_ADD_GELU``   gelu(x + conv(x) + b)                  ``dwconv_act(x + dwconv(x))``
``EPI_ACCUM_F32``  out += conv(x) + b  (fp32 NHWC)        ``out + local_position(x)``
``EPI_ADD_F32_AUX`` aux + conv(x) + b (aux fp32 NHWC)      ``out + local_position(x)``
=================  =====================================  ==========================

(``models/block.py:63-107``, ``models/layers.py:73-77``.)  Accumulation is FP32 with
FP32 taps; the result is rounded once to the activation dtype.
"""

import torch
from torch import nn

from . import hip
from .cuda import on_tensor_device

EPI_PLAIN, EPI_ADD_INPUT, EPI_GATE, EPI_ADD_GELU, EPI_ACCUM_F32, EPI_ADD_F32_AUX = range(6)
_DTYPES = (torch.float32, torch.bfloat16, torch.float16)


def is_depthwise(conv):
    """A depthwise Conv2d the fused kernel implements exactly."""
    if not isinstance(conv, nn.Conv2d):
        return False
    k = conv.kernel_size[0]
    return (conv.groups == conv.in_channels == conv.out_channels and conv.in_channels % 8 == 0
            and conv.kernel_size == (k, k) and k in (3, 5, 7) and conv.stride == (1, 1)
            and conv.padding == (k // 2, k // 2) and conv.dilation == (1, 1)
            and conv.padding_mode == "zeros")


def depthwise_taps(conv):
    """Taps-major FP32 weights ``[K*K, C]`` and FP32 bias of a depthwise Conv2d, cached on
    the module and refreshed when the weight changes (version counter, device)."""
    w = conv.weight
    key = (w.data_ptr(), w._version, str(w.device),
           None if conv.bias is None else (conv.bias.data_ptr(), conv.bias._version))
    cached = getattr(conv, "_vh_taps", None)
    if cached is None or cached[0] != key:
        taps = w.detach().float().reshape(w.shape[0], -1).t().contiguous()
        bias = conv.bias.detach().float().contiguous() if conv.bias is not None else None
        object.__setattr__(conv, "_vh_taps", (key, taps, bias))
        cached = conv._vh_taps
    return cached[1], cached[2]


def _channels_last(t):
    if not t.is_contiguous(memory_format=torch.channels_last) or t.data_ptr() % 16:
        t = t.contiguous(memory_format=torch.channels_last)
        if t.data_ptr() % 16:
            t = t.clone(memory_format=torch.channels_last)
    return t


@on_tensor_device
def depthwise_conv(x, conv, epilogue=EPI_PLAIN, aux=None, out=None):
    """Run ``conv`` on the channels-last map ``x`` with a fused epilogue (module docstring).

    For ``EPI_ACCUM_F32`` ``out`` is a contiguous FP32 ``[B, H, W, C]`` tensor updated in
    place; otherwise the result is written to ``out`` when given (channels-last, x's dtype)
    or to a new ``x``-dtype channels-last tensor (for
    ``EPI_ADD_F32_AUX``, ``aux`` is the FP32 ``[B, H, W, C]`` addend).
    """
    if not x.is_cuda or x.dtype not in _DTYPES:
        raise ValueError("depthwise_conv expects a CUDA FP32/BF16/FP16 tensor")
    if not is_depthwise(conv):
        raise ValueError("depthwise_conv needs a depthwise Conv2d with K in {3, 5, 7}, stride 1, same padding")
    batch, channels, height, width = x.shape
    if channels != conv.in_channels:
        raise ValueError("channel count does not match the convolution")
    taps, bias = depthwise_taps(conv)
    x = _channels_last(x)
    if epilogue == EPI_GATE:
        if aux is None or aux.shape != x.shape:
            raise ValueError("the gated epilogue needs a gate tensor shaped like x")
        aux = _channels_last(aux.to(x.dtype))
    if epilogue == EPI_ADD_F32_AUX:
        if (aux is None or aux.dtype != torch.float32 or tuple(aux.shape) != (batch, height, width, channels)
                or not aux.is_contiguous() or aux.data_ptr() % 16):
            raise ValueError("EPI_ADD_F32_AUX needs a contiguous FP32 [B, H, W, C] addend")
    if epilogue == EPI_ACCUM_F32:
        if (out is None or out.dtype != torch.float32 or tuple(out.shape) != (batch, height, width, channels)
                or not out.is_contiguous() or out.data_ptr() % 16):
            raise ValueError("EPI_ACCUM_F32 needs a contiguous FP32 [B, H, W, C] output")
    elif out is not None:
        if (out.dtype != x.dtype or out.shape != x.shape or not out.is_contiguous(memory_format=torch.channels_last)
                or out.data_ptr() % 16):
            raise ValueError("out must be a channels-last tensor shaped and typed like x")
    else:
        out = torch.empty_like(x, memory_format=torch.channels_last)
    lib = hip.load_library()
    hip.check(lib.vh_dwconv2d_nhwc_forward(
        hip.ptr(x), hip.dtype_code(x.dtype), hip.ptr(taps), hip.ptr(bias), conv.kernel_size[0],
        int(epilogue), hip.ptr(aux), hip.ptr(out), batch, height, width, channels, hip.stream_of(x)),
        "vh_dwconv2d_nhwc_forward")
    return out


@on_tensor_device
def depthwise_conv_add_layernorm(x, conv, weight, bias, eps):
    """``x + conv(x)`` (``EPI_ADD_INPUT``, the block CPE) and the LayerNorm over the
    channels of that sum (``visionhope_layernorm2d(..., force_channels_last=True,
    out_dtype=x.dtype)`` with ``weight``, ``bias``, ``eps``), both channels-last in x's
    dtype, from one pass and with the same bits as the two separate kernels; ``None``
    when the shape is not covered (kernel size 3 and C = 8 * 2^k <= 256, FP32 contiguous
    affine parameters), then use ``depthwise_conv`` and ``visionhope_layernorm2d``."""
    if not x.is_cuda or x.dtype not in _DTYPES or not is_depthwise(conv):
        raise ValueError("depthwise_conv_add_layernorm expects a CUDA map and a depthwise Conv2d")
    batch, channels, height, width = x.shape
    groups = channels // 8
    if (conv.kernel_size[0] != 3 or channels % 8 or groups > 32 or groups & (groups - 1)
            or weight.dtype != torch.float32 or bias.dtype != torch.float32
            or not weight.is_contiguous() or not bias.is_contiguous()
            or weight.numel() != channels or bias.numel() != channels
            or weight.data_ptr() % 16 or bias.data_ptr() % 16):
        return None
    taps, conv_bias = depthwise_taps(conv)
    x = _channels_last(x)
    out = torch.empty_like(x, memory_format=torch.channels_last)
    out_norm = torch.empty_like(x, memory_format=torch.channels_last)
    lib = hip.load_library()
    hip.check(lib.vh_dwconv2d_add_layernorm2d_forward(
        hip.ptr(x), hip.dtype_code(x.dtype), hip.ptr(taps), hip.ptr(conv_bias), 3, hip.ptr(weight),
        hip.ptr(bias), float(eps), hip.ptr(out), hip.ptr(out_norm), batch, height, width, channels,
        hip.stream_of(x)), "vh_dwconv2d_add_layernorm2d_forward")
    return out, out_norm


def depthwise_conv_gelu_grn(x, conv, gamma, eps):
    """``gelu(x + conv(x))`` (``EPI_ADD_GELU``) and the GRN scale ``[B, C]`` of that output
    (``1 + gamma * nx``, ``utils/grn.py:26-38``) from one pass over the map; ``None`` when
    the shape is outside what the fused statistics cover (then use ``depthwise_conv`` and
    ``grn_scale``)."""
    if not x.is_cuda or x.dtype not in _DTYPES or not is_depthwise(conv):
        raise ValueError("depthwise_conv_gelu_grn expects a CUDA map and a depthwise Conv2d")
    batch, channels, height, width = x.shape
    lib = hip.load_library()
    nbytes = lib.vh_dwconv2d_gelu_grn_workspace_bytes(batch, height, width, channels, conv.kernel_size[0])
    if nbytes == 0 or batch > 65535:
        return None
    taps, bias = depthwise_taps(conv)
    x = _channels_last(x)
    gamma = gamma.detach().reshape(-1).float().contiguous()
    out = torch.empty_like(x, memory_format=torch.channels_last)
    scale = torch.empty((batch, channels), device=x.device, dtype=torch.float32)
    gx = torch.empty((batch, channels), device=x.device, dtype=torch.float32)
    inv_den = torch.empty((batch,), device=x.device, dtype=torch.float32)
    ws = hip.workspace(nbytes, x.device)
    hip.check(lib.vh_dwconv2d_gelu_grn_forward(
        hip.ptr(x), hip.dtype_code(x.dtype), hip.ptr(taps), hip.ptr(bias), conv.kernel_size[0], hip.ptr(gamma),
        float(eps), hip.ptr(out), hip.ptr(gx), hip.ptr(inv_den), hip.ptr(scale), batch, height, width, channels,
        hip.ptr(ws), ws.numel() * 4, hip.stream_of(x)), "vh_dwconv2d_gelu_grn_forward")
    return out, scale
