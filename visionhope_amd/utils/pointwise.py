"""1x1 convolutions of the VisionHOPE block as bf16 matrix-core GEMMs on channels-last maps.

``pointwise_conv(x, module, epilogue)`` computes ``module`` (a 1x1 ``nn.Conv2d`` or an
``nn.Linear``) on the NHWC view ``x [..., K]`` through ``vh_pointwise_conv_nhwc_forward``
with the elementwise work around the projection fused:

===============  ===========================================  ==============================
epilogue         result (every step rounded to bf16)           reference expression
===============  ===========================================  ==============================
``EPI_BIAS``     x W^T + b                                     ``proj_in(x)``, ``fc1(x)`` ...
``EPI_GELU``     gelu(x W^T + b)                               ``ffn.act(ffn.fc1(x))``
``EPI_ADD``      r + (x W^T + b)                               ``x + ffn(...)`` (gamma folded)
``EPI_SILU``     silu(x W^T + b)                               ``head_act(head_norm(...))``
                                                               (BatchNorm folded)
===============  ===========================================  ==============================

With ``grn=(scale, beta)`` the operand is ``bf16(x * scale[image] + beta)``: the GRN output
(``grn_scale`` gives the factor), applied as the operand is loaded
(``models/block.py:70-107``, ``models/layers.py:67-80``).  Under bf16 autocast the
reference rounds the same intermediates to bf16; only the fp32 summation order differs.
"""

import torch
from torch import nn

from . import hip
from .cached_params import _key
from .cuda import on_tensor_device

EPI_BIAS, EPI_GELU, EPI_ADD, EPI_SILU = range(4)


def is_pointwise(module):
    """A Linear or an unpadded, ungrouped, stride-1 1x1 Conv2d."""
    if isinstance(module, nn.Linear):
        return True
    return (isinstance(module, nn.Conv2d) and module.kernel_size == (1, 1) and module.stride == (1, 1)
            and module.padding == (0, 0) and module.groups == 1 and module.dilation == (1, 1))


def supported(in_features, out_features):
    """Shapes the matrix-core kernel covers (K and N multiples of 32)."""
    n, k = out_features, in_features
    return k % 32 == 0 and n % 32 == 0


def pointwise_operands(module):
    """``(weight [N, K] bf16, bias [N] fp32 holding bf16-rounded values or None)``: what
    autocast casts the parameters to on every call, cached on the module while both are
    unchanged."""
    w, b = module.weight, module.bias
    key = (_key(w), None if b is None else _key(b))
    cached = getattr(module, "_vh_pointwise", None)
    if cached is None or cached[0] != key:
        weight = w.detach().reshape(w.shape[0], -1).to(torch.bfloat16).contiguous()
        bias = None if b is None else b.detach().to(torch.bfloat16).float().contiguous()
        object.__setattr__(module, "_vh_pointwise", (key, weight, bias))
        cached = module._vh_pointwise
    return cached[1], cached[2]


def pointwise_conv(x, module, epilogue=EPI_BIAS, residual=None, grn=None, out=None):
    """``x [..., K]`` contiguous bf16 (an NHWC map) -> ``[..., N]`` bf16 (module docstring).

    ``residual`` (``EPI_ADD``) is shaped like the output; ``grn`` is ``(scale [B, K],
    beta [K])`` FP32 for an ``x`` of ``B`` images of equal size; ``out`` receives the
    result when given (contiguous, shaped like the output).
    """
    weight, bias = pointwise_operands(module)
    return pointwise_gemm(x, weight, bias, epilogue, residual, grn, out)


@on_tensor_device
def pointwise_gemm(x, weight, bias, epilogue=EPI_BIAS, residual=None, grn=None, out=None):
    """``pointwise_conv`` on explicit operands: ``weight [N, K]`` contiguous bf16 and
    ``bias [N]`` fp32 (or None)."""
    if not x.is_cuda or x.dtype != torch.bfloat16 or not x.is_contiguous() or x.data_ptr() % 16:
        raise ValueError("pointwise_conv expects a contiguous 16-byte aligned CUDA bf16 tensor")
    if (weight.dtype != torch.bfloat16 or weight.dim() != 2 or not weight.is_contiguous()
            or (bias is not None and (bias.dtype != torch.float32 or bias.numel() != weight.shape[0]))):
        raise ValueError("pointwise_conv needs a contiguous bf16 weight [N, K] and an fp32 bias [N]")
    n, k = weight.shape
    if x.shape[-1] != k or not supported(k, n):
        raise ValueError(f"pointwise_conv does not cover K={x.shape[-1]} -> N={n}")
    m = x.numel() // k
    shape = (*x.shape[:-1], n)
    if out is None:
        out = torch.empty(shape, device=x.device, dtype=torch.bfloat16)
    elif out.shape != shape or out.dtype != torch.bfloat16 or not out.is_contiguous() or out.data_ptr() % 16:
        raise ValueError("out must be a contiguous bf16 tensor shaped like the result")
    if epilogue == EPI_ADD:
        if (residual is None or residual.shape != shape or residual.dtype != torch.bfloat16
                or not residual.is_contiguous() or residual.data_ptr() % 16):
            raise ValueError("EPI_ADD needs a contiguous bf16 residual shaped like the result")
    scale = beta = None
    per_image = 0
    if grn is not None:
        scale, beta = grn
        images = scale.shape[0]
        if (scale.dtype != torch.float32 or beta.dtype != torch.float32 or scale.shape != (images, k)
                or beta.numel() != k or m % images or not scale.is_contiguous() or not beta.is_contiguous()):
            raise ValueError("grn needs FP32 scale [images, K] and beta [K]")
        per_image = m // images
    lib = hip.load_library()
    hip.check(lib.vh_pointwise_conv_nhwc_forward(
        hip.ptr(x), hip.VH_DTYPE_BF16, hip.ptr(weight), hip.ptr(bias), int(epilogue), hip.ptr(residual),
        hip.ptr(scale), hip.ptr(beta), per_image, hip.ptr(out), m, n, k, hip.stream_of(x)),
        "vh_pointwise_conv_nhwc_forward")
    return out


def chain_supported(first, second):
    """Whether ``pointwise_chain`` covers ``second(first(x))``: two 1x1 projections with
    biases, ``first`` K -> N and ``second`` N -> N, with N = 64 or 128 and K % 64 == 0, or
    N = 32 and K = 32 or 64."""
    if not (is_pointwise(first) and is_pointwise(second)) or first.bias is None or second.bias is None:
        return False
    n, k = first.weight.shape[0], first.weight.shape[1]
    widths = (n in (64, 128) and k % 64 == 0) or (n == 32 and k in (32, 64))
    return widths and tuple(second.weight.shape[:2]) == (n, n)


@on_tensor_device
def pointwise_chain(x, first, second):
    """``(first(x), second(first(x)))`` for ``x [..., K]`` contiguous bf16, both rounded to
    bf16 as two ``pointwise_conv`` calls give them, in one launch
    (``vh_pointwise_chain_nhwc_forward``); ``chain_supported`` must hold."""
    if not chain_supported(first, second):
        raise ValueError("pointwise_chain covers K -> N -> N projections with N = 64 or 128 and K % 64 == 0, "
                         "or N = 32 and K = 32 or 64")
    if not x.is_cuda or x.dtype != torch.bfloat16 or not x.is_contiguous() or x.data_ptr() % 16:
        raise ValueError("pointwise_chain expects a contiguous 16-byte aligned CUDA bf16 tensor")
    w1, b1 = pointwise_operands(first)
    w2, b2 = pointwise_operands(second)
    n, k = w1.shape
    if x.shape[-1] != k:
        raise ValueError(f"pointwise_chain expects {k} input channels, got {x.shape[-1]}")
    m = x.numel() // k
    shape = (*x.shape[:-1], n)
    out = torch.empty(shape, device=x.device, dtype=torch.bfloat16)
    out2 = torch.empty(shape, device=x.device, dtype=torch.bfloat16)
    lib = hip.load_library()
    hip.check(lib.vh_pointwise_chain_nhwc_forward(
        hip.ptr(x), hip.ptr(w1), hip.ptr(b1), hip.ptr(w2), hip.ptr(b2), hip.ptr(out), hip.ptr(out2), m, n, k,
        hip.stream_of(x)), "vh_pointwise_chain_nhwc_forward")
    return out, out2


def add_layernorm_supported(module):
    """Whether ``pointwise_add_layernorm`` covers ``module`` (K -> N with bias): N = 64 with
    K = 32 or 64, or N = 128 or 256 with K = 64 or 128."""
    if not is_pointwise(module) or module.bias is None:
        return False
    n, k = module.weight.shape[0], module.weight.shape[1]
    return (n == 64 and k in (32, 64)) or (n in (128, 256) and k in (64, 128))


@on_tensor_device
def pointwise_add_layernorm(x, module, residual, ln_weight, ln_bias, eps):
    """``s = bf16(residual + module(x))`` and ``bf16(LayerNorm(s))`` over the channels, both
    ``[..., N]`` bf16, in the product's launch (``vh_pointwise_add_layernorm_nhwc_forward``):
    the bits of ``pointwise_conv`` followed by the channels-last residual add + LayerNorm
    (``visionhope_add_layernorm2d``).  ``add_layernorm_supported(module)`` must hold."""
    if not add_layernorm_supported(module):
        raise ValueError("pointwise_add_layernorm covers N = 64 (K = 32, 64) and N = 128, 256 (K = 64, 128)")
    if not x.is_cuda or x.dtype != torch.bfloat16 or not x.is_contiguous() or x.data_ptr() % 16:
        raise ValueError("pointwise_add_layernorm expects a contiguous 16-byte aligned CUDA bf16 tensor")
    weight, bias = pointwise_operands(module)
    n, k = weight.shape
    shape = (*x.shape[:-1], n)
    if (x.shape[-1] != k or residual.shape != shape or residual.dtype != torch.bfloat16
            or not residual.is_contiguous() or residual.data_ptr() % 16):
        raise ValueError("pointwise_add_layernorm needs x [..., K] and a contiguous bf16 residual [..., N]")
    lw = ln_weight.detach().float().contiguous()
    lb = ln_bias.detach().float().contiguous()
    if lw.numel() != n or lb.numel() != n:
        raise ValueError("LayerNorm weight and bias must have N entries")
    m = x.numel() // k
    out_sum = torch.empty(shape, device=x.device, dtype=torch.bfloat16)
    out_norm = torch.empty(shape, device=x.device, dtype=torch.bfloat16)
    lib = hip.load_library()
    hip.check(lib.vh_pointwise_add_layernorm_nhwc_forward(
        hip.ptr(x), hip.ptr(weight), hip.ptr(bias), hip.ptr(residual), hip.ptr(lw), hip.ptr(lb), float(eps),
        hip.ptr(out_sum), hip.ptr(out_norm), m, n, k, hip.stream_of(x)), "vh_pointwise_add_layernorm_nhwc_forward")
    return out_sum, out_norm
