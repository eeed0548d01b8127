"""Global Response Normalization (mirrors ``utils/grn.py`` of the reference).

GPU tensors always run the native HIP kernels (``vh_grn_forward``); CPU tensors
use the same formula in PyTorch FP32, as the reference does for CPU tensors
(``utils/grn.py:41-51``).  The output is FP32.
"""
import torch
from torch import nn

from .grn_cuda import visionhope_grn

__all__ = ["GlobalResponseNorm", "global_response_norm", "grn_reference"]


def _check_shape(x, gamma, beta):
    if x.ndim != 4:
        raise ValueError("GRN expects logical NCHW input with four dimensions")
    if not x.is_floating_point() or not gamma.is_floating_point() or not beta.is_floating_point():
        raise TypeError("GRN expects floating-point input and channel parameters")
    if gamma.numel() != x.shape[1] or beta.numel() != x.shape[1]:
        raise ValueError("GRN gamma and beta must each contain one value per channel")
    if gamma.device != x.device or beta.device != x.device:
        raise ValueError("GRN input, gamma and beta must be on the same device")


def grn_reference(x, gamma, beta, eps=1e-6):
    """The GRN formula in PyTorch FP32 (``utils/grn.py:26-38``)."""
    _check_shape(x, gamma, beta)
    x = x.float()
    gamma = gamma.float().reshape(1, x.shape[1], 1, 1)
    beta = beta.float().reshape(1, x.shape[1], 1, 1)
    gx = torch.norm(x, p=2, dim=(2, 3), keepdim=True)
    nx = gx / (gx.mean(dim=1, keepdim=True) + float(eps))
    return x * (1.0 + gamma * nx) + beta


def global_response_norm(x, gamma, beta, eps=1e-6):
    """FP32 GRN output; GPU tensors run the HIP kernels (``utils/grn.py:41-51``)."""
    _check_shape(x, gamma, beta)
    if x.is_cuda:
        return visionhope_grn(x, gamma, beta, float(eps))
    return grn_reference(x, gamma, beta, eps)


class GlobalResponseNorm(nn.Module):
    """GRN for logical NCHW tensors with FP32 output (``utils/grn.py:54-70``)."""

    def __init__(self, dim, eps=1e-6):
        super().__init__()
        self.gamma = nn.Parameter(torch.zeros(1, dim, 1, 1, dtype=torch.float32))
        self.beta = nn.Parameter(torch.zeros(1, dim, 1, 1, dtype=torch.float32))
        self.eps = float(eps)

    def forward(self, x):
        return global_response_norm(x, self.gamma, self.beta, self.eps)

    def extra_repr(self):
        return f"dim={self.gamma.numel()}, eps={self.eps}, output_dtype=float32"
