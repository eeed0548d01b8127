"""Residual add ``x + gamma_c * branch * drop_mask_b`` (mirrors ``utils/residual.py``).

The native kernel replaces the Triton forward kernel; output is FP32 channels-last.
"""
import torch
from torch.autograd import Function

from . import hip
from .cuda import on_tensor_device


class _VisionHOPEResidualFunction(Function):
    @staticmethod
    @on_tensor_device
    def forward(ctx, residual, branch, gamma, mask):
        batch, channels, height, width = branch.shape
        spatial = height * width
        total = batch * spatial * channels
        residual = residual.contiguous(memory_format=torch.channels_last)
        branch = branch.contiguous(memory_format=torch.channels_last)
        gamma_shape = gamma.shape
        gamma = gamma.detach().reshape(-1).float().contiguous()
        mask = mask.float().contiguous()
        out = torch.empty_like(branch, dtype=torch.float32, memory_format=torch.channels_last)
        lib = hip.load_library()
        hip.check(lib.vh_residual_add_forward(
            hip.ptr(residual), hip.dtype_code(residual.dtype), hip.ptr(branch),
            hip.dtype_code(branch.dtype), hip.ptr(gamma), hip.ptr(mask), hip.ptr(out), total,
            channels, spatial, hip.stream_of(branch)), "vh_residual_add_forward")
        ctx.save_for_backward(branch, gamma, mask)
        ctx.gamma_shape = gamma_shape
        return out

    @staticmethod
    @on_tensor_device
    def backward(ctx, dout):
        """Reference ``utils/residual.py:130-170``: dresidual = dout, dbranch in the branch's
        dtype (channels-last), FP32 dgamma."""
        branch, gamma, mask = ctx.saved_tensors
        batch, channels, height, width = branch.shape
        g = dout.to(dtype=torch.float32, memory_format=torch.channels_last)
        total = g.numel()
        dbranch = torch.empty_like(branch, memory_format=torch.channels_last)
        dgamma = torch.empty(channels, device=branch.device, dtype=torch.float32)
        lib = hip.load_library()
        ws = hip.workspace(lib.vh_residual_add_backward_workspace_bytes(total, channels), branch.device)
        hip.check(lib.vh_residual_add_backward(
            hip.ptr(g), hip.ptr(branch), hip.dtype_code(branch.dtype), hip.ptr(gamma), hip.ptr(mask),
            hip.ptr(dbranch), hip.ptr(dgamma), total, channels, height * width, hip.ptr(ws), ws.numel() * 4,
            hip.stream_of(branch)), "vh_residual_add_backward")
        return g, dbranch, dgamma.view(ctx.gamma_shape), None


def can_fuse_residual_add(residual, branch, gamma):
    """Reference eligibility test (``utils/residual.py:161-183``, minus Triton)."""
    if residual.ndim != 4 or branch.ndim != 4 or residual.shape != branch.shape:
        return False
    if not residual.is_cuda or not branch.is_cuda or not gamma.is_cuda:
        return False
    if residual.device != branch.device or gamma.device != branch.device:
        return False
    if not gamma.is_contiguous() or not gamma.is_floating_point():
        return False
    if not residual.is_contiguous(memory_format=torch.channels_last):
        return False
    if not branch.is_contiguous(memory_format=torch.channels_last):
        return False
    if (branch.dtype not in (torch.float16, torch.bfloat16, torch.float32)
            or residual.dtype not in (torch.float16, torch.bfloat16, torch.float32)):
        return False
    channels = branch.shape[1]
    return gamma.numel() == channels and channels > 0


def visionhope_residual_add(residual, branch, gamma, drop_prob, training, scale_by_keep=True):
    """``residual + branch * gamma * mask`` with stochastic depth (``utils/residual.py:186-204``)."""
    batch = branch.shape[0]
    if training and drop_prob > 0.0:
        keep_prob = 1.0 - float(drop_prob)
        mask = torch.empty((batch,), device=branch.device, dtype=torch.float32).bernoulli_(keep_prob)
        if keep_prob > 0.0 and scale_by_keep:
            mask.div_(keep_prob)
    else:
        mask = torch.ones((batch,), device=branch.device, dtype=torch.float32)
    return _VisionHOPEResidualFunction.apply(residual, branch, gamma, mask)
