"""Fused query normalisation and relayout for SRNL (mirrors ``utils/query_normalization.py``).

``[B, 4, N, heads*d]`` raw queries -> ``[B, 4, heads, N, d]`` FP32 unit vectors.
"""
import torch

from . import hip
from .cuda import on_tensor_device


class VisionHOPEQNormFunction(torch.autograd.Function):
    @staticmethod
    @on_tensor_device
    def forward(ctx, q_raw, num_heads, head_dim):
        q_raw_c = q_raw.contiguous()
        batch, directions, length, _ = q_raw_c.shape
        out = torch.empty((batch, directions, num_heads, length, head_dim), device=q_raw.device,
                          dtype=torch.float32)
        inv = torch.empty((batch, directions, num_heads, length), device=q_raw.device,
                          dtype=torch.float32)
        lib = hip.load_library()
        hip.check(lib.vh_qnorm_forward(
            hip.ptr(q_raw_c), hip.dtype_code(q_raw_c.dtype), hip.ptr(out), hip.ptr(inv), batch,
            directions, length, int(num_heads), int(head_dim), hip.stream_of(q_raw_c)),
            "vh_qnorm_forward")
        ctx.save_for_backward(out, inv)
        ctx.raw = (q_raw_c.dtype, int(num_heads), int(head_dim))
        return out

    @staticmethod
    @on_tensor_device
    def backward(ctx, d_q_out):
        """Reference ``utils/query_normalization.py:67-76``: the raw query's gradient
        ``[B, 4, N, heads*d]`` in its dtype."""
        out, inv = ctx.saved_tensors
        dtype, heads, head_dim = ctx.raw
        batch, directions, _, length, _ = out.shape
        g = d_q_out.float().contiguous()
        dq = torch.empty((batch, directions, length, heads * head_dim), device=out.device, dtype=dtype)
        lib = hip.load_library()
        hip.check(lib.vh_qnorm_backward(
            hip.ptr(g), hip.ptr(out), hip.ptr(inv), hip.ptr(dq), hip.dtype_code(dtype), batch, directions, length,
            heads, head_dim, hip.stream_of(out)), "vh_qnorm_backward")
        return dq, None, None


def can_fuse_qnorm(q_raw, num_heads, head_dim):
    """Reference eligibility test (``utils/query_normalization.py:74-83``)."""
    if not q_raw.is_cuda or q_raw.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        return False
    if q_raw.dim() != 4 or q_raw.shape[1] != 4:
        return False
    if int(head_dim) not in {4, 8, 16, 32, 64}:
        return False
    return int(q_raw.shape[-1]) == int(num_heads) * int(head_dim)


def visionhope_qnorm(q_raw, num_heads, head_dim):
    return VisionHOPEQNormFunction.apply(q_raw, int(num_heads), int(head_dim))
