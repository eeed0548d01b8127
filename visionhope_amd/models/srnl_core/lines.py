"""Long chunks and rectangular row/column scans (replaces ``models/srnl_core/lines.py``),
forward and (chunks of up to 256 tokens) backward.

The reference needs separate tiled kernels once a chunk exceeds 64 tokens
(``lines.py:183-671``); the MI355X scan tiles tokens internally, so both cases
run the same native forward with per-direction chunk lengths.
"""

import torch

from .chunk import BACKWARD_MAX_CHUNK, MAX_CHUNK, SUPPORTED_HEAD_DIMS, srnl_packed_backward, srnl_packed_forward
from ...utils.autograd import backward_unavailable


def _check_common(x, q_raw, num_heads, head_dim, directions_ok, what):
    if torch.jit.is_tracing():
        raise RuntimeError("SRNL TorchScript tracing is unsupported; use eager or CUDA Graph inference.")
    if not x.is_cuda:
        raise RuntimeError(f"SRNL {what} qraw CUDA kernel requires CUDA tensors.")
    if x.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise RuntimeError(f"SRNL {what} qraw CUDA kernel supports fp16/bf16/fp32 x, got {x.dtype}.")
    if q_raw.dtype != x.dtype:
        raise RuntimeError(
            f"SRNL {what} qraw CUDA kernel expects q_raw dtype to match x dtype, got {q_raw.dtype} vs {x.dtype}.")
    batch, directions, x_num_heads, seq_len, x_head_dim = x.shape
    if directions not in directions_ok or x_num_heads != num_heads or x_head_dim != head_dim:
        raise AssertionError(f"Invalid x shape for {what} qraw kernel.")
    if (q_raw.dim() != 4 or q_raw.shape[0] != batch or q_raw.shape[1] != directions
            or q_raw.shape[2] != seq_len):
        raise AssertionError(f"Invalid q_raw shape for {what} qraw kernel.")
    if q_raw.shape[3] != num_heads * head_dim:
        raise AssertionError("q_raw channel count does not match num_heads * head_dim.")
    if head_dim not in SUPPORTED_HEAD_DIMS:
        raise AssertionError(f"{what} CUDA kernel requires head_dim in {SUPPORTED_HEAD_DIMS}, got {head_dim}.")


class SRNLLongChunkFunction(torch.autograd.Function):
    """Forward of ``lines.py:183-399``: chunks longer than 64 tokens, 1/2/4 directions."""

    @staticmethod
    def forward(ctx, M_m_0, M_v_0, M_k_0, M_eta_0, M_alpha_0, x, q_raw, chunk_size, num_heads, head_dim):
        num_heads, head_dim, chunk_size = int(num_heads), int(head_dim), int(chunk_size)
        _check_common(x, q_raw, num_heads, head_dim, (1, 2, 4), "large-line")
        if chunk_size <= MAX_CHUNK:
            raise ValueError("large-line CUDA kernel is only intended for chunk_size > base MAX_CHUNK.")
        memories = (M_m_0, M_v_0, M_k_0, M_eta_0, M_alpha_0)
        ctx.save_for_backward(*memories, x, q_raw)
        ctx.chunks = [chunk_size] * x.shape[1]
        return srnl_packed_forward(memories, x, q_raw, ctx.chunks, q_raw=True)

    @staticmethod
    def backward(ctx, dY):
        """Reference ``lines.py:183-399`` (``lines.cu:252-760``): gradients of the memories, x
        and the raw queries, for chunks of up to 256 tokens."""
        *memories, x, q_raw = ctx.saved_tensors
        if max(ctx.chunks) > BACKWARD_MAX_CHUNK:
            backward_unavailable(f"SRNL long chunk above {BACKWARD_MAX_CHUNK}")
        grads = srnl_packed_backward(memories, x, q_raw, ctx.chunks, dY, q_raw=True)
        return (*grads, None, None, None, None)


class SRNLVariableLineFunction(torch.autograd.Function):
    """Forward of ``lines.py:402-643``: row scans chunked by W, column scans by H."""

    @staticmethod
    def forward(ctx, M_m_0, M_v_0, M_k_0, M_eta_0, M_alpha_0, x, q_raw, row_chunk_size, col_chunk_size,
                num_heads, head_dim):
        num_heads, head_dim = int(num_heads), int(head_dim)
        _check_common(x, q_raw, num_heads, head_dim, (4,), "varline")
        seq_len = x.shape[3]
        row, col = int(row_chunk_size), int(col_chunk_size)
        if row <= 0 or col <= 0 or seq_len % row or seq_len % col:
            raise ValueError("varline chunk sizes must divide the serialized length")
        memories = (M_m_0, M_v_0, M_k_0, M_eta_0, M_alpha_0)
        ctx.save_for_backward(*memories, x, q_raw)
        ctx.chunks = [row, row, col, col]
        return srnl_packed_forward(memories, x, q_raw, ctx.chunks, q_raw=True)

    @staticmethod
    def backward(ctx, dY):
        """Reference ``lines.py:645-671`` (``lines.cu:252-760``): gradients of the memories,
        x and the raw queries.  Native while both chunk lengths are at most 256."""
        *memories, x, q_raw = ctx.saved_tensors
        if max(ctx.chunks) > BACKWARD_MAX_CHUNK:
            backward_unavailable(f"SRNL variable lines with a chunk above {BACKWARD_MAX_CHUNK}")
        grads = srnl_packed_backward(memories, x, q_raw, ctx.chunks, dY, q_raw=True)
        return (*grads, None, None, None, None, None)


def srnl_long_chunk(M_m_0, M_v_0, M_k_0, M_eta_0, M_alpha_0, x, q_raw, chunk_size, num_heads, head_dim):
    return SRNLLongChunkFunction.apply(
        M_m_0, M_v_0, M_k_0, M_eta_0, M_alpha_0, x, q_raw, int(chunk_size), int(num_heads), int(head_dim))


def srnl_variable_lines(M_m_0, M_v_0, M_k_0, M_eta_0, M_alpha_0, x, q_raw, row_chunk_size,
                        col_chunk_size, num_heads, head_dim):
    return SRNLVariableLineFunction.apply(
        M_m_0, M_v_0, M_k_0, M_eta_0, M_alpha_0, x, q_raw, int(row_chunk_size), int(col_chunk_size),
        int(num_heads), int(head_dim))
