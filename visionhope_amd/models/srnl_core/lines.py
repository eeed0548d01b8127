"""Long chunks and rectangular row/column scans (replaces ``models/srnl_core/lines.py``).

The reference needs separate tiled kernels once a chunk exceeds 64 tokens or the row and
column scans differ in length (``lines.py:183-671``).  The MI355X scan takes one chunk
length per direction and tiles tokens internally, so both functions below are the same
differentiable native scan (``srnl_scan``) with the reference's argument checks; gradients
exist for chunks of up to 256 tokens.
"""

import torch

from .chunk import MAX_CHUNK, SUPPORTED_HEAD_DIMS, srnl_scan


def _check_lines(x, q_raw, num_heads, head_dim, directions_ok, what):
    if torch.jit.is_tracing():
        raise RuntimeError("SRNL TorchScript tracing is unsupported; use eager or CUDA Graph inference.")
    if not x.is_cuda:
        raise RuntimeError(f"SRNL {what} qraw CUDA kernel requires CUDA tensors.")
    if x.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise RuntimeError(f"SRNL {what} qraw CUDA kernel supports fp16/bf16/fp32 x, got {x.dtype}.")
    if q_raw.dtype != x.dtype:
        raise RuntimeError(
            f"SRNL {what} qraw CUDA kernel expects q_raw dtype to match x dtype, got {q_raw.dtype} vs {x.dtype}.")
    batch, directions, heads, length, d = x.shape
    if directions not in directions_ok or heads != num_heads or d != head_dim:
        raise AssertionError(f"Invalid x shape for {what} qraw kernel.")
    if q_raw.dim() != 4 or tuple(q_raw.shape[:3]) != (batch, directions, length):
        raise AssertionError(f"Invalid q_raw shape for {what} qraw kernel.")
    if q_raw.shape[3] != num_heads * head_dim:
        raise AssertionError("q_raw channel count does not match num_heads * head_dim.")
    if head_dim not in SUPPORTED_HEAD_DIMS:
        raise AssertionError(f"{what} CUDA kernel requires head_dim in {SUPPORTED_HEAD_DIMS}, got {head_dim}.")


def srnl_long_chunk(M_m_0, M_v_0, M_k_0, M_eta_0, M_alpha_0, x, q_raw, chunk_size, num_heads, head_dim):
    """Chunks longer than the reference's 64-token kernel, 1, 2 or 4 directions
    (reference ``lines.py:183-399``)."""
    num_heads, head_dim, chunk_size = int(num_heads), int(head_dim), int(chunk_size)
    _check_lines(x, q_raw, num_heads, head_dim, (1, 2, 4), "large-line")
    if chunk_size <= MAX_CHUNK:
        raise ValueError("large-line CUDA kernel is only intended for chunk_size > base MAX_CHUNK.")
    return srnl_scan((M_m_0, M_v_0, M_k_0, M_eta_0, M_alpha_0), x, q_raw, [chunk_size] * x.shape[1], q_raw=True)


def srnl_variable_lines(M_m_0, M_v_0, M_k_0, M_eta_0, M_alpha_0, x, q_raw, row_chunk_size,
                        col_chunk_size, num_heads, head_dim):
    """Row scans chunked by W and column scans by H (reference ``lines.py:402-671``)."""
    num_heads, head_dim = int(num_heads), int(head_dim)
    _check_lines(x, q_raw, num_heads, head_dim, (4,), "varline")
    row, col = int(row_chunk_size), int(col_chunk_size)
    length = x.shape[3]
    if row <= 0 or col <= 0 or length % row or length % col:
        raise ValueError("varline chunk sizes must divide the serialized length")
    return srnl_scan((M_m_0, M_v_0, M_k_0, M_eta_0, M_alpha_0), x, q_raw, [row, row, col, col], q_raw=True)
