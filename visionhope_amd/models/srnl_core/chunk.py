"""SRNL forward for packed sequences on MI355X (replaces ``models/srnl_core/chunk.py``).

The reference JIT-compiles CUDA with the stability constants baked in as
literals; here the same environment variables are read once at import
(``chunk.py:34-58``) and passed to the prebuilt HIP library as arguments.
Inputs may be FP16, BF16 or FP32; recurrence state is FP32.
"""

import math
import os

import torch

from ...utils import hip
from ...utils.autograd import backward_unavailable
from ...utils.cuda import on_tensor_device

MAX_CHUNK = 64            # the reference's short-chunk kernel limit (chunk.py:31); the default standalone chunk
BACKWARD_MAX_CHUNK = 256   # the backward kernel's longest chunk (the long-line range)
SUPPORTED_HEAD_DIMS = (4, 8, 16, 32, 64)


def _env_float(name, default):
    raw = os.environ.get(name)
    if raw is None:
        return float(default)
    try:
        return float(raw)
    except ValueError as exc:
        raise ValueError(f"{name} must be a float, got {raw!r}") from exc


STEP_SCALE = _env_float("VISIONHOPE_STEP_SCALE", 0.025)
MIN_RETENTION = _env_float("VISIONHOPE_MIN_RETENTION", 0.0)
RETENTION_BIAS = _env_float("VISIONHOPE_RETENTION_BIAS", 2.197224577)
INJECTION_MARGIN = _env_float("VISIONHOPE_INJECTION_MARGIN", 0.999)
SPECTRAL_CLAMP = True
SPECTRAL_MARGIN = _env_float("VISIONHOPE_SPECTRAL_MARGIN", 0.999999)

if not (0.0 <= MIN_RETENTION < 1.0):
    raise ValueError(f"MIN_RETENTION must be in [0, 1), got {MIN_RETENTION}")
if not (0.0 < INJECTION_MARGIN < 1.0):
    raise ValueError(f"INJECTION_MARGIN must be in (0, 1), got {INJECTION_MARGIN}")
if not (STEP_SCALE > 0.0):
    raise ValueError(f"STEP_SCALE must be positive, got {STEP_SCALE}")
if not (0.0 < SPECTRAL_MARGIN <= 1.0):
    raise ValueError(f"SPECTRAL_MARGIN must be in (0, 1], got {SPECTRAL_MARGIN}")


def srnl_consts():
    """The stability constants as the C ABI's ``vh_srnl_consts``."""
    return hip.make_consts(STEP_SCALE, MIN_RETENTION, RETENTION_BIAS, INJECTION_MARGIN,
                           SPECTRAL_CLAMP, SPECTRAL_MARGIN)


def _float_memories(memories, directions, heads, head_dim, n_flat):
    """Contiguous FP32 memories and whether they hold one state per line (chunk.py:192-215)."""
    m_m = memories[0]
    if m_m.dim() == 4:
        state_count, per_line = directions * heads, 0
    elif m_m.dim() == 5:
        state_count, per_line = n_flat, 1
    else:
        raise AssertionError(f"Expected memory tensors with 4 or 5 dims, got shape {tuple(m_m.shape)}.")
    mats = [m.detach().contiguous().view(state_count, head_dim, head_dim).float().contiguous()
            for m in memories[:3]]
    vecs = [m.detach().contiguous().view(state_count, head_dim).float().contiguous()
            for m in memories[3:]]
    return (*mats, *vecs), per_line


@on_tensor_device
def srnl_packed_forward(memories, x, q, chunk_sizes, *, q_raw):
    """y ``[B, R, heads, N, d]`` (x's dtype) for packed x and raw ``[B, R, N, C]`` or
    normalised ``[B, R, heads, N, d]`` FP32 queries, one chunk length per direction."""
    batch, directions, heads, length, head_dim = x.shape
    if len(chunk_sizes) != directions:
        raise ValueError("Provide one chunk length per direction")
    chunks = [int(c) for c in chunk_sizes]
    if min(chunks) <= 0:
        raise ValueError("chunk_size must be a positive integer")
    n_flat = batch * directions * heads
    states, per_line = _float_memories(memories, directions, heads, head_dim, n_flat)
    x_c = x.contiguous()
    q_c = q.contiguous() if q_raw else q.float().contiguous()
    out = torch.empty_like(x_c)
    lib = hip.load_library()
    max_chunks = max(math.ceil(length / c) for c in chunks)
    ws = hip.workspace(lib.vh_srnl_workspace_bytes(n_flat, max_chunks, head_dim), x.device)
    chunk_ptr, _keep = hip.int64_array(chunks)
    consts = srnl_consts()
    mem_ptrs = [hip.ptr(m) for m in states]
    if q_raw:
        rc = lib.vh_srnl_sequence_forward(
            hip.ptr(x_c), hip.ptr(q_c), hip.dtype_code(x_c.dtype), *mem_ptrs, per_line,
            hip.ptr(out), batch, directions, heads, length, head_dim, chunk_ptr,
            consts, hip.ptr(ws), ws.numel() * 4, hip.stream_of(x_c))
        hip.check(rc, "vh_srnl_sequence_forward")
    else:
        rc = lib.vh_srnl_forward(
            hip.ptr(x_c), hip.dtype_code(x_c.dtype), hip.ptr(q_c), *mem_ptrs, per_line,
            hip.ptr(out), batch, directions, heads, length, head_dim, chunk_ptr,
            consts, hip.ptr(ws), ws.numel() * 4, hip.stream_of(x_c))
        hip.check(rc, "vh_srnl_forward")
    return out


@on_tensor_device
def srnl_packed_backward(memories, x, q, chunk_sizes, dy, *, q_raw):
    """Gradients of ``srnl_packed_forward`` (same arguments) for the output gradient
    ``dy [B, R, heads, N, d]``: ``(dM_m, dM_v, dM_k, dM_eta, dM_alpha, dx, dq)`` shaped and
    typed like the corresponding inputs (``vh_srnl_backward``; reference
    ``chunk.cu:511-1057``, and ``lines.cu:252-760`` for chunks of 65 to 256 tokens).  The
    forward is recomputed from the inputs."""
    batch, directions, heads, length, head_dim = x.shape
    chunks = [int(c) for c in chunk_sizes]
    if len(chunks) != directions or min(chunks) <= 0 or max(chunks) > BACKWARD_MAX_CHUNK:
        raise ValueError(f"SRNL backward needs one chunk length in [1, {BACKWARD_MAX_CHUNK}] per direction")
    n_flat = batch * directions * heads
    states, per_line = _float_memories(memories, directions, heads, head_dim, n_flat)
    x_c = x.contiguous()
    q_c = q.contiguous() if q_raw else q.float().contiguous()
    dy_c = dy.float().contiguous()
    dx = torch.empty(x_c.shape, device=x.device, dtype=torch.float32)
    dq = torch.empty(q_c.shape, device=x.device, dtype=torch.float32)
    dmem = [torch.empty_like(m) for m in states]
    lib = hip.load_library()
    chunk_ptr, _keep = hip.int64_array(chunks)
    nbytes = lib.vh_srnl_backward_workspace_bytes(batch, directions, heads, length, head_dim, chunk_ptr)
    if nbytes == 0:
        raise ValueError(f"SRNL backward does not cover head_dim={head_dim} with chunks {chunks}")
    ws = hip.workspace(nbytes, x.device)
    hip.check(lib.vh_srnl_backward(
        hip.ptr(x_c), hip.ptr(q_c), hip.dtype_code(x_c.dtype), int(bool(q_raw)), hip.ptr(dy_c),
        *[hip.ptr(m) for m in states], per_line, hip.ptr(dx), hip.ptr(dq), *[hip.ptr(m) for m in dmem],
        batch, directions, heads, length, head_dim, chunk_ptr, srnl_consts(), hip.ptr(ws), ws.numel() * 4,
        hip.stream_of(x_c)), "vh_srnl_backward")
    grads = [g.view(m.shape).to(m.dtype) for g, m in zip(dmem, memories)]
    return (*grads, dx.to(x.dtype), dq.to(q.dtype))


class SRNLScanFunction(torch.autograd.Function):
    """The packed recurrence with autograd, for every path that needs gradients.

    One native forward (``srnl_packed_forward``) and one native backward
    (``srnl_packed_backward``) cover what the reference splits over its short-chunk,
    long-chunk and variable-line kernels (``chunk.py:168-588``, ``lines.py:183-671``):
    the scan takes one chunk length per direction, any length in the forward and up to
    ``BACKWARD_MAX_CHUNK`` in the backward.  ``q_raw``: queries are the unnormalised
    ``[B, R, N, C]`` projections in x's dtype; otherwise unit FP32 ``[B, R, heads, N, d]``.
    """

    @staticmethod
    def forward(ctx, M_m_0, M_v_0, M_k_0, M_eta_0, M_alpha_0, x, q, chunks, q_raw):
        if torch.jit.is_tracing():
            raise RuntimeError("SRNL TorchScript tracing is unsupported; use eager or CUDA Graph inference.")
        memories = (M_m_0, M_v_0, M_k_0, M_eta_0, M_alpha_0)
        ctx.save_for_backward(*memories, x, q)
        ctx.chunks, ctx.q_raw = list(chunks), bool(q_raw)
        return srnl_packed_forward(memories, x, q, ctx.chunks, q_raw=ctx.q_raw)

    @staticmethod
    def backward(ctx, dY):
        if max(ctx.chunks) > BACKWARD_MAX_CHUNK:
            backward_unavailable(f"SRNL scan with a chunk of {max(ctx.chunks)} tokens")
        *memories, x, q = ctx.saved_tensors
        grads = srnl_packed_backward(memories, x, q, ctx.chunks, dY, q_raw=ctx.q_raw)
        return (*grads, None, None)


def srnl_scan(memories, x, q, chunks, *, q_raw):
    """Differentiable packed SRNL: y ``[B, R, heads, N, d]`` in x's dtype."""
    return SRNLScanFunction.apply(*memories, x, q, tuple(int(c) for c in chunks), bool(q_raw))


def _check_kernel_inputs(x, head_dim, what):
    if not x.is_cuda:
        raise RuntimeError(f"{what} requires CUDA tensors.")
    if x.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise RuntimeError(f"{what} supports fp16/bf16/fp32 x, got {x.dtype}.")
    if head_dim not in SUPPORTED_HEAD_DIMS:
        raise AssertionError(f"SRNL CUDA kernel requires head_dim in {SUPPORTED_HEAD_DIMS}, got {head_dim}.")


def can_fuse_raw_query(x, q_raw, num_heads, head_dim):
    """Reference eligibility test (``chunk.py:602-619``)."""
    if not (x.is_cuda and q_raw.is_cuda):
        return False
    if x.dtype not in (torch.float16, torch.bfloat16, torch.float32) or q_raw.dtype != x.dtype:
        return False
    if x.dim() != 5 or q_raw.dim() != 4:
        return False
    if x.shape[1] != 4 or q_raw.shape[1] != 4:
        return False
    if int(head_dim) not in SUPPORTED_HEAD_DIMS:
        return False
    return (
        int(x.shape[0]) == int(q_raw.shape[0])
        and int(x.shape[3]) == int(q_raw.shape[2])
        and int(x.shape[2]) == int(num_heads)
        and int(x.shape[4]) == int(head_dim)
        and int(q_raw.shape[3]) == int(num_heads) * int(head_dim)
    )


def srnl_raw_query(M_m_0, M_v_0, M_k_0, M_eta_0, M_alpha_0, x, q_raw, chunk_size, num_heads, head_dim):
    """Four directions with raw queries in x's dtype, one chunk length for all (reference
    ``chunk.py:622-625``, chunks of at most 64 there; any length here)."""
    _check_kernel_inputs(x, int(head_dim), "SRNL qraw CUDA kernel")
    if q_raw.dtype != x.dtype:
        raise RuntimeError(
            f"SRNL qraw CUDA kernel expects q_raw dtype to match x dtype, got {q_raw.dtype} vs {x.dtype}.")
    if not can_fuse_raw_query(x, q_raw, num_heads, head_dim):
        raise AssertionError("Invalid x shape for SRNL qraw kernel.")
    return srnl_scan((M_m_0, M_v_0, M_k_0, M_eta_0, M_alpha_0), x, q_raw, [int(chunk_size)] * 4, q_raw=True)


def srnl_normalized_query(M_m_0, M_v_0, M_k_0, M_eta_0, M_alpha_0, x, q, chunk_size):
    """Unit FP32 queries ``[B, R, heads, N, d]`` (reference ``chunk.py:628-634``)."""
    if x.dtype in (torch.float16, torch.bfloat16, torch.float32) and q.dtype == torch.float32:
        _check_kernel_inputs(x, int(x.shape[-1]), "SRNL CUDA kernel")
        return srnl_scan((M_m_0, M_v_0, M_k_0, M_eta_0, M_alpha_0), x, q, [int(chunk_size)] * x.shape[1],
                         q_raw=False)
    raise RuntimeError("The release HOPE CUDA path expects fp16/bf16/fp32 x and fp32 normalized q.")


srnl_normalized_query.supports_broadcast_state = True
