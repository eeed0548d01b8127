"""Inference-only SRNL execution for spatial scans and general sequences
(replaces ``models/srnl_core/fused.py`` + ``csrc/fused.cu``).

``load_fused_cuda(io_dtype)`` returns an object exposing the reference's
pybind function names, backed by ``libvisionhope_hip.so``.  The operator's
own fast path uses ``srnl_spatial_inference`` instead, which reads the
channels-last activation and query maps directly (no serialized copies).
"""

from __future__ import annotations

import math

import torch

from .chunk import srnl_consts, srnl_packed_forward
from ...utils import hip
from ...utils.cached_params import contiguous_fp32
from ...utils.cuda import on_tensor_device

_IO_DTYPES = (torch.bfloat16, torch.float16, torch.float32)


def _fp32_states(states):
    return tuple(contiguous_fp32(state) for state in states)


@on_tensor_device
def srnl_spatial_inference(states, x_nhwc, q_nhwc, d_skip, weights, chunks):
    """Four-direction operator on channels-last maps.

    x_nhwc, q_nhwc: ``[B, H, W, C]`` (same dtype); states ``[4, heads, d, d]`` /
    ``[4, heads, d]``; d_skip ``C`` or ``4*C`` values; weights ``[4, C]``; chunks per
    direction.  Returns ``[B, H, W, C]`` FP32 = sum_r w_r (y_r + skip_r x), the
    result of ``operator.py:159-193`` / ``fused.cu:307-351``.
    """
    batch, height, width, channels = x_nhwc.shape
    head_dim = states[0].shape[-1]
    if q_nhwc.shape != x_nhwc.shape or q_nhwc.dtype != x_nhwc.dtype:
        raise ValueError("Spatial SRNL expects x and queries with the same [B, H, W, C] shape and dtype")
    mems = _fp32_states(states)
    skip = d_skip.detach().float().contiguous()
    wts = weights.detach().float().contiguous()
    if skip.numel() not in (channels, 4 * channels):
        raise RuntimeError("d_skip must contain C or 4*C values")
    x_c = x_nhwc.contiguous()
    q_c = q_nhwc.contiguous()
    out = torch.empty((batch, height, width, channels), device=x_nhwc.device, dtype=torch.float32)
    lib = hip.load_library()
    length = height * width
    max_chunks = max(math.ceil(length / int(c)) for c in chunks)
    ws = hip.workspace(lib.vh_srnl_workspace_bytes(batch * 4 * (channels // head_dim), max_chunks,
                                                   head_dim), x_nhwc.device)
    chunk_ptr, _keep = hip.int64_array(chunks)
    hip.check(lib.vh_srnl_spatial_forward(
        hip.ptr(x_c), hip.ptr(q_c), hip.dtype_code(x_c.dtype), *[hip.ptr(m) for m in mems],
        hip.ptr(skip), int(skip.numel() == 4 * channels), hip.ptr(wts), hip.ptr(out),
        batch, height, width, channels, head_dim, chunk_ptr, srnl_consts(), hip.ptr(ws),
        ws.numel() * 4, hip.stream_of(x_c)), "vh_srnl_spatial_forward")
    return out


def _chunk_array(chunks):
    return hip.int64_array([int(c) for c in chunks])


def srnl_spatial_workspace(x_nhwc, head_dim, chunks):
    """An uninitialised workspace for ``srnl_spatial_scan`` of x_nhwc ``[B, H, W, C]``."""
    batch, height, width, channels = x_nhwc.shape
    max_chunks = max(math.ceil(height * width / int(c)) for c in chunks)
    lib = hip.load_library()
    return hip.workspace(lib.vh_srnl_workspace_bytes(batch * 4 * (channels // head_dim), max_chunks, head_dim),
                         x_nhwc.device)


@on_tensor_device
def srnl_spatial_scan(states, x_nhwc, chunks, workspace=None):
    """First half of ``srnl_spatial_inference``: the four scans of x_nhwc ``[B, H, W, C]``.
    Returns the workspace holding every chunk-start content memory (``workspace`` when
    given, from ``srnl_spatial_workspace``), for ``srnl_spatial_readout``."""
    batch, height, width, channels = x_nhwc.shape
    head_dim = states[0].shape[-1]
    mems = _fp32_states(states)
    x_c = x_nhwc.contiguous()
    lib = hip.load_library()
    ws = srnl_spatial_workspace(x_nhwc, head_dim, chunks) if workspace is None else workspace
    chunk_ptr, _keep = _chunk_array(chunks)
    hip.check(lib.vh_srnl_spatial_scan(
        hip.ptr(x_c), hip.dtype_code(x_c.dtype), *[hip.ptr(m) for m in mems], batch, height, width, channels,
        head_dim, chunk_ptr, srnl_consts(), hip.ptr(ws), ws.numel() * 4, hip.stream_of(x_c)),
        "vh_srnl_spatial_scan")
    return ws


@on_tensor_device
def srnl_spatial_readout(workspace, x_nhwc, q_nhwc, d_skip, weights, chunks, head_dim, *, aux=None,
                         out_dtype=torch.float32, lepe=None):
    """Second half: sum_r w_r (y_r + skip_r x) (+ aux) as ``[B, H, W, C]`` ``out_dtype``
    (FP32 or x's dtype); aux is an optional x-dtype ``[B, H, W, C]`` addend.

    ``lepe = (taps, bias)`` (FP32 ``[25, C]`` taps-major and ``[C]`` or None) adds the
    block's 5x5 depthwise position encoding of x instead, computed in the same pass
    (``vh_srnl_spatial_readout_lepe``; output in x's dtype, no aux)."""
    batch, height, width, channels = x_nhwc.shape
    if q_nhwc.shape != x_nhwc.shape or q_nhwc.dtype != x_nhwc.dtype:
        raise ValueError("Spatial SRNL expects x and queries with the same [B, H, W, C] shape and dtype")
    if aux is not None and (aux.shape != x_nhwc.shape or aux.dtype != x_nhwc.dtype):
        raise ValueError("The readout addend must match x's shape and dtype")
    skip = d_skip.detach().float().contiguous()
    wts = weights.detach().float().contiguous()
    x_c, q_c = x_nhwc.contiguous(), q_nhwc.contiguous()
    if lepe is not None:
        taps, bias = lepe
        if aux is not None or out_dtype != x_nhwc.dtype:
            raise ValueError("The fused position encoding writes x's dtype and takes no addend")
        if taps.shape != (25, channels) or taps.dtype != torch.float32 or (
                bias is not None and (bias.shape != (channels,) or bias.dtype != torch.float32)):
            raise ValueError("Position encoding taps must be FP32 [25, C] and the bias FP32 [C]")
        taps_c = taps.contiguous()
        bias_c = None if bias is None else bias.contiguous()
        out = torch.empty((batch, height, width, channels), device=x_nhwc.device, dtype=out_dtype)
        lib = hip.load_library()
        chunk_ptr, _keep = _chunk_array(chunks)
        hip.check(lib.vh_srnl_spatial_readout_lepe(
            hip.ptr(x_c), hip.ptr(q_c), hip.dtype_code(x_c.dtype), hip.ptr(skip), int(skip.numel() == 4 * channels),
            hip.ptr(wts), hip.ptr(taps_c), hip.ptr(bias_c), hip.ptr(out), batch, height, width, channels, head_dim,
            chunk_ptr, hip.ptr(workspace), workspace.numel() * 4, hip.stream_of(x_c)),
            "vh_srnl_spatial_readout_lepe")
        return out
    aux_c = None if aux is None else aux.contiguous()
    out = torch.empty((batch, height, width, channels), device=x_nhwc.device, dtype=out_dtype)
    lib = hip.load_library()
    chunk_ptr, _keep = _chunk_array(chunks)
    hip.check(lib.vh_srnl_spatial_readout(
        hip.ptr(x_c), hip.ptr(q_c), hip.dtype_code(x_c.dtype), hip.ptr(skip), int(skip.numel() == 4 * channels),
        hip.ptr(wts), hip.ptr(aux_c), hip.ptr(out), hip.dtype_code(out_dtype), batch, height, width, channels,
        head_dim, chunk_ptr, hip.ptr(workspace), workspace.numel() * 4, hip.stream_of(x_c)),
        "vh_srnl_spatial_readout")
    return out


class FusedSRNLOps:
    """The functions of the reference's ``load_fused_cuda`` module (``fused.py:70-76``)."""

    def __init__(self, io_dtype):
        self.io_dtype = io_dtype

    def _check_line_inputs(self, X, Q_raw, D_skip, Dir_weight, what):
        if X.dtype != self.io_dtype or Q_raw.dtype != self.io_dtype:
            raise RuntimeError(f"{what} forward expects {self.io_dtype} X and Q_raw.")
        if D_skip.dtype != torch.float32 or Dir_weight.dtype != torch.float32:
            raise RuntimeError(f"{what} forward expects fp32 state, skip, and direction weights.")

    @on_tensor_device
    def srnl_line_forward_seq_noatomic(self, M_m_0, M_v_0, M_k_0, M_eta_0, M_alpha_0, X, Q_raw,
                                       D_skip, Dir_weight, H, W, D_int):
        """Serialized stacks ``X, Q_raw [B, 4, H*W, C]`` -> ``[B, H, W, C]`` FP32 (fused.cu:307-351)."""
        self._check_line_inputs(X, Q_raw, D_skip, Dir_weight, "line fused seq-layout no-atomic HOPE")
        batch, _, length, channels = X.shape
        H, W, D_int = int(H), int(W), int(D_int)
        if length != H * W or channels % D_int:
            raise RuntimeError("line fused seq-layout no-atomic HOPE got inconsistent H/W, C, and head_dim.")
        if D_skip.numel() not in (channels, 4 * channels):
            raise RuntimeError("d_skip must contain C or 4*C values")
        mems = _fp32_states((M_m_0, M_v_0, M_k_0, M_eta_0, M_alpha_0))
        x_c, q_c = X.contiguous(), Q_raw.contiguous()
        skip, wts = D_skip.contiguous(), Dir_weight.contiguous()
        out = torch.empty((batch, H, W, channels), device=X.device, dtype=torch.float32)
        lib = hip.load_library()
        ws = hip.workspace(lib.vh_srnl_workspace_bytes(batch * 4 * (channels // D_int), max(H, W), D_int),
                           X.device)
        hip.check(lib.vh_srnl_line_forward_seq_noatomic(
            hip.ptr(x_c), hip.ptr(q_c), hip.dtype_code(x_c.dtype), *[hip.ptr(m) for m in mems],
            hip.ptr(skip), int(skip.numel() == 4 * channels), hip.ptr(wts), hip.ptr(out),
            batch, H, W, channels, D_int, srnl_consts(), hip.ptr(ws), ws.numel() * 4,
            hip.stream_of(x_c)), "vh_srnl_line_forward_seq_noatomic")
        return out

    # The reference's other three spatial entries differ only in the input
    # layout (packed [B, 4, heads, L, d] vs serialized stacks) and in how the
    # four directions are summed (atomics vs a merge pass); the fusion here is
    # always the deterministic one.
    def srnl_line_forward_seq(self, *args):
        return self.srnl_line_forward_seq_noatomic(*args)

    def _packed_to_stack(self, X):
        batch, directions, heads, length, head_dim = X.shape
        return X.transpose(2, 3).reshape(batch, directions, length, heads * head_dim)

    def srnl_line_forward_noatomic(self, M_m_0, M_v_0, M_k_0, M_eta_0, M_alpha_0, X, Q_raw,
                                   D_skip, Dir_weight, H, W, D_int):
        return self.srnl_line_forward_seq_noatomic(M_m_0, M_v_0, M_k_0, M_eta_0, M_alpha_0,
                                                   self._packed_to_stack(X), Q_raw, D_skip,
                                                   Dir_weight, H, W, D_int)

    def srnl_line_forward(self, *args):
        return self.srnl_line_forward_noatomic(*args)

    def srnl_sequence_forward(self, M_m_0, M_v_0, M_k_0, M_eta_0, M_alpha_0, X, Q_raw, chunk_sizes):
        """Packed ``X [B, R, heads, N, d]``, raw ``Q_raw [B, R, N, C]`` (fused.cu:131-179)."""
        if not X.is_cuda or X.dim() != 5:
            raise RuntimeError("SRNL inference expects contiguous CUDA [B, directions, heads, N, d]")
        if X.dtype != self.io_dtype or Q_raw.dtype != X.dtype or Q_raw.device != X.device:
            raise RuntimeError("SRNL inference requires matching input/query dtype and device")
        batch, directions, heads, length, head_dim = X.shape
        if batch <= 0 or heads <= 0 or length <= 0 or directions not in (1, 2, 4):
            raise RuntimeError("SRNL inference requires nonempty inputs and 1, 2, or 4 directions")
        if head_dim not in (4, 8, 16, 32, 64):
            raise RuntimeError("Unsupported SRNL head dimension")
        if tuple(Q_raw.shape) != (batch, directions, length, heads * head_dim):
            raise RuntimeError("Invalid raw query shape")
        if len(chunk_sizes) != directions:
            raise RuntimeError("Provide one chunk length per direction")
        for state in (M_m_0, M_v_0, M_k_0):
            if state.dtype != torch.float32 or tuple(state.shape) != (directions, heads, head_dim, head_dim):
                raise RuntimeError("SRNL matrix memories must be contiguous FP32 [directions, heads, d, d]")
        for state in (M_eta_0, M_alpha_0):
            if state.dtype != torch.float32 or tuple(state.shape) != (directions, heads, head_dim):
                raise RuntimeError("SRNL vector memories must be contiguous FP32 [directions, heads, d]")
        if any(int(c) <= 0 for c in chunk_sizes):
            raise RuntimeError("Invalid SRNL chunk length or padded sequence length")
        return srnl_packed_forward((M_m_0, M_v_0, M_k_0, M_eta_0, M_alpha_0), X, Q_raw,
                                   list(chunk_sizes), q_raw=True)


_extensions = {}


def load_fused_cuda(io_dtype=torch.bfloat16):
    """Same contract as ``fused.py:56-80``; the kernels are prebuilt, nothing is compiled."""
    if io_dtype not in _IO_DTYPES:
        raise TypeError(f"SRNL inference supports FP16, BF16, and FP32, got {io_dtype}")
    hip.load_library()
    if io_dtype not in _extensions:
        _extensions[io_dtype] = FusedSRNLOps(io_dtype)
    return _extensions[io_dtype]


@on_tensor_device
def srnl_sequence_inference(states, x, queries, chunk_sizes):
    """Read a packed sequence without allocating backward intermediates (``fused.py:83-93``)."""
    if torch.jit.is_tracing():
        raise RuntimeError("SRNL TorchScript tracing is unsupported; use eager or CUDA Graph inference")
    if torch.is_grad_enabled():
        raise RuntimeError("SRNL inference requires disabled gradients")
    memories = tuple(state.contiguous().float() for state in states)
    return load_fused_cuda(x.dtype).srnl_sequence_forward(
        *memories, x.contiguous(), queries.contiguous(), chunk_sizes)
