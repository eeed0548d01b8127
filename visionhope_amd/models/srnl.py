"""Self-referential nested learning (SRNL): the five-memory chunked recurrence as a module.

The public surface is that of the reference's ``models/srnl.py:20-190``: constructor and
its checks, parameter names, shapes and initialisation, ``inference_status`` and its
reason strings, and the error types and messages of ``forward``.  Underneath there is one
computation: every call is a single native scan of the packed lines
(``srnl_core.chunk.srnl_scan``, or ``srnl_core.fused.srnl_sequence_inference`` on the
inference path), given one chunk length per direction.  The reference instead picks one of
several CUDA kernels by chunk length, map shape and query dtype (``srnl.py:128-169``);
the MI355X scan has none of those limits.
"""

import torch
from torch import nn
from torch.nn import functional as F
from torch.nn.init import trunc_normal_

from .srnl_core import MAX_CHUNK, SUPPORTED_HEAD_DIMS
from .srnl_core.chunk import srnl_scan
from ..utils.query_normalization import can_fuse_qnorm, visionhope_qnorm

_IO_DTYPES = (torch.float16, torch.bfloat16, torch.float32)
_MATRIX_MEMORIES = ("M_m_0", "M_v_0", "M_k_0")     # content, value, key
_VECTOR_MEMORIES = ("M_eta_0", "M_alpha_0")        # learning rate, retention
# A standalone sequence with chunk_size=None is cut into chunks of this many tokens.
DEFAULT_SEQUENCE_CHUNK = MAX_CHUNK


class SRNL(nn.Module):
    """The SRNL recurrence over ``directions`` scans of ``dim`` channels in heads of
    ``head_dim``, with FP32 memories learned per (direction, head).

    Two calling conventions:

    * standalone: ``x`` and optional ``queries`` of shape ``[B, N, dim]`` (one direction;
      queries default to ``x``), output ``[B, N, dim]``;
    * packed (the operator's): ``x`` ``[B, directions, heads, N, head_dim]`` and raw
      queries ``[B, directions, N, dim]`` (default: ``x`` regrouped), output like ``x``.

    Queries are normalised per head inside the scan.  ``chunk_size=None`` means 64-token
    chunks for standalone sequences and the row length (row scans) or column length
    (column scans) when ``spatial_shape=(H, W)`` is given.  A padded last chunk affects
    nothing but its own tokens.  ``fast_inference`` switches eval-mode, gradient-free calls
    to the inference entry point; otherwise calls are differentiable.
    """

    def __init__(self, dim, head_dim=16, chunk_size=None, directions=1, *,
                 fast_inference=False, _initialize=True):
        super().__init__()
        if head_dim not in SUPPORTED_HEAD_DIMS or dim <= 0 or dim % head_dim:
            raise ValueError(f"dim must be positive and divisible by head_dim in {SUPPORTED_HEAD_DIMS}")
        if directions not in (1, 2, 4):
            raise ValueError("directions must be 1, 2, or 4")
        if chunk_size is not None and (not isinstance(chunk_size, int) or chunk_size <= 0):
            raise ValueError("chunk_size must be a positive integer or None")
        if not isinstance(fast_inference, bool):
            raise TypeError("fast_inference must be a bool")
        self.dim, self.head_dim = int(dim), int(head_dim)
        self.num_heads = self.dim // self.head_dim
        self.directions = int(directions)
        self.chunk_size = chunk_size
        self.fast_inference = fast_inference
        self.memory_init_std = 0.01
        per_state = (self.directions, self.num_heads)
        for name in _MATRIX_MEMORIES:
            self.register_parameter(name, nn.Parameter(torch.empty(*per_state, self.head_dim, self.head_dim)))
        for name in _VECTOR_MEMORIES:
            self.register_parameter(name, nn.Parameter(torch.empty(*per_state, self.head_dim)))
        if _initialize:
            self.reset_parameters()

    @property
    def initial_memories(self):
        """Content, value, key, learning-rate, and retention memories, in core order."""
        return tuple(getattr(self, name) for name in _MATRIX_MEMORIES + _VECTOR_MEMORIES)

    def reset_parameters(self):
        """Matrices: truncated normal of std 0.01; gate vectors: zero (reference
        ``srnl.py:70-74``), so an untrained module has constant gates."""
        for name in _MATRIX_MEMORIES:
            trunc_normal_(getattr(self, name), std=self.memory_init_std)
        for name in _VECTOR_MEMORIES:
            nn.init.zeros_(getattr(self, name))

    # ---- path selection ---------------------------------------------------------------

    def _inference_path(self, x, query_dtype):
        """("sequence", None) when the inference entry point applies, else ("ordinary",
        the first reason it does not)."""
        blockers = (
            (not self.fast_inference, "Fast inference is disabled"),
            (self.training, "The module is in training mode"),
            (torch.is_grad_enabled(), "Gradients are enabled"),
            (not x.is_cuda, "SRNL requires CUDA inputs"),
            (x.dtype not in _IO_DTYPES, "SRNL requires FP16, BF16, or FP32 inputs"),
            (query_dtype != x.dtype, "Fast inference requires matching input and query dtypes"),
        )
        reason = next((why for blocked, why in blockers if blocked), None)
        return ("ordinary", reason) if reason else ("sequence", None)

    def inference_status(self, x, queries=None):
        """Report path selection for valid inputs in the current eval/grad context."""
        path, reason = self._inference_path(x, x.dtype if queries is None else queries.dtype)
        return {"path": path, "reason": reason}

    def _validate_memories(self, device):
        """The five memories, checked for shape, floating dtype and device."""
        shapes = [(self.directions, self.num_heads, self.head_dim, self.head_dim)] * 3
        shapes += [(self.directions, self.num_heads, self.head_dim)] * 2
        states = self.initial_memories
        for i, (state, shape) in enumerate(zip(states, shapes)):
            if (not isinstance(state, torch.Tensor) or tuple(state.shape) != shape
                    or not state.is_floating_point() or state.device != device):
                raise ValueError(f"SRNL memory {i} must be floating point, shape {shape}, on {device}")
        return states

    def _chunk_lengths(self, spatial_shape):
        """One chunk length per direction."""
        if self.chunk_size is not None:
            return [self.chunk_size] * self.directions
        if spatial_shape is None:
            return [DEFAULT_SEQUENCE_CHUNK] * self.directions
        height, width = spatial_shape
        return [width, width, height, height]   # row scans, then column scans

    def _unit_queries(self, queries):
        """Raw ``[B, R, N, dim]`` queries -> unit FP32 ``[B, R, heads, N, head_dim]``, for
        queries whose dtype differs from x's (the scan then reads them as given)."""
        if can_fuse_qnorm(queries, self.num_heads, self.head_dim):
            return visionhope_qnorm(queries, self.num_heads, self.head_dim)
        batch, directions, length, _ = queries.shape
        grouped = queries.reshape(batch, directions, length, self.num_heads, self.head_dim).transpose(2, 3)
        return F.normalize(grouped.float(), p=2.0, dim=-1, eps=1e-12).contiguous()

    # ---- computation ------------------------------------------------------------------

    def _packed_forward(self, x, queries, spatial_shape):
        batch, directions, heads, length, head_dim = x.shape
        if (directions, heads, head_dim) != (self.directions, self.num_heads, self.head_dim):
            raise ValueError("Packed input dimensions do not match this SRNL instance")
        if tuple(queries.shape) != (batch, directions, length, self.dim):
            raise ValueError("Packed queries must have shape [B, directions, N, dim]")
        if not x.is_cuda or x.device != queries.device:
            raise ValueError("SRNL inputs and memories must be on the same CUDA device")
        if x.dtype not in _IO_DTYPES:
            raise TypeError("SRNL input must be FP16, BF16, or FP32")
        if queries.dtype not in _IO_DTYPES:
            raise TypeError("SRNL queries must be FP16, BF16, or FP32")
        states = self._validate_memories(x.device)
        if batch <= 0 or length <= 0:
            raise ValueError("SRNL requires nonempty batches and sequences")
        if spatial_shape is not None:
            height, width = spatial_shape
            if min(height, width) <= 0 or height * width != length or directions != 4:
                raise ValueError("spatial_shape must match the four serialized image scans")
        chunks = self._chunk_lengths(spatial_shape)
        if self._inference_path(x, queries.dtype)[0] == "sequence":
            from .srnl_core.fused import srnl_sequence_inference

            return srnl_sequence_inference(states, x, queries, chunks)
        if queries.dtype == x.dtype:
            return srnl_scan(states, x, queries, chunks, q_raw=True)
        return srnl_scan(states, x, self._unit_queries(queries), chunks, q_raw=False)

    def forward(self, x, queries=None, *, spatial_shape=None):
        if x.ndim == 5:
            if queries is None:
                queries = x.transpose(2, 3).flatten(3)
            return self._packed_forward(x, queries, spatial_shape)
        if x.ndim != 3 or self.directions != 1 or x.shape[-1] != self.dim:
            raise ValueError("Standalone SRNL expects [B, N, dim] and directions=1")
        queries = x if queries is None else queries
        if queries.shape != x.shape:
            raise ValueError("Standalone queries must have the same shape as input")
        batch, length, _ = x.shape
        lines = x.reshape(batch, 1, length, self.num_heads, self.head_dim).transpose(2, 3).contiguous()
        y = self._packed_forward(lines, queries.unsqueeze(1), spatial_shape)
        return y[:, 0].transpose(1, 2).reshape(batch, length, self.dim)

    def extra_repr(self):
        return (f"dim={self.dim}, head_dim={self.head_dim}, directions={self.directions}, "
                f"chunk_size={self.chunk_size}, fast_inference={self.fast_inference}")
