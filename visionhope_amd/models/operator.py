"""The four-direction VisionHOPE operator on a spatial feature map.

The public surface is that of the reference's ``models/operator.py:15-193``: constructor
arguments and checks, parameter names and shapes (``W_q``, ``d_skip``,
``direction_scale`` / ``direction_logits``), ``project_queries``, ``serialize``,
``direction_weights``, ``inference_status`` and its reasons, and the error types and
messages.  The implementation has three execution paths:

* spatial (inference, chunks = row / column lengths): the native spatial entry reads the
  channels-last input and query maps directly, scans the four orders and fuses them in
  one readout; no serialized copy of x or q is made;
* sequence (inference, any other fixed chunk length): the packed native scan over
  serialized copies, then the native direction fusion;
* ordinary (training or gradients enabled): the same packed scan and fusion through
  their autograd Functions.
"""

import torch
from torch import nn
from torch.nn import functional as F
from torch.nn.init import trunc_normal_

from .srnl import SRNL
from ..utils.cached_params import linear_weights
from ..utils.cuda import on_tensor_device
from ..utils.direction_fusion import visionhope_postprocess_scale

_MERGE_MODES = ("sum", "scale", "softmax")


def scan_orders(seq_hw, height, width):
    """Row-major tokens ``[B, H*W, C]`` -> the four scan orders ``[B, 4, H*W, C]``: row-major,
    row-major reversed, column-major, column-major reversed (scan index maps t0..t3 of
    ``operator.py:79-86``)."""
    batch, length, channels = seq_hw.shape
    col_major = seq_hw.reshape(batch, height, width, channels).transpose(1, 2).reshape(batch, length, channels)
    return torch.stack((seq_hw, seq_hw.flip(1), col_major, col_major.flip(1)), dim=1)


def _query_dtype(x):
    """The dtype W_q produces for x: autocast's on CUDA when it is enabled."""
    if x.is_cuda and torch.is_autocast_enabled("cuda"):
        return torch.get_autocast_dtype("cuda")
    return x.dtype


class VisionHOPEOperator(nn.Module):
    """SRNL over the four row/column scans of a ``[B, dim, H, W]`` map, with a learned
    channel-wise skip and a channel-wise merge of the four directions.

    ``W_q`` projects each pixel once and every scan reuses its query.  ``d_skip`` is
    ``[heads, head_dim]`` (shared by the directions) or ``[4, heads, head_dim]``
    (``share_direction_skip=False``).  ``direction_merge``: "scale" (learned
    ``direction_scale``), "softmax" (4 x softmax of ``direction_logits`` over directions)
    or "sum".  ``fast_inference`` is the SRNL's flag (shared).
    """

    def __init__(self, dim, head_dim=16, chunk_size=None, direction_merge="scale",
                 share_direction_skip=True, *, fast_inference=False, _initialize=True):
        super().__init__()
        if not isinstance(share_direction_skip, bool):
            raise TypeError("share_direction_skip must be a bool")
        if direction_merge not in _MERGE_MODES:
            raise ValueError("direction_merge must be sum, scale, or softmax")
        self.dim, self.head_dim = int(dim), int(head_dim)
        self.share_direction_skip = share_direction_skip
        self.direction_merge = direction_merge
        self.srnl = SRNL(dim, head_dim, chunk_size, directions=4, fast_inference=fast_inference,
                         _initialize=False)
        self.num_heads = self.srnl.num_heads
        self.W_q = nn.Linear(dim, dim)
        skip_shape = (self.num_heads, self.head_dim)
        self.d_skip = nn.Parameter(torch.zeros(skip_shape if share_direction_skip else (4,) + skip_shape))
        self.direction_scale = nn.Parameter(torch.ones(4, dim)) if direction_merge == "scale" else None
        self.direction_logits = nn.Parameter(torch.zeros(4, dim)) if direction_merge == "softmax" else None
        if _initialize:
            self.reset_parameters()

    @property
    def fast_inference(self):
        return self.srnl.fast_inference

    @fast_inference.setter
    def fast_inference(self, enabled):
        self.srnl.fast_inference = enabled

    def reset_parameters(self):
        """SRNL memories as ``SRNL.reset_parameters``; ``W_q`` truncated normal (std 0.02)
        with zero bias; zero skip; unit scales, zero logits."""
        self.srnl.reset_parameters()
        trunc_normal_(self.W_q.weight, std=0.02)
        nn.init.zeros_(self.W_q.bias)
        nn.init.zeros_(self.d_skip)
        for param, value in ((self.direction_scale, 1.0), (self.direction_logits, 0.0)):
            if param is not None:
                nn.init.constant_(param, value)

    def project_queries(self, seq_hw, height, width):
        """Queries of the four scan orders ``[B, 4, H*W, dim]`` from row-major tokens
        ``[B, H*W, dim]``: ``W_q`` is applied once, then reordered."""
        return scan_orders(self.W_q(seq_hw), height, width)

    def announce_query_projection(self, x_nhwc):
        """Runs ``W_q``'s registered forward pre-hooks with the tensor about to be projected,
        for inference paths that compute the projection without calling the module (a
        native kernel, or a cached-weight product), so that hooks such as the query-once
        audit see every projection exactly as a module call would show it."""
        for hook in tuple(self.W_q._forward_pre_hooks.values()):
            hook(self.W_q, (x_nhwc,))

    def direction_weights(self):
        """``[4, dim]`` merge weights of the four directions."""
        if self.direction_merge == "scale":
            return self.direction_scale
        if self.direction_merge == "softmax":
            return 4.0 * torch.softmax(self.direction_logits, dim=0)
        return self.d_skip.new_ones((4, self.dim))

    @staticmethod
    def serialize(x, seq_hw=None):
        """``[B, C, H, W]`` -> the four scan orders ``[B, 4, H*W, C]``."""
        if seq_hw is None:
            seq_hw = x.flatten(2).transpose(1, 2)
        return scan_orders(seq_hw, x.shape[-2], x.shape[-1])

    # ---- path selection ---------------------------------------------------------------

    def _inference_path(self, x):
        if self.training:
            return "ordinary", "The operator is in training mode"
        path, reason = self.srnl._inference_path(x, _query_dtype(x))
        if path == "ordinary":
            return path, reason
        height, width = x.shape[-2:]
        chunk = self.srnl.chunk_size
        return ("spatial", None) if chunk is None or chunk == height == width else ("sequence", None)

    def inference_status(self, x):
        """Report path selection for a valid NCHW input in the current context."""
        path, reason = self._inference_path(x)
        return {"path": path, "reason": reason}

    # ---- computation ------------------------------------------------------------------

    def forward(self, x, *, channels_last=None):
        if x.ndim != 4 or x.shape[1] != self.dim:
            raise ValueError(f"VisionHOPEOperator expects [B, {self.dim}, H, W]")
        if channels_last is None:
            channels_last = x.is_contiguous(memory_format=torch.channels_last)
        path = self._inference_path(x)[0]
        if path == "ordinary":
            return self._sequence_forward(x, channels_last)
        out_nchw = self._forward_fast(x, path).permute(0, 3, 1, 2)
        return out_nchw.contiguous(memory_format=torch.channels_last if channels_last else torch.contiguous_format)

    def _sequence_forward(self, x, channels_last, *, memories=None):
        """Packed scan of the serialized orders, then the native restoring fusion.  With
        ``memories`` (the inference sequence path) the scan is the gradient-free entry."""
        batch, _, height, width = x.shape
        seq_hw = x.flatten(2).transpose(1, 2)
        lines = scan_orders(seq_hw, height, width)
        lines = lines.reshape(batch, 4, height * width, self.num_heads, self.head_dim).transpose(2, 3).contiguous()
        queries = self.project_queries(seq_hw, height, width)
        if memories is None:
            y = self.srnl(lines, queries, spatial_shape=(height, width))
        else:
            from .srnl_core.fused import srnl_sequence_inference

            y = srnl_sequence_inference(memories, lines, queries, [self.srnl.chunk_size] * 4)
        # Every merge mode runs the native fusion kernel (FP32 skip and weights; the
        # reference's eligibility test is can_fuse_scale_postprocess, operator.py:116-119).
        return visionhope_postprocess_scale(y, lines, self.d_skip.float(), self.direction_weights().float(),
                                            height, width, channels_last)

    def _merge_weights(self):
        """FP32 merge weights for the inference kernels (no autograd)."""
        if self.direction_merge == "softmax":
            return 4.0 * torch.softmax(self.direction_logits.detach().float(), dim=0)
        return self.direction_weights().detach().float()

    @on_tensor_device
    def _forward_fast(self, x, path):
        """Inference forward, returning ``[B, H, W, dim]`` FP32 (contiguous NHWC, what the
        output projection reads)."""
        if torch.jit.is_tracing():
            raise RuntimeError("SRNL TorchScript tracing is unsupported; use eager or CUDA Graph inference.")
        if x.ndim != 4 or not x.is_cuda or x.shape[1] != self.dim or min(x.shape) <= 0:
            raise ValueError(f"Fused VisionHOPE expects nonempty CUDA [B, {self.dim}, H, W]")
        height, width = x.shape[-2:]
        memories = self.srnl._validate_memories(x.device)
        skip_shape = (self.num_heads, self.head_dim) if self.share_direction_skip else (4, self.num_heads,
                                                                                        self.head_dim)
        if self.d_skip.shape != skip_shape or self.d_skip.device != x.device:
            raise ValueError("Directional skip has an invalid shape or device")
        for weights in (self.direction_scale, self.direction_logits):
            if weights is not None and (weights.shape != (4, self.dim) or weights.device != x.device):
                raise ValueError("Directional fusion weights have an invalid shape or device")
        if path == "sequence":
            return self._sequence_forward(x, True, memories=memories).permute(0, 2, 3, 1).contiguous()
        from .srnl_core.fused import srnl_spatial_inference

        x_nhwc = x.permute(0, 2, 3, 1)
        if torch.is_autocast_enabled("cuda"):
            # autocast's linear, with the weight cast once and cached instead of per call
            weight, bias = linear_weights(self.W_q, torch.get_autocast_dtype("cuda"))
            self.announce_query_projection(x_nhwc)
            q_nhwc = F.linear(x_nhwc.to(weight.dtype), weight, bias)
        else:
            q_nhwc = self.W_q(x_nhwc)
        return srnl_spatial_inference(memories, x_nhwc, q_nhwc, self.d_skip, self._merge_weights(),
                                      (width, width, height, height))
