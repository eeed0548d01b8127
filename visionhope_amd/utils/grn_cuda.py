"""Native GRN forward on MI355X (replaces ``utils/grn_cuda.py`` + ``utils/csrc/grn_cuda.cu``).

For C % 8 == 0 maps whose images split into at most 64 register-resident pieces, one
launch on the current stream reads x once: each piece publishes its per-channel sums of
x^2, waits for the other pieces of its image, then applies the FP32 affine output to the
rows it holds.  Other maps take two or three launches (partial sums, statistics, apply).
"""
import ctypes

import torch
from torch.autograd import Function

from . import hip
from .cuda import on_tensor_device

# One GRN workspace per (device, stream) outside graph capture, and one per captured graph.
# Its leading synchronisation words must be zero when a call starts and every call leaves
# them zero, so a buffer zeroed when it is created is reused as is; calls on one stream
# never overlap.  Inside a capture nothing done outside the graph can be relied on (graphs
# replay in any order, long after they were captured), so the first call of a capture
# creates the graph's own workspace, whose zero fill is a node of that graph ahead of the
# call, and the capture's later calls reuse it.  Captured workspaces are kept for the life
# of the process: a graph may be replayed at any time.
_STREAM_WORKSPACES = {}
_HEADER_FLOATS = 32768 // 4   # the synchronisation header of vh_grn_workspace_bytes


def _capture_id(lib, stream):
    """0 outside graph capture, else 1 + the capture's identifier (vh_stream_capture_id)."""
    capturing, ident = ctypes.c_int32(0), ctypes.c_uint64(0)
    hip.check(lib.vh_stream_capture_id(ctypes.c_void_p(stream.cuda_stream), ctypes.byref(capturing),
                                       ctypes.byref(ident)), "vh_stream_capture_id")
    return ident.value + 1 if capturing.value else 0


def _stream_workspace(nbytes, device):
    stream = torch.cuda.current_stream(device)
    key = (device.index, stream.cuda_stream, _capture_id(hip.load_library(), stream))
    ws = _STREAM_WORKSPACES.get(key)
    if ws is None or ws.numel() * 4 < nbytes:
        # zeroed on creation: in a capture, by a fill node of this graph
        ws = _STREAM_WORKSPACES[key] = torch.zeros(max(_HEADER_FLOATS, (int(nbytes) + 255) // 256 * 64),
                                                   dtype=torch.float32, device=device)
    return ws


def grn_wait_fallbacks(device=None):
    """How many times a workgroup of the one-pass GRN kernel, on any stream's workspace of
    ``device``, stopped waiting for the rest of its image and computed the image's
    statistics from its input itself (its output stays correct; a non-zero count shows
    that workgroups of one launch did not all run together).  Synchronises those streams:
    a diagnostic, not for use inside graph capture."""
    device = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
    lib = hip.load_library()
    total = 0
    for (index, handle, _), ws in list(_STREAM_WORKSPACES.items()):
        if index != device.index:
            continue
        count = ctypes.c_int64(0)
        hip.check(lib.vh_grn_workspace_fallbacks(hip.ptr(ws), ws.numel() * 4, ctypes.c_void_p(handle),
                                                 ctypes.byref(count)), "vh_grn_workspace_fallbacks")
        total += count.value
    return total


class _VisionHOPEGRNFunction(Function):
    @staticmethod
    @on_tensor_device
    def forward(ctx, x, gamma, beta, eps, out_dtype=torch.float32):
        batch, channels, height, width = x.shape
        if not x.is_contiguous(memory_format=torch.channels_last):
            x = x.contiguous(memory_format=torch.channels_last)
        gamma_shape, beta_shape = gamma.shape, beta.shape
        gamma = gamma.detach().reshape(-1).float().contiguous()
        beta = beta.detach().reshape(-1).float().contiguous()
        y = torch.empty_like(x, dtype=out_dtype, memory_format=torch.channels_last)
        gx = torch.empty((batch, channels), device=x.device, dtype=torch.float32)
        inv_den = torch.empty((batch,), device=x.device, dtype=torch.float32)
        lib = hip.load_library()
        ws = _stream_workspace(lib.vh_grn_workspace_bytes(batch, channels, height, width), x.device)
        hip.check(lib.vh_grn_forward(
            hip.ptr(x), hip.dtype_code(x.dtype), hip.ptr(gamma), hip.ptr(beta), hip.ptr(y),
            hip.dtype_code(out_dtype), hip.ptr(gx), hip.ptr(inv_den), batch, channels, height, width,
            float(eps),
            hip.ptr(ws), ws.numel() * 4, hip.stream_of(x)), "vh_grn_forward")
        ctx.save_for_backward(x, gamma, gx, inv_den)
        ctx.param_shapes = (gamma_shape, beta_shape)
        return y

    @staticmethod
    @on_tensor_device
    def backward(ctx, dout):
        """Reference ``utils/grn_cuda.py:51-82``: dx in x's dtype (channels-last), FP32
        dgamma and dbeta in the parameters' shapes."""
        x, gamma, gx, inv_den = ctx.saved_tensors
        batch, channels, height, width = x.shape
        g = dout.to(dtype=torch.float32, memory_format=torch.channels_last)
        dx = torch.empty_like(x, memory_format=torch.channels_last)
        dgamma = torch.empty(channels, device=x.device, dtype=torch.float32)
        dbeta = torch.empty(channels, device=x.device, dtype=torch.float32)
        lib = hip.load_library()
        ws = hip.workspace(lib.vh_grn_backward_workspace_bytes(batch, channels, height, width), x.device)
        hip.check(lib.vh_grn_backward(
            hip.ptr(g), hip.ptr(x), hip.dtype_code(x.dtype), hip.ptr(gamma), hip.ptr(gx), hip.ptr(inv_den),
            hip.ptr(dx), hip.ptr(dgamma), hip.ptr(dbeta), batch, channels, height, width, hip.ptr(ws),
            ws.numel() * 4, hip.stream_of(x)), "vh_grn_backward")
        gamma_shape, beta_shape = ctx.param_shapes
        return dx, dgamma.view(gamma_shape), dbeta.view(beta_shape), None, None


def can_fuse_grn(x, gamma, beta):
    """Reference eligibility test (``utils/grn_cuda.py:83-98``)."""
    if x.ndim != 4 or not x.is_cuda or not x.is_contiguous(memory_format=torch.channels_last):
        return False
    if x.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        return False
    channels = x.shape[1]
    spatial = x.shape[2] * x.shape[3]
    if x.shape[0] < 1 or x.shape[0] > 65535 or channels < 1 or spatial < 1:
        return False
    return (gamma.device == x.device and beta.device == x.device
            and gamma.dtype == torch.float32 and beta.dtype == torch.float32
            and gamma.is_contiguous() and beta.is_contiguous()
            and gamma.numel() == channels and beta.numel() == channels)


def visionhope_grn(x, gamma, beta, eps, out_dtype=torch.float32):
    """FP32 GRN output (the reference's contract); ``out_dtype`` stores the same values
    rounded to a 16-bit type when the consumer casts them anyway (autocast)."""
    if x.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise TypeError("GRN supports FP32, FP16 and BF16 input")
    if x.shape[0] < 1 or x.shape[0] > 65535:
        raise ValueError("GRN expects nonempty input and batch <= 65535")
    return _VisionHOPEGRNFunction.apply(x, gamma, beta, eps, out_dtype)


def grn_statistics_supported(channels, numel):
    """Whether ``grn_scale`` takes a map of ``channels`` channels and ``numel`` elements
    (the limits of ``vh_grn_scale_forward``: C % 8 == 0, C <= 2048, fewer than 2^31
    elements; channels-last and 16-byte aligned as torch allocates them)."""
    return channels % 8 == 0 and 0 < channels <= 2048 and numel < (1 << 31)


@on_tensor_device
def grn_scale(x, gamma, eps):
    """GRN statistics of the channels-last map ``x [B, C, H, W]``: the FP32 factor
    ``scale [B, C] = 1 + gamma * nx`` with ``GRN(x) = x * scale + beta``
    (``utils/grn.py:26-38``), for consumers that apply it while loading x."""
    batch, channels, height, width = x.shape
    if x.dtype not in (torch.float16, torch.bfloat16, torch.float32) or not 1 <= batch <= 65535:
        raise ValueError("GRN statistics expect FP32/FP16/BF16 input and 1 <= batch <= 65535")
    if not x.is_contiguous(memory_format=torch.channels_last) or x.data_ptr() % 16:
        raise ValueError("GRN statistics expect a 16-byte aligned channels-last map")
    gamma = gamma.detach().reshape(-1).float().contiguous()
    scale = torch.empty((batch, channels), device=x.device, dtype=torch.float32)
    gx = torch.empty((batch, channels), device=x.device, dtype=torch.float32)
    inv_den = torch.empty((batch,), device=x.device, dtype=torch.float32)
    lib = hip.load_library()
    ws = hip.workspace(lib.vh_grn_workspace_bytes(batch, channels, height, width), x.device)
    hip.check(lib.vh_grn_scale_forward(
        hip.ptr(x), hip.dtype_code(x.dtype), hip.ptr(gamma), hip.ptr(gx), hip.ptr(inv_den), hip.ptr(scale),
        batch, channels, height, width, float(eps), hip.ptr(ws), ws.numel() * 4, hip.stream_of(x)),
        "vh_grn_scale_forward")
    return scale
