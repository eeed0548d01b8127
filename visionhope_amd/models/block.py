"""The VisionHOPE block: its module tree (the checkpoint key format of the reference's
``models/block.py``), its reference-order forward, and the fused inference forward that
prepared models run on the GPU."""

import torch
from torch import nn
from torch.nn import functional as F
from torch.nn.init import trunc_normal_

from .droppath import DropPath
from .layers import FeedForwardNetwork, LayerNorm2d, build_norm
from .operator import VisionHOPEOperator
from .srnl_core.fused import srnl_spatial_readout, srnl_spatial_scan, srnl_spatial_workspace
from ..utils import dwconv, pointwise
from ..utils.cached_params import contiguous_fp32, linear_weights
from ..utils.grn import GlobalResponseNorm
from ..utils.grn_cuda import grn_scale, grn_statistics_supported, visionhope_grn
from ..utils.layer_norm_cuda import (can_fuse_add_layernorm2d, can_fuse_layernorm2d, visionhope_add_layernorm2d,
                                     visionhope_layernorm2d)
from ..utils.residual import can_fuse_residual_add, visionhope_residual_add


_SIDE_STREAMS = {}

# CPE and norm1 of the fused block path in one kernel where the map allows; False runs the
# two kernels (for measurements).  A module attribute, not an environment variable, so the
# path a forward takes does not depend on the caller's environment.
FUSE_CPE_LAYERNORM = True

# The spatial operator's scan on a side stream, overlapping the query projection and the
# position encoding (True), or all of them in order on the caller's stream (False, the
# default: in a HIP graph the fork and the join each left the GPU idle for 5-10 us, more
# than the overlap saved; Tiny forward 9.52 -> 9.42 ms measured on MI355X).
OVERLAP_SCAN = False

# proj_in and local_gate (gated local mixing) as one chained launch where the widths allow
# (True), or as two projections (False, for measurements); the same bits either way.
FUSE_GATE_CHAIN = True

# proj_out with the residual add and norm2 in its epilogue where the block width allows
# (True), or the projection followed by the add + LayerNorm kernel (False, for
# measurements); the same bits either way.
FUSE_OUT_NORM = True

# The local position encoding (5x5 depthwise of x_local) computed inside the operator's
# readout (True: one pass, the same bits) or as a separate depthwise pass whose result the
# readout adds (False, for measurements).
FUSE_LEPE_READOUT = True


def _side_stream(device):
    """One default-priority side stream per device for work overlapped with the scan."""
    stream = _SIDE_STREAMS.get(device.index)
    if stream is None:
        stream = _SIDE_STREAMS[device.index] = torch.cuda.Stream(device=device)
    return stream


def _is_pointwise(conv):
    return (isinstance(conv, nn.Conv2d) and conv.kernel_size == (1, 1) and conv.stride == (1, 1)
            and conv.padding == (0, 0) and conv.groups == 1)


# Short (few-pixel) products with K x N at or above this go to the library GEMM: on the
# Tiny stage-4 fc1 (6272 pixels, 512 -> 2048 channels) its tiles keep the matrix cores
# busier than the native kernel's, more than the fused epilogue saves (measured on
# MI355X, whole forward).  Every other projection takes the native kernel, and so does an
# fc2 that takes the GRN on its operand (the library path needs a separate GRN pass:
# Tiny forward 9.57 -> 9.50 ms with the stage-4 fc2 native).
_LIBRARY_MIN_KN = 1 << 20
_LIBRARY_MAX_PIXELS = 16384


def _matrix_core_ok(t_nhwc, module, grn_prologue=False):
    """Whether the bf16 matrix-core 1x1 kernel takes ``module`` on the NHWC view ``t``
    (otherwise the library GEMM runs on the autocast-cast operands); ``grn_prologue``: the
    product would take the GRN on its operand."""
    weight = module.weight
    n, k = weight.shape[0], weight.shape[1]
    pixels = t_nhwc.numel() // max(t_nhwc.shape[-1], 1)
    return (t_nhwc.is_contiguous() and t_nhwc.data_ptr() % 16 == 0 and module.bias is not None
            and pointwise.supported(k, n) and t_nhwc.shape[-1] == k
            and (grn_prologue or _native_size(pixels, k, n)))


def _native_size(pixels, k, n):
    """The size rule of ``_matrix_core_ok``: the library GEMM keeps deep, short products."""
    return pixels >= _LIBRARY_MAX_PIXELS or k * n < _LIBRARY_MIN_KN


def _grn_beta(grn):
    """GRN beta as a contiguous FP32 ``[C]`` vector (cached while unchanged)."""
    return contiguous_fp32(grn.beta.detach().reshape(-1))


def _is_exact_gelu(act):
    return type(act) is nn.GELU and act.approximate == "none"


# Depthwise kernel of the local mixing for each local_mode.
_LOCAL_KERNELS = {"gated_dwconv7": 7, "residual_dwconv": 3, "silu_dwconv": 3}


def _depthwise(channels, kernel):
    return nn.Conv2d(channels, channels, kernel, padding=kernel // 2, groups=channels)


class VisionHOPEBlock(nn.Module):
    """Pre-norm VisionHOPE block on NCHW maps (reference ``models/block.py:13-107``):

        x = x + cpe(x)                                   (optional 3x3 depthwise)
        x = x + drop_path(gamma1 * spatial(norm1(x)))
        x = x + drop_path(gamma2 * ffn(norm2(x)))

    where ``spatial(h) = proj_out(operator(l) + lepe(l))`` with ``l`` the local mixing of
    ``proj_in(h)`` (``local_mode``) and ``lepe`` an optional 5x5 depthwise position
    encoding.  The operator runs on ``mixer_dim`` channels (default ``dim``).
    """

    def __init__(self, dim, head_dim=16, chunk_size=None, mlp_ratio=4.0,
                 drop_path=0.0, mixer_dim=None, local_mode="gated_dwconv7",
                 norm_layer="layernorm2d", layer_scale_init_value=1e-6,
                 use_grn=True, use_mlp_dwconv=True, use_direction_scale=True,
                 direction_merge="sum", use_block_cpe=True, use_output_lepe=True,
                 share_direction_skip=True):
        super().__init__()
        if local_mode not in _LOCAL_KERNELS:
            raise ValueError("Unsupported local_mode")
        mixer_dim = dim if mixer_dim is None else int(mixer_dim)
        self.dim, self.mixer_dim, self.local_mode = dim, mixer_dim, local_mode
        self._inference_prepared = False
        self.cpe = _depthwise(dim, 3) if use_block_cpe else None
        self.norm1 = build_norm(dim, norm_layer)

        # spatial branch; a learned per-direction scale replaces the plain sum
        self.proj_in = nn.Conv2d(dim, mixer_dim, 1)
        merge = "scale" if use_direction_scale and direction_merge == "sum" else direction_merge
        self.operator = VisionHOPEOperator(mixer_dim, head_dim, chunk_size, merge, share_direction_skip,
                                           _initialize=False)
        self.local_conv = _depthwise(mixer_dim, _LOCAL_KERNELS[local_mode])
        self.local_gate = nn.Conv2d(mixer_dim, mixer_dim, 1) if local_mode == "gated_dwconv7" else None
        self.local_act = nn.SiLU() if local_mode == "silu_dwconv" else nn.Identity()
        self.local_position = _depthwise(mixer_dim, 5) if use_output_lepe else None
        self.proj_out = nn.Linear(mixer_dim, dim)
        self.operator.reset_parameters()
        trunc_normal_(self.proj_out.weight, std=0.02)
        nn.init.zeros_(self.proj_out.bias)

        # feed-forward branch
        self.drop_path = DropPath(drop_path) if drop_path > 0.0 else nn.Identity()
        self.norm2 = build_norm(dim, norm_layer)
        self.ffn = FeedForwardNetwork(dim, int(dim * mlp_ratio), use_grn=use_grn, use_dwconv=use_mlp_dwconv)
        scaled = layer_scale_init_value is not None and layer_scale_init_value > 0.0
        for name in ("gamma1", "gamma2"):
            value = nn.Parameter(torch.full((dim, 1, 1), float(layer_scale_init_value))) if scaled else None
            setattr(self, name, value)

    def _fused_eligible(self, x):
        """Whether ``forward`` may take the fused inference path for ``x``.

        The fused path computes the same block as ``forward`` (same modules, same
        rounding points under autocast) with the depthwise convolutions and their
        surrounding elementwise work in single native passes, the 1x1 projections as
        channels-last GEMMs, LayerNorm/GRN writing the dtype their consumer reads, and
        the local position encoding accumulated into the operator's FP32 output.
        """
        if not self._inference_prepared or self.training or not x.is_cuda or x.ndim != 4:
            return False
        if not x.is_contiguous(memory_format=torch.channels_last) or x.data_ptr() % 16:
            return False
        autocast = torch.is_autocast_enabled("cuda")
        if autocast:
            if torch.get_autocast_dtype("cuda") not in (torch.bfloat16, torch.float16):
                return False
        elif x.dtype != torch.float32 or any(p.dtype != torch.float32 for p in self.parameters()):
            return False
        ffn = self.ffn
        if type(ffn) is not FeedForwardNetwork or not _is_exact_gelu(ffn.act):
            return False
        if ffn.use_dwconv and not (dwconv.is_depthwise(ffn.dwconv) and _is_exact_gelu(ffn.dwconv_act)):
            return False
        if not isinstance(ffn.grn, (GlobalResponseNorm, nn.Identity)):
            return False
        if not all(_is_pointwise(c) for c in (self.proj_in, ffn.fc1, ffn.fc2)):
            return False
        if self.local_gate is not None and not _is_pointwise(self.local_gate):
            return False
        for conv in (self.cpe, self.local_conv, self.local_position):
            if conv is not None and not dwconv.is_depthwise(conv):
                return False
        for norm in (self.norm1, self.norm2):
            if type(norm) is not LayerNorm2d:
                return False
        return (can_fuse_layernorm2d(x, self.norm1.weight, self.norm1.bias)
                and self.dim % 8 == 0 and self.mixer_dim % 8 == 0 and ffn.fc1.out_channels % 8 == 0)

    def _fused_forward(self, x):
        """Inference forward of the block on a channels-last map (``_fused_eligible``)."""
        autocast = torch.is_autocast_enabled("cuda")
        act = torch.get_autocast_dtype("cuda") if autocast else torch.float32

        def project(t_nhwc, module, epilogue=pointwise.EPI_BIAS):
            # bf16: the matrix-core kernel with the epilogue fused; otherwise the
            # library GEMM on the autocast-cast operands and the epilogue after it.
            if act == torch.bfloat16 and _matrix_core_ok(t_nhwc, module):
                return pointwise.pointwise_conv(t_nhwc, module, epilogue)
            weight, bias = linear_weights(module, act)
            y = F.linear(t_nhwc.to(act), weight, bias)
            return F.gelu(y) if epilogue == pointwise.EPI_GELU else y

        def nchw(t_nhwc):
            return t_nhwc.permute(0, 3, 1, 2)

        # CPE and norm1: one pass (the sum and its LayerNorm) where the map allows
        # (FUSE_CPE_LAYERNORM = False runs the two kernels, for measurements).
        h = None
        if self.cpe is not None:
            fused = (dwconv.depthwise_conv_add_layernorm(x, self.cpe, self.norm1.weight, self.norm1.bias,
                                                         self.norm1.eps)
                     if x.dtype == act and FUSE_CPE_LAYERNORM else None)
            if fused is not None:
                x, h = fused
            else:
                x = dwconv.depthwise_conv(x, self.cpe, dwconv.EPI_ADD_INPUT)
        # Token-mixer branch.
        if h is None:
            h = visionhope_layernorm2d(x, self.norm1.weight, self.norm1.bias, self.norm1.eps,
                                       force_channels_last=True, out_dtype=act)
        h_nhwc = h.permute(0, 2, 3, 1)
        gate = None
        if (self.local_mode == "gated_dwconv7" and FUSE_GATE_CHAIN and act == torch.bfloat16
                and pointwise.chain_supported(self.proj_in, self.local_gate) and _matrix_core_ok(h_nhwc, self.proj_in)
                and _native_size(h_nhwc.numel() // h_nhwc.shape[-1], self.local_gate.weight.shape[1],
                                 self.local_gate.weight.shape[0])):
            # proj_in and local_gate in one launch (the same bits as the two projections)
            inner, gate = pointwise.pointwise_chain(h_nhwc, self.proj_in, self.local_gate)
        else:
            inner = project(h_nhwc, self.proj_in)
        if self.local_mode == "gated_dwconv7":
            if gate is None:
                gate = project(inner, self.local_gate)
            x_local = dwconv.depthwise_conv(nchw(inner), self.local_conv, dwconv.EPI_GATE, aux=nchw(gate))
        elif self.local_mode == "residual_dwconv":
            x_local = dwconv.depthwise_conv(nchw(inner), self.local_conv, dwconv.EPI_ADD_INPUT)
        else:
            x_local = F.silu(dwconv.depthwise_conv(nchw(inner), self.local_conv))
        path, _ = self.operator._inference_path(x_local)
        x_h = None   # (x + branch, norm2 of it) when proj_out's launch produced them
        if path == "ordinary":
            branch = self._spatial_tail(x_local, True)
        elif path == "spatial" and x_local.dtype == act:
            op_out = self._spatial_overlapped(x_local)
            x_nhwc = x.permute(0, 2, 3, 1)
            if (FUSE_OUT_NORM and self.gamma1 is None and act == torch.bfloat16
                    and pointwise.add_layernorm_supported(self.proj_out) and _matrix_core_ok(op_out, self.proj_out)
                    and x.dtype == act and x_nhwc.is_contiguous() and x_nhwc.data_ptr() % 16 == 0
                    and isinstance(self.norm2, LayerNorm2d)):
                # proj_out, the residual add and norm2 in one launch (the same bits)
                s_nhwc, h_nhwc = pointwise.pointwise_add_layernorm(op_out, self.proj_out, x_nhwc, self.norm2.weight,
                                                                   self.norm2.bias, self.norm2.eps)
                x_h = (nchw(s_nhwc), nchw(h_nhwc))
                branch = None
            else:
                branch = nchw(project(op_out, self.proj_out))
        else:
            out = self.operator._forward_fast(x_local, path)
            if self.local_position is not None:
                # The position encoding is added to the FP32 operator output and the sum is
                # rounded once to the compute dtype, the input dtype of proj_out.
                out = dwconv.depthwise_conv(x_local, self.local_position, dwconv.EPI_ADD_F32_AUX,
                                            aux=out).permute(0, 2, 3, 1)
            branch = nchw(project(out, self.proj_out))
        # Feed-forward branch (the residual add fused into norm2 when LayerScale is folded).
        ffn = self.ffn
        if x_h is not None:
            x, h = x_h
        elif self.gamma1 is None and can_fuse_add_layernorm2d(x, branch, self.norm2.weight, self.norm2.bias):
            x, h = visionhope_add_layernorm2d(x, branch, self.norm2.weight, self.norm2.bias, self.norm2.eps,
                                              out_dtype=act)
        else:
            x = self._residual_add(x, branch, self.gamma1)
            h = visionhope_layernorm2d(x, self.norm2.weight, self.norm2.bias, self.norm2.eps,
                                       force_channels_last=True, out_dtype=act)
        f = project(h.permute(0, 2, 3, 1), ffn.fc1, pointwise.EPI_GELU)
        use_grn = isinstance(ffn.grn, GlobalResponseNorm)
        x_nhwc = x.permute(0, 2, 3, 1)
        # the GRN statistics of fc2's operand must be computable natively for the fused fc2
        grn_stats_ok = not use_grn or grn_statistics_supported(f.shape[-1], f.numel())
        fc2_fused = (act == torch.bfloat16 and self.gamma2 is None and x.dtype == act and x_nhwc.is_contiguous()
                     and grn_stats_ok and _matrix_core_ok(f, ffn.fc2, grn_prologue=use_grn))
        scale = None
        if ffn.use_dwconv:
            fused = None
            if fc2_fused and use_grn:
                # GRN statistics taken in the depthwise pass that produces GRN's input.
                fused = dwconv.depthwise_conv_gelu_grn(nchw(f), ffn.dwconv, ffn.grn.gamma, ffn.grn.eps)
            if fused is not None:
                f, scale = fused[0].permute(0, 2, 3, 1), fused[1]
            else:
                f = dwconv.depthwise_conv(nchw(f), ffn.dwconv, dwconv.EPI_ADD_GELU).permute(0, 2, 3, 1)
        if fc2_fused:
            # GRN applied to fc2's operand as it is loaded, residual add in fc2's epilogue.
            grn = None
            if use_grn:
                if scale is None:
                    scale = grn_scale(nchw(f), ffn.grn.gamma, ffn.grn.eps)
                grn = (scale, _grn_beta(ffn.grn))
            out = pointwise.pointwise_conv(f, ffn.fc2, pointwise.EPI_ADD, residual=x_nhwc, grn=grn)
            return nchw(out)
        if use_grn:
            f = visionhope_grn(nchw(f), ffn.grn.gamma, ffn.grn.beta, ffn.grn.eps,
                               out_dtype=act).permute(0, 2, 3, 1)
        branch = nchw(project(f, ffn.fc2))
        return self._residual_add(x, branch, self.gamma2)

    def _spatial_overlapped(self, x_local):
        """Operator output plus local position encoding, ``[B, H, W, C]`` in x_local's dtype.

        The scan, then the query projection; the readout fuses the four directions,
        computes and adds the position encoding (``FUSE_LEPE_READOUT``; otherwise a separate
        depthwise pass ahead of it) and rounds once (``operator.py:159-193`` +
        ``block.py:77-78``).  With ``OVERLAP_SCAN`` the scan runs on a side stream
        instead, overlapping the other two; every tensor that both streams touch (the
        scan's workspace) is allocated on the caller's stream before the fork.
        """
        op = self.operator
        dev = x_local.device
        memories = op.srnl._validate_memories(dev)
        skip_shape = (op.num_heads, op.head_dim) if op.share_direction_skip else (4, op.num_heads, op.head_dim)
        if op.d_skip.shape != skip_shape or op.d_skip.device != dev:
            raise ValueError("Directional skip has an invalid shape or device")
        weights = op._merge_weights()
        batch, channels, height, width = x_local.shape
        chunks = (width, width, height, height)
        x_nhwc = x_local.permute(0, 2, 3, 1)
        ws = srnl_spatial_workspace(x_nhwc, op.head_dim, chunks)
        main = torch.cuda.current_stream(dev)
        op.announce_query_projection(x_nhwc)
        if OVERLAP_SCAN:
            side = _side_stream(dev)
            side.wait_stream(main)
            with torch.cuda.stream(side):
                srnl_spatial_scan(memories, x_nhwc, chunks, workspace=ws)
        else:
            srnl_spatial_scan(memories, x_nhwc, chunks, workspace=ws)
        with torch.autocast("cuda", enabled=False):
            # Operands already in the compute dtype: the product autocast would run.
            if x_local.dtype == torch.bfloat16 and _matrix_core_ok(x_nhwc, op.W_q):
                q = pointwise.pointwise_conv(x_nhwc, op.W_q)
            else:
                weight, bias = linear_weights(op.W_q, x_local.dtype)
                q = torch.addmm(bias, x_nhwc.reshape(-1, channels), weight.t()).view(x_nhwc.shape)
            lepe = fused_lepe = None
            if self.local_position is not None:
                if FUSE_LEPE_READOUT and self.local_position.kernel_size == (5, 5) and dwconv.is_depthwise(
                        self.local_position):
                    fused_lepe = dwconv.depthwise_taps(self.local_position)
                else:
                    lepe = dwconv.depthwise_conv(x_local, self.local_position, dwconv.EPI_PLAIN)
        if OVERLAP_SCAN:
            main.wait_stream(side)
        return srnl_spatial_readout(ws, x_nhwc, q, op.d_skip, weights, chunks, op.head_dim,
                                    aux=None if lepe is None else lepe.permute(0, 2, 3, 1),
                                    out_dtype=x_local.dtype, lepe=fused_lepe)

    def _local_features(self, x):
        """``proj_in`` followed by the local mixing of ``local_mode``."""
        inner = self.proj_in(x)
        conv = self.local_conv(inner)
        if self.local_mode == "gated_dwconv7":
            return inner + torch.sigmoid(self.local_gate(inner)) * conv
        conv = self.local_act(conv)
        return conv if self.local_mode == "silu_dwconv" else inner + conv

    def spatial_branch(self, x):
        channels_last = x.is_contiguous(memory_format=torch.channels_last)
        return self._spatial_tail(self._local_features(x), channels_last)

    def _spatial_tail(self, x_local, channels_last):
        if self._inference_prepared:
            path, _ = self.operator._inference_path(x_local)
            if path != "ordinary":
                out = self.operator._forward_fast(x_local, path)
                if self.local_position is not None:
                    out = out + self.local_position(x_local).permute(0, 2, 3, 1)
                out = self.proj_out(out)
                # NHWC storage is already channels-last; NCHW callers get a dense copy.
                out = out.permute(0, 3, 1, 2)
                return out if channels_last else out.contiguous()

        out = self.operator(x_local, channels_last=channels_last)
        if self.local_position is not None:
            out = out + self.local_position(x_local)
        out = F.conv2d(out, self.proj_out.weight[:, :, None, None], self.proj_out.bias)
        if channels_last:
            return out.contiguous(memory_format=torch.channels_last)
        return out.contiguous()

    def _residual_add(self, x, branch, gamma):
        if gamma is None:
            return x + self.drop_path(branch)
        if can_fuse_residual_add(x, branch, gamma):
            return visionhope_residual_add(x, branch, gamma,
                                           getattr(self.drop_path, "drop_prob", 0.0), self.training,
                                           getattr(self.drop_path, "scale_by_keep", True))
        return x + self.drop_path(gamma * branch)

    def forward(self, x):
        if self.training and self._inference_prepared:
            raise RuntimeError("A block with folded LayerScale weights cannot be trained")
        if self._fused_eligible(x):
            return self._fused_forward(x)
        if self.cpe is not None:
            x = x + self.cpe(x)
        x = self._residual_add(x, self.spatial_branch(self.norm1(x)), self.gamma1)
        return self._residual_add(x, self.ffn(self.norm2(x)), self.gamma2)
