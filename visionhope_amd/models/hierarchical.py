"""The four-stage hierarchical VisionHOPE backbone and classifier.

Architecture and module names of the reference's ``models/hierarchical.py:11-85`` (the
module tree is the checkpoint key format): a patch-embedding stem, three 2x downsamples,
four stages of ``VisionHOPEBlock``, and a projection head (norm, 1x1 conv, BatchNorm,
SiLU, average pool, linear).  ``_fused_head`` is this build's prepared-inference head.
"""

import torch
from torch import nn

from .block import VisionHOPEBlock
from .common import ClassificationModel, initialize_weights
from .layers import Downsample, LayerNorm2d, PatchEmbedding, build_norm


def _four(values):
    values = list(values)
    if len(values) != 4:
        raise ValueError("Hierarchical VisionHOPE requires four stage configurations")
    return values


class HierarchicalVisionHOPE(ClassificationModel):
    """VisionHOPE backbone with a projection classifier head.

    Stage i runs ``depths[i]`` blocks of width ``embed_dims[i]`` whose operator mixes
    ``mixer_dims[i]`` channels in heads of ``head_dim``.  ``chunk_sizes=None`` scans in
    chunks of the row and column lengths of whatever map arrives (rectangular maps
    included); four explicit values fix each stage's chunk length.  Stochastic depth
    rises linearly from 0 to ``drop_path_rate`` over all blocks.
    """

    def __init__(self, in_chans=3, num_classes=1000, embed_dims=(64, 128, 256, 512),
                 mixer_dims=(32, 64, 128, 256), depths=(3, 4, 18, 4), chunk_sizes=None,
                 mlp_ratios=(4.0, 4.0, 4.0, 4.0), head_dim=16, img_size=None,
                 drop_path_rate=0.1, local_mode="gated_dwconv7", norm_layer="layernorm2d",
                 layer_scale_init_value=1e-6, use_grn=True, use_mlp_dwconv=True,
                 use_direction_scale=True, direction_merge="sum", use_block_cpe=True,
                 use_output_lepe=True, projection_dim=1024, share_direction_skip=True):
        super().__init__()
        if isinstance(mlp_ratios, (int, float)):
            mlp_ratios = (float(mlp_ratios),) * 4
        self.num_classes = num_classes
        self.embed_dims = _four(embed_dims)
        self.mixer_dims = _four(embed_dims if mixer_dims is None else mixer_dims)
        self.depths = _four(depths)
        self.chunk_sizes = _four((None,) * 4 if chunk_sizes is None else chunk_sizes)
        mlp_ratios = _four(mlp_ratios)
        if min(self.depths) < 1 or min(self.embed_dims) < 1:
            raise ValueError("Stage depths and widths must be positive")
        self.head_dim = int(head_dim)
        self.img_size = img_size
        self.share_direction_skip = share_direction_skip

        widths = self.embed_dims
        self.downsample_layers = nn.ModuleList(
            [PatchEmbedding(in_chans, widths[0])] + [Downsample(widths[i - 1], widths[i]) for i in range(1, 4)])
        drop_rates = torch.linspace(0, drop_path_rate, sum(self.depths)).tolist()
        block_options = dict(head_dim=head_dim, local_mode=local_mode, norm_layer=norm_layer,
                             layer_scale_init_value=layer_scale_init_value, use_grn=use_grn,
                             use_mlp_dwconv=use_mlp_dwconv, use_direction_scale=use_direction_scale,
                             direction_merge=direction_merge, use_block_cpe=use_block_cpe,
                             use_output_lepe=use_output_lepe, share_direction_skip=share_direction_skip)
        self.stages = nn.ModuleList()
        first = 0
        for width, mixer, depth, chunk, ratio in zip(widths, self.mixer_dims, self.depths, self.chunk_sizes,
                                                     mlp_ratios):
            self.stages.append(nn.Sequential(*(
                VisionHOPEBlock(dim=width, chunk_size=chunk, mlp_ratio=ratio, drop_path=drop_rates[first + j],
                                mixer_dim=mixer, **block_options)
                for j in range(depth))))
            first += depth
        self.norm = build_norm(widths[-1], norm_layer)
        self.head_pre_logits = nn.Conv2d(widths[-1], projection_dim, 1)
        self.head_norm = nn.BatchNorm2d(projection_dim)
        self.head_act = nn.SiLU()
        self.num_features = int(projection_dim)
        self.head = nn.Linear(self.num_features, num_classes)
        self.grad_checkpointing = False
        self.apply(initialize_weights)

    def _stage_outputs(self, x):
        for downsample, stage in zip(self.downsample_layers, self.stages):
            x = self._run_blocks(stage, downsample(x))
            yield x

    def forward_intermediates(self, x):
        """The four stage feature maps (inputs of detection and segmentation heads)."""
        return tuple(self._stage_outputs(x))

    def forward_features(self, x):
        """Pooled pre-logits ``[B, projection_dim]``."""
        for x in self._stage_outputs(x):
            pass
        if self._fused_head_ok(x):
            return self._fused_head(x)
        h = self.head_act(self.head_norm(self.head_pre_logits(self.norm(x))))
        return h.mean(dim=(2, 3))

    def _fused_head_ok(self, x):
        """Prepared for inference, eval mode, bf16 autocast on a channels-last CUDA map,
        LayerNorm2d norm, a foldable head BatchNorm, and SiLU."""
        if (not getattr(self, "_vh_fold_head", False) or self.training or not x.is_cuda
                or not torch.is_autocast_enabled("cuda") or torch.get_autocast_dtype("cuda") != torch.bfloat16
                or not isinstance(self.norm, LayerNorm2d) or type(self.head_act) is not nn.SiLU):
            return False
        from ..utils import pointwise
        from ..utils.conv_bn import foldable
        from ..utils.layer_norm_cuda import can_fuse_layernorm2d
        conv = self.head_pre_logits
        return (x.is_contiguous(memory_format=torch.channels_last)
                and can_fuse_layernorm2d(x, self.norm.weight, self.norm.bias)
                and pointwise.is_pointwise(conv) and foldable(conv, self.head_norm)
                and pointwise.supported(conv.in_channels, conv.out_channels))

    def _fused_head(self, x):
        """``mean(silu(head_norm(head_pre_logits(norm(x)))))`` in two native passes: the
        LayerNorm stored as bf16 (the value autocast feeds the 1x1 conv), then the 1x1 conv
        with the eval BatchNorm folded into it and the SiLU in the GEMM epilogue, each
        rounded to bf16 as the autocast reference rounds them (reference
        ``models/hierarchical.py:78-85``)."""
        from ..utils import pointwise
        from ..utils.conv_bn import folded_weights
        from ..utils.layer_norm_cuda import visionhope_layernorm2d

        h = visionhope_layernorm2d(x, self.norm.weight, self.norm.bias, self.norm.eps,
                                   force_channels_last=True, out_dtype=torch.bfloat16)
        conv = self.head_pre_logits
        weight, bias = folded_weights(conv, self.head_norm)
        cached = getattr(conv, "_vh_head_gemm", None)
        if cached is None or cached[0] is not weight:
            object.__setattr__(conv, "_vh_head_gemm", (weight, weight.reshape(weight.shape[0], -1)
                                                       .to(torch.bfloat16).contiguous()))
            cached = conv._vh_head_gemm
        y = pointwise.pointwise_gemm(h.permute(0, 2, 3, 1), cached[1], bias, pointwise.EPI_SILU)
        return y.permute(0, 3, 1, 2).mean(dim=[2, 3])
