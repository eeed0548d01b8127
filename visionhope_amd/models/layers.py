"""Layers of the VisionHOPE backbone around the blocks: channel LayerNorm, the MLP, the
convolutional stem and the stage downsample (reference ``models/layers.py``)."""

import torch
from torch import nn
from torch.nn import functional as F

from ..utils.grn import GlobalResponseNorm
from ..utils.layer_norm_cuda import can_fuse_layernorm2d, visionhope_layernorm2d


def _layer_norm_result_dtype(x):
    """dtype F.layer_norm would return: FP32 under CUDA autocast or for FP32 input."""
    if x.dtype == torch.float32 or (x.is_cuda and torch.is_autocast_enabled("cuda")):
        return torch.float32
    return x.dtype


class LayerNorm2d(nn.Module):
    """LayerNorm over channels of an NCHW map (``models/layers.py:9-35``).

    GPU tensors run the native kernel.  In ``inference_layout`` mode the result
    is channels-last storage with ``F.layer_norm``'s dtype (``layers.py:18-20``);
    otherwise FP32 in the input's storage order, as the fused reference kernel.
    """

    def __init__(self, dim, eps=1e-6):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(dim))
        self.bias = nn.Parameter(torch.zeros(dim))
        self.eps = eps
        self.inference_layout = False

    def forward(self, x):
        if x.is_cuda and can_fuse_layernorm2d(x, self.weight, self.bias):
            if self.inference_layout:
                y = visionhope_layernorm2d(x, self.weight, self.bias, self.eps, force_channels_last=True)
                dtype = _layer_norm_result_dtype(x)
                return y if dtype == torch.float32 else y.to(dtype)
            channels_last = x.is_contiguous(memory_format=torch.channels_last)
            y = visionhope_layernorm2d(x, self.weight, self.bias, self.eps)
            if channels_last:
                return y
            dtype = _layer_norm_result_dtype(x)
            return y if dtype == torch.float32 else y.to(dtype)
        if x.is_cuda:
            raise ValueError(f"LayerNorm2d: unsupported input {tuple(x.shape)} {x.dtype} on {x.device}")
        # CPU tensors: the reference formula (layers.py:25-35).
        channels_last = x.is_contiguous(memory_format=torch.channels_last)
        y = F.layer_norm(x.permute(0, 2, 3, 1), (x.shape[1],), self.weight, self.bias, self.eps)
        y = y.permute(0, 3, 1, 2)
        if self.inference_layout:
            return y
        return y.contiguous(memory_format=torch.channels_last) if channels_last else y.contiguous()


def build_norm(dim, norm_layer="group"):
    if norm_layer == "group":
        return nn.GroupNorm(1, dim)
    if norm_layer == "layernorm2d":
        return LayerNorm2d(dim)
    raise ValueError(f"Unsupported norm_layer={norm_layer!r}.")


class FeedForwardNetwork(nn.Module):
    """Pointwise MLP on NCHW maps (reference ``models/layers.py:38-82``):

        h = act(fc1(x));  h = act(h + dwconv3x3(h)) if use_dwconv;  h = grn(h) if use_grn
        y = fc2(dropout(h)), then dropout

    with 1x1 convolutions for fc1 / fc2 and a depthwise 3x3 ``dwconv``.
    """

    def __init__(self, in_features, hidden_features=None, out_features=None, act_layer=nn.GELU,
                 drop=0.0, use_grn=False, use_dwconv=False):
        super().__init__()
        hidden = hidden_features or in_features
        self.fc1 = nn.Conv2d(in_features, hidden, kernel_size=1)
        self.act = act_layer()
        self.use_dwconv = use_dwconv
        if use_dwconv:
            self.dwconv = nn.Conv2d(hidden, hidden, kernel_size=3, padding=1, groups=hidden)
            self.dwconv_act = act_layer()
        else:
            self.dwconv = nn.Identity()
            self.dwconv_act = nn.Identity()
        self.grn = GlobalResponseNorm(hidden) if use_grn else nn.Identity()
        self.fc2 = nn.Conv2d(hidden, out_features or in_features, kernel_size=1)
        self.drop = nn.Dropout(drop)

    def forward(self, x):
        h = self.act(self.fc1(x))
        if self.use_dwconv:
            h = self.dwconv_act(h + self.dwconv(h))
        return self.drop(self.fc2(self.drop(self.grn(h))))


# Stem stages: (fraction of embed_dim as width divisor, stride, GELU after the BatchNorm).
_STEM = ((2, 2, True), (2, 1, True), (1, 2, True), (1, 1, False))


class PatchEmbedding(nn.Module):
    """Stride-4 convolutional stem (reference ``models/layers.py:85-107``): four 3x3
    convolutions of widths embed_dim/2, embed_dim/2, embed_dim, embed_dim and strides 2,
    1, 2, 1, each followed by BatchNorm and, except the last, GELU (``proj``, a
    Sequential whose indices are the checkpoint keys)."""

    def __init__(self, in_chans, embed_dim, patch_size=4):
        super().__init__()
        if patch_size != 4:
            raise ValueError("The VisionHOPE stem requires patch_size=4")
        if embed_dim // 2 <= 0:
            raise ValueError("embed_dim is too small for the convolutional stem")
        modules, channels = [], in_chans
        for divisor, stride, gelu in _STEM:
            width = embed_dim // divisor
            modules += [nn.Conv2d(channels, width, 3, stride=stride, padding=1), nn.BatchNorm2d(width)]
            if gelu:
                modules.append(nn.GELU())
            channels = width
        self.proj = nn.Sequential(*modules)
        self.norm = nn.Identity()

    def forward(self, x):
        if self._folded_path(x):
            from ..utils.conv_bn import ACT_GELU, ACT_NONE, conv_bn_act, conv_bn_act_padded, padded_native_ok
            mods = list(self.proj)
            i = 0
            while i < len(mods):
                gelu = i + 2 < len(mods) and isinstance(mods[i + 2], nn.GELU)
                act = ACT_GELU if gelu else ACT_NONE
                conv = mods[i]
                last = i + (3 if gelu else 2) >= len(mods)
                # Widths off the implicit GEMM's multiples of 32 (Base: 48): zero-padded
                # channels inside the stem; the stem's output keeps its real width.
                narrow = conv.out_channels % 32 != 0 or x.shape[1] != conv.in_channels
                if narrow and padded_native_ok(x, conv) and (not last or conv.out_channels % 32 == 0):
                    x = conv_bn_act_padded(x, conv, mods[i + 1], act, pad_out=not last)
                else:
                    if x.shape[1] != conv.in_channels:   # drop the zero padding for the library path
                        x = x[:, :conv.in_channels].contiguous(memory_format=torch.channels_last)
                    x = conv_bn_act(x, conv, mods[i + 1], act)
                i += 3 if gelu else 2
            return self.norm(x)
        return self.norm(self.proj(x))

    def _folded_path(self, x):
        """Prepared for inference, eval mode, channels-last CUDA input, and every stage a
        foldable (Conv2d, BatchNorm2d[, exact GELU]) group."""
        if not getattr(self, "_vh_fold_bn", False) or self.training or not x.is_cuda:
            return False
        if not x.is_contiguous(memory_format=torch.channels_last):
            return False
        from ..utils.conv_bn import foldable
        mods = list(self.proj)
        i = 0
        while i < len(mods):
            if i + 1 >= len(mods) or not foldable(mods[i], mods[i + 1]):
                return False
            nxt = mods[i + 2] if i + 2 < len(mods) else None
            if isinstance(nxt, nn.GELU):
                if nxt.approximate != "none":
                    return False
                i += 3
            else:
                i += 2
        return True


class Downsample(nn.Module):
    """Stage transition (reference ``models/layers.py:110-119``): a 3x3, stride-2 convolution
    without bias, then BatchNorm."""

    def __init__(self, in_dim, out_dim):
        super().__init__()
        self.proj = nn.Conv2d(in_dim, out_dim, 3, stride=2, padding=1, bias=False)
        self.norm = nn.BatchNorm2d(out_dim)

    def forward(self, x):
        if (getattr(self, "_vh_fold_bn", False) and not self.training and x.is_cuda
                and x.is_contiguous(memory_format=torch.channels_last)):
            from ..utils.conv_bn import conv_bn_act, foldable
            if foldable(self.proj, self.norm):
                return conv_bn_act(x, self.proj, self.norm)
        return self.norm(self.proj(x))
