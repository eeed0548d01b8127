"""Enable the MI355X inference path for SRNL components and VisionHOPE models
(mirrors ``inference/prepare.py``)."""

import torch

from ..models.block import VisionHOPEBlock
from ..models.layers import Downsample, LayerNorm2d, PatchEmbedding
from ..models.operator import VisionHOPEOperator
from ..models.srnl import SRNL
from ..utils.grn import GlobalResponseNorm


def prepare_for_inference(model):
    """Set evaluation mode and enable fast inference (``inference/prepare.py:12-54``).

    Blocks fold LayerScale into projection weights in place; use an eval-only copy.
    Returns preparation counts by component; ``line_mixer`` counts prepared blocks.
    """
    blocks = [module for module in model.modules() if isinstance(module, VisionHOPEBlock)]
    for block in blocks:
        if type(block.operator) is not VisionHOPEOperator or type(block.operator.srnl) is not SRNL:
            raise ValueError("Production fusion requires the unmodified VisionHOPE operator and SRNL")
    model.eval()
    counts = dict(line_mixer=0, srnl=0, operator=0, layernorm2d=0, grn=0, layerscale=0)
    for module in model.modules():
        if isinstance(module, SRNL):
            module.fast_inference = True
            counts["srnl"] += 1
        elif isinstance(module, VisionHOPEOperator):
            counts["operator"] += 1
        elif isinstance(module, LayerNorm2d):
            module.inference_layout = True
            counts["layernorm2d"] += 1
        elif isinstance(module, GlobalResponseNorm):
            counts["grn"] += 1
        elif isinstance(module, (PatchEmbedding, Downsample)):
            # Eval-mode BatchNorm folded into the convolution on the GPU path (no
            # parameter changes: the folded copy is cached beside the module).
            module._vh_fold_bn = True
        if hasattr(module, "head_pre_logits") and hasattr(module, "head_norm"):
            # The classifier head's BatchNorm likewise, with the LayerNorm and SiLU fused
            # around the 1x1 projection.
            module._vh_fold_head = True
    with torch.no_grad():
        for block in blocks:
            counts["line_mixer"] += 1
            for gamma_name, projection in (("gamma1", block.proj_out), ("gamma2", block.ffn.fc2)):
                gamma = getattr(block, gamma_name)
                if gamma is None:
                    continue
                scale = gamma.detach().view(-1).to(dtype=projection.weight.dtype,
                                                   device=projection.weight.device)
                shape = (-1,) + (1,) * (projection.weight.ndim - 1)
                projection.weight.mul_(scale.view(shape))
                if projection.bias is not None:
                    projection.bias.mul_(scale)
                setattr(block, gamma_name, None)
                counts["layerscale"] += 1
            block._inference_prepared = True
    if blocks:
        model._inference_prepared = True
    return counts
