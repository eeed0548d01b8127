"""One-time switch of a VisionHOPE model (or a bare SRNL / operator) to its inference path.

Public surface of the reference's ``inference/prepare.py:12-54``: ``prepare_for_inference``
returns the same counts and folds LayerScale into the projections it scales, in place.
"""

import torch

from ..models.block import VisionHOPEBlock
from ..models.layers import Downsample, LayerNorm2d, PatchEmbedding
from ..models.operator import VisionHOPEOperator
from ..models.srnl import SRNL
from ..utils.grn import GlobalResponseNorm

_COUNT_KEYS = ("line_mixer", "srnl", "operator", "layernorm2d", "grn", "layerscale")


def _enable(module):
    """Switch one module to its inference path; the count key it belongs to, if any."""
    if isinstance(module, SRNL):
        module.fast_inference = True
        return "srnl"
    if isinstance(module, VisionHOPEOperator):
        return "operator"
    if isinstance(module, LayerNorm2d):
        module.inference_layout = True
        return "layernorm2d"
    if isinstance(module, GlobalResponseNorm):
        return "grn"
    if isinstance(module, (PatchEmbedding, Downsample)):
        # Eval BatchNorm folded into the convolution on the GPU path (a cached copy beside
        # the module; the parameters are unchanged).
        module._vh_fold_bn = True
    if hasattr(module, "head_pre_logits") and hasattr(module, "head_norm"):
        # The classifier head: its BatchNorm likewise, LayerNorm and SiLU fused around the
        # 1x1 projection.
        module._vh_fold_head = True
    return None


def _fold_layer_scale(block):
    """Multiply each LayerScale into the output channels of the projection it scales
    (``proj_out`` for ``gamma1``, ``ffn.fc2`` for ``gamma2``) and drop it.  Returns the
    number folded."""
    folded = 0
    for name, projection in (("gamma1", block.proj_out), ("gamma2", block.ffn.fc2)):
        gamma = getattr(block, name)
        if gamma is None:
            continue
        scale = gamma.detach().reshape(-1).to(device=projection.weight.device, dtype=projection.weight.dtype)
        projection.weight.mul_(scale.reshape((-1,) + (1,) * (projection.weight.dim() - 1)))
        if projection.bias is not None:
            projection.bias.mul_(scale)
        setattr(block, name, None)
        folded += 1
    return folded


def prepare_for_inference(model):
    """Evaluation mode, fast inference everywhere, LayerScale folded into the blocks'
    projection weights in place (prepare an eval-only copy).  Returns counts per
    component; ``line_mixer`` counts the prepared blocks."""
    blocks = [m for m in model.modules() if isinstance(m, VisionHOPEBlock)]
    if any(type(b.operator) is not VisionHOPEOperator or type(b.operator.srnl) is not SRNL for b in blocks):
        raise ValueError("Production fusion requires the unmodified VisionHOPE operator and SRNL")
    model.eval()
    counts = dict.fromkeys(_COUNT_KEYS, 0)
    for module in model.modules():
        key = _enable(module)
        if key is not None:
            counts[key] += 1
    with torch.no_grad():
        for block in blocks:
            counts["layerscale"] += _fold_layer_scale(block)
            counts["line_mixer"] += 1
            block._inference_prepared = True
    if blocks:
        model._inference_prepared = True
    return counts
