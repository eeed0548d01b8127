"""End-to-end parity of the VisionHOPE-Tiny classification forward.

The prepared model runs on the GPU through the fused block path and the HIP SRNL kernels.
The reference is the same model on the CPU in FP32, taking the ordinary block path, with
every operator computed by the FP64 CPU oracle. Blocks are perturbed so that every branch
contributes, and BatchNorm statistics are set from the images so the logits depend on them.
"""

import copy

import numpy as np
import pytest
import torch
from torch import nn

from tests.helpers import oracle_operator, perturb_block, rel_err

pytestmark = pytest.mark.gpu


def _tiny_pair(oracle, seed, images):
    """Perturbed Tiny model whose BatchNorm statistics are those of ``images`` (as after
    training, so the pooled features and the logits depend on the input), and its
    prepared CPU copy."""
    from visionhope_amd.inference.prepare import prepare_for_inference
    from visionhope_amd.models import create_model
    from visionhope_amd.models.block import VisionHOPEBlock

    torch.manual_seed(seed)
    model = create_model("visionhope_tiny").eval()
    for i, block in enumerate(m for m in model.modules() if isinstance(m, VisionHOPEBlock)):
        perturb_block(block, seed=seed + i)
    norms = [m for m in model.modules() if isinstance(m, nn.BatchNorm2d)]
    for norm in norms:
        norm.reset_running_stats()
        norm.momentum = None
        norm.train()
    with oracle_operator(oracle), torch.no_grad():
        model(images)
    model.eval()
    reference = copy.deepcopy(model)
    prepare_for_inference(reference)
    return model, reference


# FP32: the operator tolerance holds end to end.  bf16 autocast: every convolution, GEMM
# and activation of 29 blocks rounds to bf16 (as in the reference under autocast), so the
# logits carry a few percent of rounding against the FP32 reference; the bar there is the
# top-1 class, with the logit error bounded loosely.
@pytest.mark.parametrize("autocast,tol", [(False, 1e-4), (True, 6e-2)])
def test_tiny_logits_and_top1(oracle, device, autocast, tol):
    from visionhope_amd.inference.prepare import prepare_for_inference

    gen = torch.Generator().manual_seed(1234)
    calibration = torch.randn(8, 3, 224, 224, generator=gen)
    model, reference = _tiny_pair(oracle, 100, calibration)
    images = calibration[:4]
    with oracle_operator(oracle), torch.no_grad():
        expected = reference(images).double().numpy()

    gpu = model.to(device).to(memory_format=torch.channels_last)
    prepare_for_inference(gpu)
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16, enabled=autocast):
        logits = gpu(images.to(device).contiguous(memory_format=torch.channels_last))
    got = logits.double().cpu().numpy()
    err = rel_err(got, expected)
    print(f"tiny logits autocast={autocast}: normwise relative error {err:.3e}")
    assert err <= tol, f"logits normwise error {err:.3e} > {tol:.0e}"
    # Top-1 must agree wherever the reference's top-2 margin exceeds the observed
    # largest logit error: there the comparison is decided by more than rounding.
    bound = np.abs(got - expected).max()
    top2 = np.sort(expected, axis=1)[:, -2:]
    decided = (top2[:, 1] - top2[:, 0]) > 2 * bound
    assert decided.any(), "no sample has a top-2 margin above the error bound"
    assert (got.argmax(1) == expected.argmax(1))[decided].all()
