"""Config 4 (VisionHOPE-Base at 512x512, dense-prediction features) on the GPU at full size
(chunks of 128 tokens at stage 1): the prepared fused bf16 path is as close to the FP32
module path as the unprepared bf16 module path is, and repeatable."""

import pytest
import torch

from tests.helpers import rel_err

pytestmark = pytest.mark.gpu


def test_base512_features_fused_matches_module_path(device):
    import copy

    from visionhope_amd.inference.prepare import prepare_for_inference
    from visionhope_amd.models import create_model

    torch.manual_seed(0)
    model = create_model("visionhope_base", drop_path_rate=0.0).to(device).to(memory_format=torch.channels_last)
    model.eval()
    prepared = copy.deepcopy(model)
    prepare_for_inference(prepared)
    gen = torch.Generator().manual_seed(5)
    images = torch.randn(2, 3, 512, 512, generator=gen).to(device).contiguous(memory_format=torch.channels_last)
    with torch.no_grad():
        truth = model.forward_intermediates(images)
        with torch.autocast("cuda", dtype=torch.bfloat16):
            module_bf16 = model.forward_intermediates(images)
            got = prepared.forward_intermediates(images)
            again = prepared.forward_intermediates(images)
    shapes = [(2, 96, 128, 128), (2, 192, 64, 64), (2, 448, 32, 32), (2, 640, 16, 16)]
    for i, (g, m, t, a, shape) in enumerate(zip(got, module_bf16, truth, again, shapes)):
        assert tuple(g.shape) == shape and torch.isfinite(g).all(), f"stage {i}"
        assert torch.equal(g, a), f"stage {i} not repeatable"
        t = t.float().cpu().numpy()
        e_fused = rel_err(g.float().cpu().numpy(), t)
        e_module = rel_err(m.float().cpu().numpy(), t)
        print(f"stage {i}: bf16 fused {e_fused:.3e}, bf16 module {e_module:.3e} (normwise vs FP32)")
        assert e_fused <= 1.25 * e_module + 5e-3, f"stage {i}: fused {e_fused:.3e} vs module {e_module:.3e}"
