"""End-to-end parity of the VisionHOPE-Tiny classification forward.

The prepared model runs on the GPU through the fused block path and the HIP SRNL kernels.
The reference is the same model on the CPU in FP32, taking the ordinary block path, with
every operator computed by the FP64 CPU oracle. Blocks are perturbed so that every branch
contributes, and BatchNorm statistics are set from the images so the logits depend on them.

Top-1 (``north_star``: "the same top-1 argmax on backbone logits"; the reference's own
check is ``analysis/benchmark.py:74-87``): an image's class is decided when the oracle's
top-2 margin exceeds twice the largest logit error the GPU shows on that image, so that no
rounding of that size can swap the two classes.  Every decided image must agree, and at
least half of the images must be decided.
"""

import copy

import numpy as np
import pytest
import torch
from torch import nn

from tests.helpers import oracle_operator, perturb_block, rel_err

pytestmark = pytest.mark.gpu

N_IMAGES = 32


def _tiny_model(oracle, seed, images):
    """Perturbed Tiny model whose BatchNorm statistics are those of ``images`` (as after
    training, so the pooled features and the logits depend on the input)."""
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
    return model


@pytest.fixture(scope="module")
def tiny_case(oracle):
    """(unprepared CPU model, 32 images, float64-oracle logits of the prepared CPU model)."""
    from visionhope_amd.inference.prepare import prepare_for_inference

    gen = torch.Generator().manual_seed(1234)
    images = torch.randn(N_IMAGES, 3, 224, 224, generator=gen)
    model = _tiny_model(oracle, 100, images)
    reference = copy.deepcopy(model)
    prepare_for_inference(reference)
    with oracle_operator(oracle), torch.no_grad():
        expected = reference(images).double().numpy()
    return model, images, expected


def _gpu_logits(model, images, device, autocast):
    from visionhope_amd.inference.prepare import prepare_for_inference

    gpu = copy.deepcopy(model).to(device).to(memory_format=torch.channels_last)
    prepare_for_inference(gpu)
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16, enabled=autocast):
        logits = gpu(images.to(device).contiguous(memory_format=torch.channels_last))
    return logits.double().cpu().numpy()


def _check_top1(got, expected, what):
    """Top-1 agreement on every decided image; at least half the images decided."""
    bound = np.abs(got - expected).max(axis=1)              # per-image largest logit error
    top2 = np.sort(expected, axis=1)[:, -2:]
    margin = top2[:, 1] - top2[:, 0]
    decided = margin > 2 * bound
    agree = got.argmax(1) == expected.argmax(1)
    q = np.quantile(margin / np.maximum(bound, 1e-30), [0.0, 0.25, 0.5, 0.75, 1.0])
    print(f"{what}: decided {decided.sum()}/{len(decided)}, agreeing {agree.sum()}/{len(agree)} "
          f"(decided ones {agree[decided].sum()}); margin / error bound quantiles "
          f"{np.array2string(q, precision=2)}; margins {np.array2string(np.quantile(margin, [0, .5, 1]), precision=4)}",
          flush=True)
    assert agree[decided].all(), f"{what}: top-1 differs on a decided image"
    assert decided.sum() * 2 >= len(decided), f"{what}: only {decided.sum()} of {len(decided)} images decided"


# FP32: the operator tolerance holds end to end.  bf16 autocast: every convolution, GEMM
# and activation of 29 blocks rounds to bf16 (as in the reference under autocast), so the
# logits carry a few percent of rounding against the FP32 reference; the bar there is the
# top-1 class, with the logit error bounded loosely.
@pytest.mark.parametrize("autocast,tol", [(False, 1e-4), (True, 6e-2)])
def test_tiny_logits_and_top1(tiny_case, device, autocast, tol):
    model, images, expected = tiny_case
    got = _gpu_logits(model, images, device, autocast)
    err = rel_err(got, expected)
    print(f"tiny logits autocast={autocast}: normwise relative error {err:.3e} over {len(images)} images",
          flush=True)
    assert err <= tol, f"logits normwise error {err:.3e} > {tol:.0e}"
    _check_top1(got, expected, f"top-1 autocast={autocast}")


def test_checkpoint_round_trip_prepared_gpu(tiny_case, device, tmp_path):
    """Native-name weights (``tools/checkpoint.py:17-38``): the perturbed model's state_dict
    saved, loaded into a freshly built Tiny, prepared and run on the GPU in FP32, gives the
    oracle model's logits (1e-4)."""
    from visionhope_amd.models import create_model
    from visionhope_amd.tools.checkpoint import load_checkpoint, save_weights

    model, images, expected = tiny_case
    path = tmp_path / "visionhope_tiny.pth"
    save_weights(path, model.state_dict())
    torch.manual_seed(999)                                  # a different init, overwritten by the load
    fresh = create_model("visionhope_tiny").eval()
    result = load_checkpoint(fresh, path)
    assert not result.missing_keys and not result.unexpected_keys
    got = _gpu_logits(fresh, images[:8], device, False)
    err = rel_err(got, expected[:8])
    print(f"checkpoint round trip: logits normwise {err:.3e}", flush=True)
    assert err <= 1e-4


@pytest.mark.parametrize("overlap", [False, True])
def test_graph_replays_match_eager_forward(tiny_case, device, monkeypatch, overlap):
    """The prepared Tiny forward as the bench runs it (bf16 autocast, inference mode; every
    block's scan, query projection and position encoding in order on one stream, or with
    ``OVERLAP_SCAN`` the scan on a side stream joined before the readout) captured in one
    HIP graph: three replays, with an eager forward and a synchronisation between replays,
    give the eager logits bit for bit, and the eager forwards agree with each other."""
    from visionhope_amd.inference.prepare import prepare_for_inference
    from visionhope_amd.models import block as block_mod

    monkeypatch.setattr(block_mod, "OVERLAP_SCAN", overlap)
    model, images, _ = tiny_case
    gpu = copy.deepcopy(model).to(device).to(memory_format=torch.channels_last)
    prepare_for_inference(gpu)
    batch = images[:16].to(device).contiguous(memory_format=torch.channels_last)
    with torch.inference_mode(), torch.autocast("cuda", dtype=torch.bfloat16):
        eager = gpu(batch)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            captured = gpu(batch)
        for replay in range(3):
            captured.zero_()
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(captured, eager), f"replay {replay} differs from the eager forward"
            again = gpu(batch)
            torch.cuda.synchronize()
            assert torch.equal(again, eager), f"eager forward after replay {replay} differs"


def test_graph_replay_on_changed_input_matches_independent_eager(tiny_case, device):
    """The reference's graph validation (``analysis/benchmark.py:74-87``): the graph is
    captured on one batch, new images are copied into its input buffer, and the replay is
    compared with an independent eager forward of the new images (bf16: atol 1e-3, rtol
    1e-2; the kernels are deterministic, so the logits are also equal bit for bit).  A
    graph that had baked in a stale buffer or a value of the capture batch would fail."""
    from visionhope_amd.inference.prepare import prepare_for_inference

    model, images, _ = tiny_case
    gpu = copy.deepcopy(model).to(device).to(memory_format=torch.channels_last)
    prepare_for_inference(gpu)
    static = images[:8].to(device).contiguous(memory_format=torch.channels_last)
    fresh = images[8:16].flip(-1).to(device).contiguous(memory_format=torch.channels_last)
    with torch.inference_mode(), torch.autocast("cuda", dtype=torch.bfloat16):
        gpu(static)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            captured = gpu(static)
        outputs = []
        for replay in range(2):
            static.copy_(fresh if replay == 0 else images[:8].to(device))
            graph.replay()
            torch.cuda.synchronize()
            expected = gpu(static.clone().contiguous(memory_format=torch.channels_last))
            torch.cuda.synchronize()
            torch.testing.assert_close(captured.float(), expected.float(), atol=1e-3, rtol=1e-2)
            assert torch.equal(captured, expected), f"replay {replay} on changed input differs from eager"
            outputs.append(captured.clone())
    assert not torch.equal(outputs[0], outputs[1]), "the two input batches gave the same logits"


@pytest.mark.parametrize("autocast", [False, True])
def test_query_once_and_launch_audit(tiny_case, device, autocast):
    """The reference's fast-path audit (``inference/audit.py:11-99``,
    ``analysis/benchmark.py:48-71``) on the prepared Tiny forward: each of the 29 operators
    projects B*H*W queries exactly once, and the profiler trace holds exactly one scan and
    one readout launch per operator call."""
    from visionhope_amd.inference.audit import audit_fast_path
    from visionhope_amd.inference.prepare import prepare_for_inference

    model, images, _ = tiny_case
    gpu = copy.deepcopy(model).to(device).to(memory_format=torch.channels_last)
    prepare_for_inference(gpu)
    batch = images[:4].to(device).contiguous(memory_format=torch.channels_last)
    with torch.inference_mode(), torch.autocast("cuda", dtype=torch.bfloat16, enabled=autocast):
        gpu(batch)
        _, evidence = audit_fast_path(gpu, lambda: gpu(batch))
    print(f"audit autocast={autocast}: {evidence}", flush=True)
    assert evidence["fused_operators"] == 29 and evidence["fused_srnl_calls"] == 29
    assert evidence["scan_kernels"] == 29 and evidence["readout_kernels"] == 29
    assert evidence["query_once"] is True
    # every block's position encoding is computed inside its readout
    assert evidence["separate_lepe_kernels"] == 0
