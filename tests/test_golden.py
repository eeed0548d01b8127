"""Committed golden fixtures (tests/golden/*.npz, written by tests/golden/make_fixtures.py
from the fp64 oracle): the fp32 oracle on the CPU and the HIP kernels on the GPU must
both reproduce them."""

from pathlib import Path

import numpy as np
import pytest
import torch

from tests.helpers import assert_close

GOLDEN = Path(__file__).resolve().parent / "golden"
NAMES = ("M_m", "M_v", "M_k", "M_eta", "M_alpha")


def _load(name):
    with np.load(GOLDEN / name, allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


@pytest.mark.parametrize("kind", ["default", "perturbed"])
def test_oracle_reproduces_config1_fixture(oracle, kind):
    g = _load("srnl_config1.npz")
    mems = tuple(g[f"{kind}_{n}"] for n in NAMES)
    x = g["x"]
    packed = x.reshape(2, 1, 196, 2, 32).transpose(0, 1, 3, 2, 4)
    y = oracle.sequence_forward(packed, x.reshape(2, 1, 196, 64), mems, [14])
    assert_close(y[:, 0].transpose(0, 2, 1, 3).reshape(2, 196, 64), g[f"{kind}_y"], 1e-5, kind)


def test_oracle_reproduces_operator_fixture(oracle):
    g = _load("operator_7x9.npz")
    out = oracle.operator_forward(g["x"], g["q"], tuple(g[n] for n in NAMES), g["d_skip"],
                                  g["weights"], 16)
    assert_close(out, g["out"], 1e-5, "operator")


@pytest.mark.gpu
@pytest.mark.parametrize("kind", ["default", "perturbed"])
def test_gpu_srnl_module_reproduces_config1_fixture(device, kind):
    from visionhope_amd.models import SRNL

    g = _load("srnl_config1.npz")
    module = SRNL(64, head_dim=32, chunk_size=14).to(device).eval()
    with torch.no_grad():
        for n in NAMES:
            getattr(module, f"{n}_0").copy_(torch.from_numpy(g[f"{kind}_{n}"]))
        y = module(torch.from_numpy(g["x"]).to(device)).cpu().numpy()
    assert_close(y, g[f"{kind}_y"], 1e-4, kind)


@pytest.mark.gpu
def test_gpu_operator_reproduces_fixture(device):
    from visionhope_amd.models.srnl_core.fused import srnl_spatial_inference

    g = _load("operator_7x9.npz")
    mems = tuple(torch.from_numpy(g[n]).to(device) for n in NAMES)
    out = srnl_spatial_inference(mems, torch.from_numpy(g["x"]).to(device),
                                 torch.from_numpy(g["q"]).to(device),
                                 torch.from_numpy(g["d_skip"]).reshape(-1).to(device),
                                 torch.from_numpy(g["weights"]).to(device), (9, 9, 7, 7))
    assert_close(out.cpu().numpy(), g["out"], 1e-4, "operator")
