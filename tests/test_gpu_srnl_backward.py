"""GPU parity of the SRNL backward (vh_srnl_backward) against autograd of the float64
PyTorch oracle (itself pinned by finite differences in test_oracle_backward.py)."""

import numpy as np
import pytest
import torch

from tests.helpers import assert_close, memories, randn

pytestmark = pytest.mark.gpu

GRAD_TOL = 2e-3   # fp32 recurrence and reductions against float64, relative to each gradient's scale


def _oracle_grads(x, q, mems, chunks, dy, q_raw):
    from oracle.oracle_torch import sequence_forward_torch

    xs = x.double().requires_grad_()
    qs = q.double().requires_grad_()
    ms = [torch.from_numpy(m).double().requires_grad_() for m in mems]
    y = sequence_forward_torch(xs, qs, ms, chunks, q_raw=q_raw)
    (y * dy.double()).sum().backward()
    return [m.grad.numpy() for m in ms] + [xs.grad.numpy(), qs.grad.numpy()]


def _check(got, want, what, tol=GRAD_TOL):
    names = ["dM_m", "dM_v", "dM_k", "dM_eta", "dM_alpha", "dx", "dq"]
    for name, g, w in zip(names, got, want):
        assert g.shape == w.shape, f"{what} {name} shape"
        assert_close(g.detach().double().cpu().numpy(), w, tol, f"{what} {name}")


@pytest.mark.parametrize("head_dim", [4, 8, 16, 32])
@pytest.mark.parametrize("q_raw", [True, False])
@pytest.mark.parametrize("kind", ["perturbed", "strong"])
def test_srnl_backward_matches_oracle(device, head_dim, q_raw, kind):
    from visionhope_amd.models.srnl_core.chunk import srnl_packed_backward

    batch, directions, heads, length = 2, 4, 2, 23
    chunks = [5, 7, 4, 9]                   # ragged last chunks, one length per direction
    mems = memories(directions, heads, head_dim, kind=kind, seed=head_dim + (7 if q_raw else 0))
    x = randn(batch, directions, heads, length, head_dim, seed=3)
    if q_raw:
        q = randn(batch, directions, length, heads * head_dim, seed=4)
    else:
        q = randn(batch, directions, heads, length, head_dim, seed=4)
        q = q / q.norm(dim=-1, keepdim=True)
    dy = randn(batch, directions, heads, length, head_dim, seed=5)
    want = _oracle_grads(x, q, mems, chunks, dy, q_raw)
    got = srnl_packed_backward(tuple(torch.from_numpy(m).to(device) for m in mems), x.to(device), q.to(device),
                               chunks, dy.to(device), q_raw=q_raw)
    _check(got, want, f"d={head_dim} q_raw={q_raw} {kind}")


@pytest.mark.parametrize("heads", [4, 8])
@pytest.mark.parametrize("head_dim", [4, 8, 16])
@pytest.mark.parametrize("q_raw", [True, False])
def test_srnl_backward_packed_lines_match_oracle(device, heads, head_dim, q_raw):
    """Head counts divisible by 4 run the variant that packs 4 lines (consecutive heads of
    one image and direction) into a workgroup for head_dim 4, 8 and 16 with chunks of 64
    or less; raw and normalised queries, ragged chunks, perturbed memories."""
    from visionhope_amd.models.srnl_core.chunk import srnl_packed_backward

    batch, directions, length = 2, 4, 21
    chunks = [6, 4, 8, 5]
    mems = memories(directions, heads, head_dim, kind="perturbed", seed=100 + heads + head_dim)
    x = randn(batch, directions, heads, length, head_dim, seed=31)
    if q_raw:
        q = randn(batch, directions, length, heads * head_dim, seed=32)
    else:
        q = randn(batch, directions, heads, length, head_dim, seed=32)
        q = q / q.norm(dim=-1, keepdim=True)
    dy = randn(batch, directions, heads, length, head_dim, seed=33)
    want = _oracle_grads(x, q, mems, chunks, dy, q_raw)
    got = srnl_packed_backward(tuple(torch.from_numpy(m).to(device) for m in mems), x.to(device), q.to(device),
                               chunks, dy.to(device), q_raw=q_raw)
    _check(got, want, f"heads={heads} d={head_dim} q_raw={q_raw}")


def test_srnl_backward_tiny_stage3_shape(device):
    """The Tiny stage-3 operator shape the packed variant trains on: 8 heads of d = 16 on
    a 14 x 14 map (196-token lines, chunks of 14), one image, raw queries."""
    from visionhope_amd.models.srnl_core.chunk import srnl_packed_backward

    batch, directions, heads, length, d = 1, 4, 8, 196, 16
    chunks = [14, 14, 14, 14]
    mems = memories(directions, heads, d, kind="perturbed", seed=77)
    x = randn(batch, directions, heads, length, d, seed=34)
    q = randn(batch, directions, length, heads * d, seed=35)
    dy = randn(batch, directions, heads, length, d, seed=36)
    want = _oracle_grads(x, q, mems, chunks, dy, True)
    got = srnl_packed_backward(tuple(torch.from_numpy(m).to(device) for m in mems), x.to(device), q.to(device),
                               chunks, dy.to(device), q_raw=True)
    _check(got, want, "Tiny stage 3")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_srnl_backward_low_precision_inputs(device, dtype):
    """bf16 / fp16 x and raw q: the kernel reads the rounded values and computes in fp32;
    the oracle differentiates at the same rounded values."""
    from visionhope_amd.models.srnl_core.chunk import srnl_packed_backward

    batch, directions, heads, length, d = 2, 4, 2, 30, 16
    chunks = [6, 6, 10, 10]
    mems = memories(directions, heads, d, kind="perturbed", seed=21)
    x = randn(batch, directions, heads, length, d, seed=22).to(dtype)
    q = randn(batch, directions, length, heads * d, seed=23).to(dtype)
    dy = randn(batch, directions, heads, length, d, seed=24)
    want = _oracle_grads(x.float(), q.float(), mems, chunks, dy, True)
    got = srnl_packed_backward(tuple(torch.from_numpy(m).to(device) for m in mems), x.to(device), q.to(device),
                               chunks, dy.to(device), q_raw=True)
    assert got[5].dtype == dtype and got[6].dtype == dtype
    _check([g.float() for g in got], want, f"{dtype}", tol=1e-2)   # dx, dq returned rounded to the input dtype


def test_srnl_backward_per_line_memories(device):
    """5-D memories (one state per line): the per-line gradients are not summed."""
    from visionhope_amd.models.srnl_core.chunk import srnl_packed_backward

    batch, directions, heads, length, d = 2, 4, 1, 17, 8
    chunks = [4, 4, 4, 4]
    shared = memories(directions, heads, d, kind="strong", seed=31)
    gen = np.random.default_rng(32)
    mems = tuple(np.ascontiguousarray(np.stack([m + 0.05 * gen.standard_normal(m.shape).astype(np.float32)
                                                for _ in range(batch)]), dtype=np.float32) for m in shared)
    x = randn(batch, directions, heads, length, d, seed=33)
    q = randn(batch, directions, length, heads * d, seed=34)
    dy = randn(batch, directions, heads, length, d, seed=35)
    # oracle: per-line states as lines of one batch each
    from oracle.oracle_torch import srnl_lines_torch
    n = batch * directions * heads
    xs = x.double().requires_grad_()
    qs = q.double().requires_grad_()
    ms = [torch.from_numpy(m).double().requires_grad_() for m in mems]
    q_lines = qs.reshape(batch, directions, length, heads, d).permute(0, 1, 3, 2, 4).reshape(n, length, d)
    y = srnl_lines_torch(xs.reshape(n, length, d), q_lines,
                         [m.reshape((n,) + tuple(m.shape[3:])) for m in ms], list(range(n)), [4] * n)
    (y.reshape(dy.shape) * dy.double()).sum().backward()
    want = [m.grad.numpy() for m in ms] + [xs.grad.numpy(), qs.grad.numpy()]
    got = srnl_packed_backward(tuple(torch.from_numpy(m).to(device) for m in mems), x.to(device), q.to(device),
                               chunks, dy.to(device), q_raw=True)
    _check(got, want, "per-line memories")


def test_srnl_raw_query_function_backward(device):
    """Through the autograd Function (the module's ordinary path): gradients land on the
    parameters and inputs with their shapes and dtypes."""
    from visionhope_amd.models.srnl_core.chunk import srnl_raw_query

    batch, heads, length, d = 2, 2, 20, 16
    mems = [torch.from_numpy(m).to(device).requires_grad_() for m in memories(4, heads, d, kind="perturbed", seed=41)]
    x = randn(batch, 4, heads, length, d, seed=42).to(device).requires_grad_()
    q = randn(batch, 4, length, heads * d, seed=43).to(device).requires_grad_()
    y = srnl_raw_query(*mems, x, q, 6, heads, d)
    dy = randn(*y.shape, seed=44).to(device)
    (y * dy).sum().backward()
    want = _oracle_grads(x.detach().cpu(), q.detach().cpu(), [m.detach().cpu().numpy() for m in mems], [6] * 4,
                         dy.cpu(), True)
    _check([m.grad for m in mems] + [x.grad, q.grad], want, "autograd Function")


def test_srnl_backward_rejects(device):
    from visionhope_amd.models.srnl_core.chunk import srnl_packed_backward

    mems = tuple(torch.from_numpy(m).to(device) for m in memories(4, 1, 16, seed=51))
    x = torch.zeros(1, 4, 1, 270, 16, device=device)
    q = torch.zeros(1, 4, 270, 16, device=device)
    with pytest.raises(ValueError):
        srnl_packed_backward(mems, x, q, [257, 8, 8, 8], torch.zeros_like(x), q_raw=True)   # chunk > 256


@pytest.mark.parametrize("head_dim,chunks,length", [(16, [100, 100, 65, 65], 230), (32, [128, 128, 128, 128], 300),
                                                    (8, [256, 3, 256, 3], 260)])
def test_srnl_backward_long_chunks(device, head_dim, chunks, length):
    """Chunks of 65 to 256 tokens (the long-line range; 256-token LDS buffers), mixed with
    short chunks in other directions, ragged last chunks."""
    from visionhope_amd.models.srnl_core.chunk import srnl_packed_backward

    batch, directions, heads = 1, 4, 2
    mems = memories(directions, heads, head_dim, kind="perturbed", seed=head_dim + 61)
    x = randn(batch, directions, heads, length, head_dim, seed=62, scale=0.5)
    q = randn(batch, directions, length, heads * head_dim, seed=63)
    dy = randn(batch, directions, heads, length, head_dim, seed=64)
    want = _oracle_grads(x, q, mems, chunks, dy, True)
    got = srnl_packed_backward(tuple(torch.from_numpy(m).to(device) for m in mems), x.to(device), q.to(device),
                               chunks, dy.to(device), q_raw=True)
    _check(got, want, f"d={head_dim} chunks={chunks}")


def test_srnl_long_chunk_function_backward(device):
    """Through the long-chunk autograd Function (chunk 96 > 64)."""
    from visionhope_amd.models.srnl_core.lines import srnl_long_chunk

    batch, heads, length, d = 1, 2, 200, 16
    mems = [torch.from_numpy(m).to(device).requires_grad_() for m in memories(4, heads, d, kind="perturbed", seed=71)]
    x = randn(batch, 4, heads, length, d, seed=72, scale=0.5).to(device).requires_grad_()
    q = randn(batch, 4, length, heads * d, seed=73).to(device).requires_grad_()
    y = srnl_long_chunk(*mems, x, q, 96, heads, d)
    dy = randn(*y.shape, seed=74).to(device)
    (y * dy).sum().backward()
    want = _oracle_grads(x.detach().cpu(), q.detach().cpu(), [m.detach().cpu().numpy() for m in mems], [96] * 4,
                         dy.cpu(), True)
    _check([m.grad for m in mems] + [x.grad, q.grad], want, "long-chunk Function")


@pytest.mark.parametrize("head_dim", [4, 8, 16])
@pytest.mark.parametrize("heads", [2, 4, 8])
@pytest.mark.parametrize("q_raw", [True, False])
def test_srnl_backward_lines_per_workgroup(device, head_dim, heads, q_raw):
    """Both launch shapes of the backward: heads % 4 == 0 packs 4 lines (consecutive heads of
    one image and direction) into a workgroup at d <= 16, otherwise 1 line per workgroup.
    Ragged last chunks, one length per direction."""
    from visionhope_amd.models.srnl_core.chunk import srnl_packed_backward

    batch, directions, length = 2, 4, 19
    chunks = [6, 4, 7, 5]
    mems = memories(directions, heads, head_dim, kind="perturbed", seed=100 + heads * head_dim)
    x = randn(batch, directions, heads, length, head_dim, seed=101)
    if q_raw:
        q = randn(batch, directions, length, heads * head_dim, seed=102)
    else:
        q = randn(batch, directions, heads, length, head_dim, seed=102)
        q = q / q.norm(dim=-1, keepdim=True)
    dy = randn(batch, directions, heads, length, head_dim, seed=103)
    want = _oracle_grads(x, q, mems, chunks, dy, q_raw)
    got = srnl_packed_backward(tuple(torch.from_numpy(m).to(device) for m in mems), x.to(device), q.to(device),
                               chunks, dy.to(device), q_raw=q_raw)
    _check(got, want, f"d={head_dim} heads={heads} q_raw={q_raw}")


def test_srnl_backward_tiny_stage3_shape(device):
    """The Tiny stage-3 operator's lines (8 heads of 16, 14x14 map, chunks of 14: the shape
    the packed variant trains on), at batch 2, bf16 inputs as under autocast."""
    from visionhope_amd.models.srnl_core.chunk import srnl_packed_backward

    batch, directions, heads, d, length = 2, 4, 8, 16, 196
    mems = memories(directions, heads, d, kind="perturbed", seed=111)
    x = randn(batch, directions, heads, length, d, seed=112).bfloat16()
    q = randn(batch, directions, length, heads * d, seed=113).bfloat16()
    dy = randn(batch, directions, heads, length, d, seed=114)
    want = _oracle_grads(x.float(), q.float(), mems, [14] * 4, dy, True)
    got = srnl_packed_backward(tuple(torch.from_numpy(m).to(device) for m in mems), x.to(device), q.to(device),
                               [14] * 4, dy.to(device), q_raw=True)
    _check([g.float() for g in got], want, "Tiny stage 3", tol=1e-2)
