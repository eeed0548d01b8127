"""GPU parity of the operator-tail backward kernels (direction fusion, GRN, LayerNorm2d,
query normalisation, residual add) against autograd of the float64 oracle (pinned by
finite differences in test_oracle_backward.py).  Each case runs the module's autograd
Function, so the gradients come from the C-ABI entry points."""

import pytest
import torch

from tests.helpers import assert_close, randn

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-4, torch.bfloat16: 1e-2, torch.float16: 1e-2}


def _grads(fn, inputs, dout):
    """Gradients of sum(fn(*inputs) * dout) in float64 on the CPU."""
    leaves = [t.detach().double().cpu().requires_grad_() for t in inputs]
    (fn(*leaves) * dout.double().cpu()).sum().backward()
    return [t.grad for t in leaves]


def _check(got, want, tol, what):
    for i, (g, w) in enumerate(zip(got, want)):
        assert g is not None, f"{what}: gradient {i} missing"
        assert tuple(g.shape) == tuple(w.shape), f"{what}: gradient {i} shape {tuple(g.shape)} vs {tuple(w.shape)}"
        assert_close(g.detach().double().cpu().numpy(), w.numpy(), tol, f"{what} gradient {i}")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("per_dir", [False, True])
@pytest.mark.parametrize("channels_last", [False, True])
@pytest.mark.parametrize("shape", [(2, 3, 8, 5, 7), (2, 5, 64, 4, 6), (8, 6, 16, 28, 28), (2, 4, 4, 6, 5),
                                   (2, 12, 16, 9, 10), (1, 1, 16, 1, 1)])
def test_direction_fusion_backward(device, dtype, per_dir, channels_last, shape):
    from oracle.oracle_torch import direction_fusion_torch
    from visionhope_amd.utils.direction_fusion import visionhope_postprocess_scale

    b, heads, d, h, w = shape
    c, length = heads * d, h * w
    y = randn(b, 4, heads, length, d, seed=1).to(dtype)
    x = randn(b, 4, heads, length, d, seed=2).to(dtype)
    skip = randn(*((4, heads, d) if per_dir else (heads, d)), seed=3)
    scale = randn(4, c, seed=4)
    dout = randn(b, c, h, w, seed=5)
    want = _grads(lambda *a: direction_fusion_torch(*a, h, w), (y, x, skip, scale), dout)
    leaves = [t.to(device).requires_grad_() for t in (y, x, skip, scale)]
    out = visionhope_postprocess_scale(*leaves, h, w, channels_last=channels_last)
    g = dout.to(device)
    if channels_last:
        g = g.contiguous(memory_format=torch.channels_last)
    out.backward(g)
    assert leaves[0].grad.dtype == dtype and leaves[2].grad.dtype == torch.float32
    _check([t.grad for t in leaves], want, TOL[dtype], f"fusion {shape} {dtype} per_dir={per_dir}")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape", [(2, 24, 5, 7), (3, 300, 4, 4), (4, 96, 28, 28), (1, 8, 1, 1)])
def test_grn_backward(device, dtype, shape):
    from oracle.oracle_torch import grn_torch
    from visionhope_amd.utils.grn_cuda import visionhope_grn

    b, c, h, w = shape
    x = randn(*shape, seed=11).to(dtype)
    x[0, 1] = 0          # a channel with zero norm: its normalisation term drops out
    gamma, beta = randn(c, seed=12), randn(c, seed=13)
    dout = randn(*shape, seed=14)
    want = _grads(grn_torch, (x, gamma, beta), dout)
    leaves = [x.to(device).contiguous(memory_format=torch.channels_last).requires_grad_(),
              gamma.to(device).requires_grad_(), beta.to(device).requires_grad_()]
    visionhope_grn(*leaves, 1e-6).backward(dout.to(device))
    assert leaves[0].grad.dtype == dtype
    _check([t.grad for t in leaves], want, TOL[dtype], f"GRN {shape} {dtype}")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("channels", [8, 24, 96, 192, 384, 768, 1000, 3])
@pytest.mark.parametrize("channels_last", [True, False])
def test_layernorm2d_backward(device, dtype, channels, channels_last):
    from oracle.oracle_torch import layernorm2d_torch
    from visionhope_amd.utils.layer_norm_cuda import visionhope_layernorm2d

    # 96 channels at 56x56x4 rows runs the grid-stride loop more than once
    b, h, w = (4, 56, 56) if channels == 96 else (2, 7, 9)
    shape = (b, channels, h, w)
    x = (randn(*shape, seed=21) * 2 + 0.5).to(dtype)
    weight, bias = randn(channels, seed=22), randn(channels, seed=23)
    dout = randn(*shape, seed=24)
    want = _grads(layernorm2d_torch, (x, weight, bias), dout)
    xd = x.to(device)
    if channels_last:
        xd = xd.contiguous(memory_format=torch.channels_last)
    leaves = [xd.requires_grad_(), weight.to(device).requires_grad_(), bias.to(device).requires_grad_()]
    visionhope_layernorm2d(*leaves, 1e-6).backward(dout.to(device))
    assert leaves[0].grad.dtype == dtype
    _check([t.grad for t in leaves], want, TOL[dtype], f"LN C={channels} {dtype} cl={channels_last}")


def test_layernorm2d_backward_rejects_wide_rows(device):
    from visionhope_amd.utils.layer_norm_cuda import visionhope_layernorm2d

    x = torch.zeros(1, 1040, 2, 2, device=device, requires_grad=True)
    y = visionhope_layernorm2d(x, torch.ones(1040, device=device), torch.zeros(1040, device=device), 1e-6)
    with pytest.raises(RuntimeError, match="at most 1024 channels"):
        y.sum().backward()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("head_dim", [4, 16, 64])
def test_qnorm_backward(device, dtype, head_dim):
    from oracle.oracle_torch import qnorm_torch
    from visionhope_amd.utils.query_normalization import visionhope_qnorm

    b, heads, length = 2, 3, 11
    q = randn(b, 4, length, heads * head_dim, seed=31).to(dtype)
    q[1, 2, 3, :head_dim] = 0      # zero query: the epsilon branch (no projection term)
    dout = randn(b, 4, heads, length, head_dim, seed=32)
    dout[1, 2, 0, 3] *= 1e-12      # its gradient is dout / 1e-12; keep it on the others' scale
    want = _grads(lambda t: qnorm_torch(t, heads, head_dim), (q,), dout)
    leaf = q.to(device).requires_grad_()
    visionhope_qnorm(leaf, heads, head_dim).backward(dout.to(device))
    assert leaf.grad.dtype == dtype
    _check([leaf.grad], want, TOL[dtype], f"qnorm d={head_dim} {dtype}")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape", [(2, 24, 5, 7), (3, 300, 4, 4), (4, 96, 28, 28)])
def test_residual_add_backward(device, dtype, shape):
    from oracle.oracle_torch import residual_add_torch
    from visionhope_amd.utils.residual import _VisionHOPEResidualFunction

    b = shape[0]
    res = randn(*shape, seed=41)
    branch = randn(*shape, seed=42).to(dtype)
    gamma = randn(shape[1], seed=43)
    drop = torch.tensor([0.0, 2.0, 1.0, 0.5][:b])
    dout = randn(*shape, seed=44)
    want = _grads(lambda r_, b_, g_: residual_add_torch(r_, b_, g_, drop), (res, branch, gamma), dout)
    cl = torch.channels_last
    leaves = [res.to(device).contiguous(memory_format=cl).requires_grad_(),
              branch.to(device).contiguous(memory_format=cl).requires_grad_(), gamma.to(device).requires_grad_()]
    _VisionHOPEResidualFunction.apply(*leaves, drop.to(device)).backward(dout.to(device))
    assert leaves[1].grad.dtype == dtype
    _check([t.grad for t in leaves], want, TOL[dtype], f"residual {shape} {dtype}")


class _torch_oracle_operator:
    """Context manager: the operator's ordinary forward computed by the differentiable
    oracle (CPU tensors, their dtype), so a whole block can be differentiated on the CPU."""

    def __enter__(self):
        from oracle.oracle_torch import direction_fusion_torch, sequence_forward_torch
        from visionhope_amd.models import operator as op_mod

        def seq_forward(op, x, channels_last, *, memories=None):
            b, _, h, w = x.shape
            seq_hw = x.flatten(2).transpose(1, 2)
            xs = op.serialize(x, seq_hw)
            xc = xs.view(b, 4, xs.shape[2], op.num_heads, op.head_dim).transpose(2, 3).contiguous()
            q_raw = op.project_queries(seq_hw, h, w)
            chunk = op.srnl.chunk_size
            chunks = [chunk] * 4 if chunk is not None else [w, w, h, h]
            y = sequence_forward_torch(xc, q_raw, list(op.srnl.initial_memories), chunks, q_raw=True)
            return direction_fusion_torch(y, xc, op.d_skip, op.direction_weights(), h, w)

        self._module = op_mod
        self._original = op_mod.VisionHOPEOperator._sequence_forward
        op_mod.VisionHOPEOperator._sequence_forward = seq_forward
        return self

    def __exit__(self, *exc):
        self._module.VisionHOPEOperator._sequence_forward = self._original
        return False


@pytest.mark.parametrize("hw", [(8, 8), (6, 10)])
def test_block_training_gradients(device, hw):
    """One training step's gradients of a whole VisionHOPE block (CPE, LayerNorm, the SRNL
    operator with fusion, gated local branch, GRN FFN, LayerScale residuals) on the GPU
    against the same block on the CPU with the oracle operator (float32 there too: the
    module contract makes LayerNorm and GRN return FP32)."""
    import copy

    from tests.helpers import perturb_block
    from visionhope_amd.models.block import VisionHOPEBlock

    torch.manual_seed(0)
    block = VisionHOPEBlock(32, head_dim=16, layer_scale_init_value=0.5)
    perturb_block(block, seed=81)
    block.train()
    ref = copy.deepcopy(block)
    h, w = hw
    x = randn(2, 32, h, w, seed=82)
    dout = randn(2, 32, h, w, seed=83)
    xr = x.clone().requires_grad_()
    with _torch_oracle_operator():
        (ref(xr) * dout).sum().backward()
    gpu = block.to(device)
    xg = x.to(device).contiguous(memory_format=torch.channels_last).requires_grad_()
    (gpu(xg) * dout.to(device)).sum().backward()
    assert_close(xg.grad.double().cpu().numpy(), xr.grad.numpy(), 1e-3, f"block {hw} dx")
    for (name, p), (_, q) in zip(gpu.named_parameters(), ref.named_parameters()):
        assert p.grad is not None, f"{name} has no gradient"
        assert_close(p.grad.double().cpu().numpy(), q.grad.numpy(), 1e-3, f"block {hw} d{name}")
