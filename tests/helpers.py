"""Shared test helpers: seeded inputs, parameter sets, error metrics."""

import numpy as np
import torch

SEED = 1234


def rel_err(actual, expected):
    """Normwise relative error ||a - b|| / ||b|| in float64."""
    a = np.asarray(actual, dtype=np.float64)
    b = np.asarray(expected, dtype=np.float64)
    denom = np.linalg.norm(b)
    return float(np.linalg.norm(a - b) / denom) if denom > 0 else float(np.linalg.norm(a))


def max_rel_err(actual, expected):
    """max |a - b| / max |b| (elementwise error on the output's scale)."""
    a = np.asarray(actual, dtype=np.float64)
    b = np.asarray(expected, dtype=np.float64)
    scale = np.abs(b).max()
    return float(np.abs(a - b).max() / scale) if scale > 0 else float(np.abs(a).max())


def assert_close(actual, expected, tol, what=""):
    r, m = rel_err(actual, expected), max_rel_err(actual, expected)
    assert r <= tol and m <= tol, f"{what}: normwise {r:.3e}, elementwise {m:.3e} > {tol:.1e}"


def memories(directions, heads, head_dim, *, kind="perturbed", seed=SEED):
    """SRNL memories as numpy fp32 ``[R, heads, d, d]`` x3 and ``[R, heads, d]`` x2.

    default   — the reference's init (``srnl.py:70-74``): trunc-normal std 0.01 matrices,
                zero gate vectors (every gate constant).
    perturbed — gate vectors ~ N(0, 0.1^2) so the gates vary per token.
    strong    — matrices std 0.3 and gate vectors ~ N(0, 0.5^2): large steps, active
                soft cap and spectral clamp.
    """
    gen = torch.Generator().manual_seed(seed)
    shape_m = (directions, heads, head_dim, head_dim)
    shape_v = (directions, heads, head_dim)
    std = 0.3 if kind == "strong" else 0.01
    mats = []
    for _ in range(3):
        t = torch.empty(shape_m)
        torch.nn.init.trunc_normal_(t, std=std, generator=gen)
        mats.append(t.numpy())
    if kind == "default":
        vecs = [np.zeros(shape_v, np.float32), np.zeros(shape_v, np.float32)]
    else:
        vstd = 0.5 if kind == "strong" else 0.1
        vecs = [(torch.randn(shape_v, generator=gen) * vstd).numpy() for _ in range(2)]
    return tuple(np.ascontiguousarray(m, dtype=np.float32) for m in (*mats, *vecs))


def randn(*shape, seed=SEED, scale=1.0):
    gen = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=gen) * scale)


def to_dev(arrays, device):
    return tuple(torch.as_tensor(a).to(device) for a in arrays)


def perturb_block(block, seed):
    """Parameters of a VisionHOPE block at scales that exercise every branch: LayerScale
    in [0.5, 1], gate vectors ~ N(0, 0.1^2), other tensors offset by small noise; the SRNL
    matrix memories keep their init."""
    gen = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for name, p in block.named_parameters():
            if name.startswith("operator.srnl.M_") and p.ndim == 3:
                continue
            if name in ("gamma1", "gamma2"):
                p.copy_(0.5 + 0.5 * torch.rand(p.shape, generator=gen))
            elif name.startswith("operator.srnl.M_"):
                p.copy_(torch.randn(p.shape, generator=gen) * 0.1)
            else:
                p.add_(torch.randn(p.shape, generator=gen) * (0.05 if p.ndim > 1 else 0.1))


class oracle_operator:
    """Context manager: VisionHOPEOperator.forward computed by the FP64 CPU oracle (CPU
    tensors; the result is returned in the input's dtype, NCHW)."""

    def __init__(self, oracle):
        self.oracle = oracle

    def __enter__(self):
        from visionhope_amd.models import operator as op_mod

        oracle = self.oracle

        def forward(op, xin, *, channels_last=None):
            x_nhwc = xin.permute(0, 2, 3, 1).contiguous()
            with torch.no_grad():
                q = op.W_q(x_nhwc)
            mems = tuple(m.detach().double().numpy() for m in op.srnl.initial_memories)
            out = oracle.operator_forward(x_nhwc.double().numpy(), q.double().numpy(), mems,
                                          op.d_skip.detach().double().numpy(),
                                          op.direction_weights().detach().double().numpy(),
                                          op.head_dim, dtype=np.float64)
            return torch.from_numpy(out).to(xin.dtype).permute(0, 3, 1, 2)

        self._module = op_mod
        self._original = op_mod.VisionHOPEOperator.forward
        op_mod.VisionHOPEOperator.forward = forward
        return self

    def __exit__(self, *exc):
        self._module.VisionHOPEOperator.forward = self._original
        return False
