"""Pins of the differentiable SRNL oracle (the checker of the backward kernels): its
forward against the C oracle and the NumPy formulation, its gradients against central
finite differences."""

import numpy as np
import pytest
import torch

from tests.helpers import memories, randn


def _case(d, length, kind, seed, lines=3):
    mems = memories(1, lines, d, kind=kind, seed=seed)
    mems = tuple(m.reshape((lines,) + m.shape[2:]) for m in mems)
    x = randn(lines, length, d, seed=seed + 1).numpy()
    q = randn(lines, length, d, seed=seed + 2).numpy()
    return x, q, mems


@pytest.mark.parametrize("d,length,chunk", [(4, 11, 3), (8, 9, 4), (16, 20, 7)])
@pytest.mark.parametrize("kind", ["perturbed", "strong"])
@pytest.mark.parametrize("q_raw", [True, False])
def test_torch_oracle_forward_matches_c_and_numpy(oracle, d, length, chunk, kind, q_raw):
    from oracle.oracle_torch import srnl_lines_torch

    x, q, mems = _case(d, length, kind, seed=d * 7 + length)
    if not q_raw:
        q = q / np.linalg.norm(q, axis=-1, keepdims=True)
    idx = np.arange(x.shape[0])
    chunks = np.full(x.shape[0], chunk)
    got = srnl_lines_torch(torch.from_numpy(x).double(), torch.from_numpy(q).double(),
                           [torch.from_numpy(m).double() for m in mems], idx, chunks, q_raw=q_raw).numpy()
    c_ref = oracle.srnl_lines(x, q, mems, idx, chunks, q_raw=q_raw, dtype=np.float64)
    np_ref = oracle.srnl_lines_numpy(x, q, mems, idx, chunks, q_raw=q_raw)
    scale = np.abs(c_ref).max()
    assert np.abs(got - c_ref).max() <= 1e-12 * max(scale, 1.0)
    assert np.abs(got - np_ref).max() <= 1e-12 * max(scale, 1.0)


@pytest.mark.parametrize("kind", ["perturbed", "strong"])
@pytest.mark.parametrize("q_raw", [True, False])
def test_torch_oracle_gradients_match_finite_differences(kind, q_raw):
    """gradcheck on every input: x, q and the five memories (two lines share a state)."""
    from oracle.oracle_torch import srnl_lines_torch

    d, length, chunk = 4, 7, 3
    x, q, mems = _case(d, length, kind, seed=11, lines=2)
    xs = torch.from_numpy(x).double().requires_grad_()
    qs = torch.from_numpy(q).double().requires_grad_()
    ms = [torch.from_numpy(m[:1]).double().requires_grad_() for m in mems]   # one state shared by both lines

    def fn(x_, q_, *m_):
        return srnl_lines_torch(x_, q_, m_, [0, 0], [chunk, chunk], q_raw=q_raw)

    assert torch.autograd.gradcheck(fn, (xs, qs, *ms), eps=1e-6, atol=1e-7, rtol=1e-5)


def test_torch_oracle_catches_a_dropped_state_term():
    """A planted mistake: without the refresh of the value memory the output differs, so
    the forward pin above is sensitive to the state path the backward differentiates."""
    from oracle.oracle_torch import srnl_lines_torch

    x, q, mems = _case(8, 12, "strong", seed=5, lines=1)
    tx, tq = torch.from_numpy(x).double(), torch.from_numpy(q).double()
    tm = [torch.from_numpy(m).double() for m in mems]
    y = srnl_lines_torch(tx, tq, tm, [0], [4])
    frozen = [tm[0], tm[1].detach() * 0 + tm[1], tm[2], tm[3], tm[4]]
    y2 = srnl_lines_torch(tx, tq, frozen, [0], [4])
    assert torch.equal(y, y2)   # same inputs, same output (determinism)
    tm_bad = [tm[0], tm[1] * 0, tm[2], tm[3], tm[4]]
    assert (srnl_lines_torch(tx, tq, tm_bad, [0], [4]) - y).abs().max() > 1e-3


def _np(t):
    return t.detach().numpy()


def test_residual_add_special_cases(oracle):
    """oracle.residual_add pinned without a second restatement: gamma = 0 or a dropped
    sample (drop scale 0) returns the residual bit for bit; gamma = drop = 1 is the fp32
    sum; scaling the branch by 2 scales the increment by exactly 2 (powers of two are exact
    in fp32); the drop scale applies per sample, not per channel."""
    rng = np.random.default_rng(3)
    res = rng.normal(size=(3, 4, 5, 6)).astype(np.float32)
    br = rng.normal(size=(3, 4, 5, 6)).astype(np.float32)
    gamma = rng.normal(size=6).astype(np.float32)
    ones = np.ones(3, np.float32)
    np.testing.assert_array_equal(oracle.residual_add(res, br, np.zeros(6, np.float32), ones), res)
    drop = np.array([1.0, 0.0, 2.0], np.float32)
    out = oracle.residual_add(res, br, gamma, drop)
    np.testing.assert_array_equal(out[1], res[1])
    np.testing.assert_array_equal(oracle.residual_add(res, br, np.ones(6, np.float32), ones), res + br)
    inc1 = oracle.residual_add(np.zeros_like(res), br, gamma, drop)
    inc2 = oracle.residual_add(np.zeros_like(res), 2 * br, gamma, drop)
    np.testing.assert_array_equal(inc2, 2 * inc1)
    np.testing.assert_array_equal(inc1[2], 2 * oracle.residual_add(np.zeros_like(res), br, gamma, ones)[2])


def test_torch_tail_forwards_match_numpy_oracle(oracle):
    """Each tail forward of the differentiable oracle against the NumPy restatement."""
    from oracle import oracle_torch as ot

    b, heads, d, h, w = 2, 3, 4, 5, 7
    c, length = heads * d, h * w
    y = randn(b, 4, heads, length, d, seed=61).double()
    x = randn(b, 4, heads, length, d, seed=62).double()
    for skip_shape in ((heads, d), (4, heads, d)):
        skip = randn(*skip_shape, seed=63).double()
        scale = randn(4, c, seed=64).double()
        want = oracle.direction_fusion(_np(y), _np(x), _np(skip), _np(scale), h, w)
        got = _np(ot.direction_fusion_torch(y, x, skip, scale, h, w))
        assert np.abs(got - want).max() <= 1e-5 * np.abs(want).max()
    xm = randn(b, c, h, w, seed=65).double()
    gamma, beta = randn(c, seed=66).double(), randn(c, seed=67).double()
    want = oracle.grn(_np(xm), _np(gamma), _np(beta))
    assert np.abs(_np(ot.grn_torch(xm, gamma, beta)) - want).max() <= 1e-5 * np.abs(want).max()
    want = oracle.layernorm2d(_np(xm), _np(gamma), _np(beta))
    assert np.abs(_np(ot.layernorm2d_torch(xm, gamma, beta)) - want).max() <= 1e-5 * np.abs(want).max()
    q = randn(b, 4, length, c, seed=68).double()
    q[0, 1, 2, :d] = 0.0
    want, _ = oracle.qnorm(_np(q), heads, d)
    assert np.abs(_np(ot.qnorm_torch(q, heads, d)) - want).max() <= 1e-6
    res = randn(b, c, h, w, seed=69).double()
    drop = torch.tensor([0.0, 2.0], dtype=torch.float64)
    want = oracle.residual_add(_np(res).transpose(0, 2, 3, 1), _np(xm).transpose(0, 2, 3, 1), _np(gamma), _np(drop))
    got = _np(ot.residual_add_torch(res, xm, gamma, drop)).transpose(0, 2, 3, 1)
    assert np.abs(got - want).max() <= 1e-5 * np.abs(want).max()


def test_torch_tail_gradients_match_finite_differences():
    from oracle import oracle_torch as ot

    b, heads, d, h, w = 2, 2, 2, 3, 4
    c, length = heads * d, h * w
    f64 = dict(dtype=torch.float64, requires_grad=True)
    y = torch.randn(b, 4, heads, length, d, **f64)
    x = torch.randn(b, 4, heads, length, d, **f64)
    for skip_shape in ((heads, d), (4, heads, d)):
        skip = torch.randn(*skip_shape, **f64)
        scale = torch.randn(4, c, **f64)
        assert torch.autograd.gradcheck(lambda *a: ot.direction_fusion_torch(*a, h, w), (y, x, skip, scale))
    xm = torch.randn(b, c, h, w, **f64)
    gamma, beta = torch.randn(c, **f64), torch.randn(c, **f64)
    assert torch.autograd.gradcheck(ot.grn_torch, (xm, gamma, beta))
    assert torch.autograd.gradcheck(ot.layernorm2d_torch, (xm, gamma, beta))
    q = torch.randn(b, 4, length, c, **f64)
    assert torch.autograd.gradcheck(lambda t: ot.qnorm_torch(t, heads, d), (q,))
    res = torch.randn(b, c, h, w, **f64)
    drop = torch.tensor([0.0, 2.0], dtype=torch.float64)
    assert torch.autograd.gradcheck(lambda r_, b_, g_: ot.residual_add_torch(r_, b_, g_, drop), (res, xm, gamma))


def test_torch_fusion_catches_a_swapped_direction():
    """A planted mistake: exchanging the two column scans changes the fused output, so the
    forward pin above checks the restore maps the gradients are routed through."""
    from oracle import oracle_torch as ot

    b, heads, d, h, w = 1, 1, 2, 3, 4
    y = randn(b, 4, heads, h * w, d, seed=71).double()
    x = randn(b, 4, heads, h * w, d, seed=72).double()
    skip, scale = randn(heads, d, seed=73).double(), torch.ones(4, heads * d, dtype=torch.float64)
    good = ot.direction_fusion_torch(y, x, skip, scale, h, w)
    bad = ot.direction_fusion_torch(y[:, [0, 1, 3, 2]], x[:, [0, 1, 3, 2]], skip, scale, h, w)
    assert (good - bad).abs().max() > 1e-3
