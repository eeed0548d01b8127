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
