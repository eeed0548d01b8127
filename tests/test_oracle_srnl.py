"""Pin the SRNL CPU oracle (oracle/srnl_oracle.c) without the reference.

The reference ships no golden vectors and its SRNL exists only as CUDA source
(and cannot be built here), so the oracle is pinned by:
  * an independent NumPy fp64 formulation (chunk-level matrix algebra),
  * closed forms: first chunk = plain GEMM; zero key/value memories = pure decay by
    sigma(ln 9) = 0.9 per token; zero memories = zero output; chunk length 1 by hand,
  * library routines: the gates at pre-activations on both sides of the +-10 clamp
    against torch's softplus, sigmoid and clamp,
  * invariants: causality, padding invariance, non-expansion of every chunk gain,
    query scale invariance, and the operator's rot180 / transpose symmetries,
  * planted mistakes (oracle `mutation` switch): each is caught by one of the above.
"""

import math

import numpy as np
import pytest

from tests.helpers import memories

ALPHA0 = 1.0 / (1.0 + math.exp(-2.197224577))  # retention at zero gate vectors, = 0.9


def _lines(seed, n, length, d, scale=1.0):
    rng = np.random.default_rng(seed)
    return rng.normal(size=(n, length, d)) * scale, rng.normal(size=(n, length, d))


def _run(oracle, x, q, mems, chunk, *, dtype=np.float64, q_raw=True, mutation=0, **kw):
    n = x.shape[0]
    s = mems[0].shape[0]
    return oracle.srnl_lines(x, q, mems, np.arange(n) % s, np.full(n, chunk), q_raw=q_raw,
                             dtype=dtype, mutation=mutation, **kw)


def _flat(mems):
    return tuple(m.reshape((-1,) + m.shape[2:]) for m in mems)


@pytest.mark.parametrize("d", [4, 8, 16, 32])
@pytest.mark.parametrize("kind", ["default", "perturbed", "strong"])
@pytest.mark.parametrize("length,chunk", [(1, 1), (9, 3), (23, 5), (64, 64), (70, 64)])
def test_c_oracle_matches_independent_numpy(oracle, d, kind, length, chunk):
    mems = _flat(memories(1, 2, d, kind=kind, seed=d))
    x, q = _lines(d + length, 2, length, d)
    ref = oracle.srnl_lines_numpy(x, q, mems, np.arange(2), np.full(2, chunk))
    y64 = _run(oracle, x, q, mems, chunk)
    y32 = _run(oracle, x, q, mems, chunk, dtype=np.float32)
    scale = np.abs(ref).max()
    assert np.abs(y64 - ref).max() <= 1e-12 * max(scale, 1.0)
    assert np.abs(y32 - ref).max() <= 2e-5 * scale


def test_normalized_query_input_is_used_as_given(oracle):
    mems = _flat(memories(1, 1, 8, kind="strong", seed=3))
    x, q = _lines(5, 1, 20, 8)
    qn = q / np.linalg.norm(q, axis=-1, keepdims=True)
    a = _run(oracle, x, qn, mems, 4, q_raw=False)
    b = _run(oracle, x, q, mems, 4, q_raw=True)
    np.testing.assert_allclose(a, b, rtol=1e-12, atol=1e-14)
    ref = oracle.srnl_lines_numpy(x, qn, mems, [0], [4], q_raw=False)
    np.testing.assert_allclose(a, ref, rtol=1e-10, atol=1e-14)


def test_first_chunk_is_plain_gemm(oracle):
    """Chunk 0 reads the initial content memory only: y_t = M_m q_hat_t for every gate setting."""
    d, chunk = 16, 10
    mems = _flat(memories(1, 1, d, kind="strong", seed=11))
    x, q = _lines(12, 1, 30, d, scale=3.0)
    y = _run(oracle, x, q, mems, chunk)
    q_hat = q[0, :chunk] / np.linalg.norm(q[0, :chunk], axis=-1, keepdims=True)
    np.testing.assert_allclose(y[0, :chunk], q_hat @ mems[0][0].T, rtol=1e-12, atol=1e-14)


@pytest.mark.parametrize("chunk", [1, 7, 14])
def test_zero_key_value_memories_decay(oracle, chunk):
    """M_k = M_v = 0 and zero gate vectors: k = v = 0, alpha = 0.9, so G = 0.9^C I and
    y_t = 0.9^(C * floor(t / C)) M_m q_hat_t."""
    d, length = 8, 3 * 14 + 5
    rng = np.random.default_rng(4)
    m_m = rng.normal(size=(1, d, d))
    zeros_m, zeros_v = np.zeros((1, d, d)), np.zeros((1, d))
    x, q = _lines(6, 1, length, d)
    y = _run(oracle, x, q, (m_m, zeros_m, zeros_m, zeros_v, zeros_v), chunk)
    t = np.arange(length)
    q_hat = q[0] / np.linalg.norm(q[0], axis=-1, keepdims=True)
    expected = (q_hat @ m_m[0].T) * (ALPHA0 ** (chunk * (t // chunk)))[:, None]
    np.testing.assert_allclose(y[0], expected, rtol=1e-9, atol=1e-15)


def test_zero_memories_give_zero_output(oracle):
    d = 16
    zeros = (np.zeros((1, d, d)),) * 3 + (np.zeros((1, d)),) * 2
    x, q = _lines(7, 2, 50, d)
    assert np.abs(_run(oracle, x, q, zeros, 14)).max() == 0.0


def _chunk_one_by_hand(m_m, m_v, m_k, x, q):
    """Two tokens, chunk length 1, zero gate vectors (alpha = 0.9, eta = 0.025 ln 2):
    G = alpha I - eta^ (2k - v) k^T after token 0; y_1 = (M_m G) q_hat_1."""
    d = x.shape[-1]
    kr = m_k @ x[0]
    k = kr / np.sqrt(kr @ kr + 1e-6)
    v = m_v @ x[0]
    alpha, eta = ALPHA0, 0.025 * math.log(2.0)
    dn = math.sqrt(((k - v) ** 2).sum() + 1e-12)
    cap = 0.999 * (1 - alpha) / (dn + 1e-6)
    eff = min(cap * -math.expm1(-eta / cap), 2 * 0.999999 * alpha / max(k @ k, 1e-20))
    gain = alpha * np.eye(d) - eff * np.outer(2 * k - v, k)
    q1 = q[1] / np.linalg.norm(q[1])
    return (m_m @ gain) @ q1


def _hand_case(d=4):
    rng = np.random.default_rng(8)
    m_m, m_v, m_k = (rng.normal(size=(d, d)) for _ in range(3))
    x = rng.normal(size=(2, d))
    q = rng.normal(size=(2, d))
    return m_m, m_v, m_k, x, q


def test_chunk_length_one_by_hand(oracle):
    m_m, m_v, m_k, x, q = _hand_case()
    d = x.shape[-1]
    zeros_v = np.zeros((1, d))
    y = _run(oracle, x[None], q[None], (m_m[None], m_v[None], m_k[None], zeros_v, zeros_v), 1)
    np.testing.assert_allclose(y[0, 1], _chunk_one_by_hand(m_m, m_v, m_k, x, q), rtol=1e-12)


@pytest.mark.parametrize("pre_e", [-12.0, -3.0, 0.0, 3.0, 12.0])
@pytest.mark.parametrize("pre_a", [-12.0, -3.0, 0.0, 3.0, 12.0])
@pytest.mark.parametrize("min_retention", [0.0, 0.3])
def test_gates_match_library_routines(oracle, pre_e, pre_a, min_retention):
    """The gates at non-zero gate vectors, pinned by library routines: chunk length 1,
    gate vectors chosen so that x.e = pre_e and x.a = pre_a (+-12 lies beyond the +-10
    pre-activation clamp).  The learning rate is step_scale * softplus(clamp(x.e)) with
    torch's softplus (beta 1, threshold 20) and the retention min_r + (1 - min_r) *
    sigmoid(clamp(x.a + bias)) with torch's sigmoid, both in float64; the first step's
    gain is then alpha I - eff (2k - v) k^T as in _chunk_one_by_hand."""
    import torch
    from oracle.oracle import Consts

    consts = Consts(min_retention=min_retention)
    m_m, m_v, m_k, x, q = _hand_case()
    d = x.shape[-1]
    e = pre_e * x[0] / (x[0] @ x[0])
    a = pre_a * x[0] / (x[0] @ x[0])
    y = _run(oracle, x[None], q[None], (m_m[None], m_v[None], m_k[None], e[None], a[None]), 1, consts=consts)

    f64 = torch.float64
    ep = torch.clamp(torch.tensor(pre_e, dtype=f64), -10.0, 10.0)
    ap = torch.clamp(torch.tensor(pre_a, dtype=f64) + consts.retention_bias, -10.0, 10.0)
    eta = consts.step_scale * torch.nn.functional.softplus(ep, beta=1.0, threshold=20.0)
    alpha = min_retention + (1.0 - min_retention) * torch.sigmoid(ap)
    kr = torch.from_numpy(m_k @ x[0])
    k = kr / torch.sqrt(kr @ kr + 1e-6)
    v = torch.from_numpy(m_v @ x[0])
    dn = torch.sqrt(((k - v) ** 2).sum() + 1e-12)
    cap = consts.injection_margin * (1 - alpha) / (dn + 1e-6)
    eff = cap * -torch.expm1(-eta / cap)
    lim = torch.nextafter(2 * consts.spectral_margin * alpha / torch.clamp_min(k @ k, 1e-20),
                          torch.tensor(0.0, dtype=f64))
    eff = torch.minimum(eff, lim)
    gain = alpha * torch.eye(d, dtype=f64) - eff * torch.outer(2 * k - v, k)
    q1 = torch.from_numpy(q[1] / np.linalg.norm(q[1]))
    want = (torch.from_numpy(m_m) @ gain @ q1).numpy()
    np.testing.assert_allclose(y[0, 1], want, rtol=1e-12, atol=1e-15)
    if abs(pre_a + consts.retention_bias) > 10:   # clamped: any larger pre-activation gives the same output
        a2 = 2 * a
        y2 = _run(oracle, x[None], q[None], (m_m[None], m_v[None], m_k[None], e[None], a2[None]), 1, consts=consts)
        np.testing.assert_array_equal(y2, y)


def test_causality(oracle):
    d, chunk, length = 8, 6, 40
    mems = _flat(memories(1, 1, d, kind="strong", seed=2))
    x, q = _lines(9, 1, length, d)
    base = _run(oracle, x, q, mems, chunk)
    # x in chunk c only influences outputs of later chunks
    c = 3
    x2 = x.copy()
    x2[0, c * chunk:] += 1.0
    y2 = _run(oracle, x2, q, mems, chunk)
    np.testing.assert_array_equal(y2[0, :(c + 1) * chunk], base[0, :(c + 1) * chunk])
    assert np.abs(y2[0, (c + 1) * chunk:] - base[0, (c + 1) * chunk:]).max() > 1e-6
    # q_s only influences y_s
    q2 = q.copy()
    q2[0, 17] *= -2.0
    y3 = _run(oracle, x, q2, mems, chunk)
    changed = np.nonzero(np.abs(y3[0] - base[0]).max(axis=-1))[0]
    assert changed.tolist() == [17]


def test_padding_invariance(oracle):
    """The final partial chunk is zero-padded: identical to explicit zero padding."""
    d, chunk, length = 8, 7, 31
    mems = _flat(memories(1, 1, d, kind="strong", seed=21))
    x, q = _lines(10, 1, length, d)
    y = _run(oracle, x, q, mems, chunk)
    pad = (-length) % chunk
    xp = np.concatenate([x, np.zeros((1, pad, d))], axis=1)
    qp = np.concatenate([q, np.ones((1, pad, d))], axis=1)
    yp = _run(oracle, xp, qp, mems, chunk)
    np.testing.assert_array_equal(yp[0, :length], y[0])


def test_every_chunk_gain_is_non_expansive(oracle):
    """Spectral clamp gives |A_t| <= alpha_t, the soft cap |B_t| < mu (1 - alpha_t),
    so every chunk gain has spectral norm <= 1 (README's stability claim)."""
    d, chunk = 16, 16
    mems = _flat(memories(1, 4, d, kind="strong", seed=31))
    x, q = _lines(11, 4, 8 * chunk, d, scale=4.0)
    _, gains = _run(oracle, x, q, mems, chunk, want_gains=True)
    norms = np.linalg.norm(gains.reshape(-1, d, d), ord=2, axis=(1, 2))
    assert norms.max() <= 1.0 + 1e-9
    assert norms.min() < 0.999  # the clamp is actually exercised, not vacuous


def test_query_scale_invariance(oracle):
    d = 8
    mems = _flat(memories(1, 1, d, kind="strong", seed=41))
    x, q = _lines(12, 1, 33, d)
    a = _run(oracle, x, q, mems, 5)
    b = _run(oracle, x, q * np.linspace(0.01, 100, 33)[None, :, None], mems, 5)
    np.testing.assert_allclose(a, b, rtol=1e-11, atol=1e-14)


def test_long_scan_fp32_matches_fp64(oracle):
    """Base-512 stage-1 scan length (128 chunks of 128 tokens): the fp32 restatement stays
    within the 1e-4 parity budget of the fp64 one."""
    d, chunk = 16, 128
    mems = _flat(memories(1, 2, d, kind="perturbed", seed=51))
    x, q = _lines(13, 2, 128 * chunk, d)
    y64 = _run(oracle, x, q, mems, chunk)
    y32 = _run(oracle, x, q, mems, chunk, dtype=np.float32)
    rel = np.linalg.norm(y32 - y64) / np.linalg.norm(y64)
    assert rel < 1e-5, rel


# ---------------------------------------------------------------------------------
# four-direction operator symmetries (pin restore_index and the chunk assignment)
# ---------------------------------------------------------------------------------

def _operator_case(height, width, heads=2, d=8, seed=5):
    rng = np.random.default_rng(seed)
    c = heads * d
    x = rng.normal(size=(2, height, width, c))
    q = rng.normal(size=(2, height, width, c))
    mems = memories(4, heads, d, kind="strong", seed=seed)
    skip = rng.normal(size=(4, c)) * 0.3
    w = 1 + rng.normal(size=(4, c)) * 0.3
    return x, q, mems, skip, w, d


def _swap(mems, skip, w, perm):
    return tuple(m[perm] for m in mems), skip[perm], w[perm]


def test_operator_rot180_symmetry(oracle):
    x, q, mems, skip, w, d = _operator_case(5, 7)
    out = oracle.operator_forward(x, q, mems, skip, w, d, dtype=np.float64)
    mems2, skip2, w2 = _swap(mems, skip, w, [1, 0, 3, 2])
    rot = lambda a: a[:, ::-1, ::-1]
    out2 = oracle.operator_forward(rot(x), rot(q), mems2, skip2, w2, d, dtype=np.float64)
    np.testing.assert_allclose(out2, rot(out), rtol=1e-11, atol=1e-13)


def test_operator_transpose_symmetry(oracle):
    x, q, mems, skip, w, d = _operator_case(6, 6)
    out = oracle.operator_forward(x, q, mems, skip, w, d, dtype=np.float64)
    mems2, skip2, w2 = _swap(mems, skip, w, [2, 3, 0, 1])
    tr = lambda a: a.transpose(0, 2, 1, 3)
    out2 = oracle.operator_forward(tr(x), tr(q), mems2, skip2, w2, d, dtype=np.float64)
    np.testing.assert_allclose(out2, tr(out), rtol=1e-11, atol=1e-13)


def test_operator_first_chunks_closed_form(oracle):
    """Row 0 is chunk 0 of scan 0, row H-1 chunk 0 of scan 1, column 0 chunk 0 of scan 2,
    column W-1 chunk 0 of scan 3: pixel (0, 0) reads M_m of scans 0 and 2 (first chunk)."""
    x, q, mems, skip, w, d = _operator_case(4, 5)
    out = oracle.operator_forward(x, q, mems, skip, w, d, dtype=np.float64)
    heads = x.shape[-1] // d
    qh = q[0, 0, 0].reshape(heads, d)
    qh = qh / np.linalg.norm(qh, axis=-1, keepdims=True)
    y0 = np.concatenate([mems[0][0, h] @ qh[h] for h in range(heads)])
    y2 = np.concatenate([mems[0][2, h] @ qh[h] for h in range(heads)])
    xv = x[0, 0, 0]
    partial = w[0] * (y0 + skip[0] * xv) + w[2] * (y2 + skip[2] * xv)
    # scans 1 and 3 reach pixel (0, 0) in their last chunk; subtract the full output's
    # dependence by recomputing with those directions' weights zeroed
    w_only02 = w.copy()
    w_only02[[1, 3]] = 0
    out02 = oracle.operator_forward(x, q, mems, skip, w_only02, d, dtype=np.float64)
    np.testing.assert_allclose(out02[0, 0, 0], partial, rtol=1e-11, atol=1e-13)
    assert not np.allclose(out[0, 0, 0], partial)


# ---------------------------------------------------------------------------------
# planted mistakes are caught
# ---------------------------------------------------------------------------------

def test_mutation_transposed_refresh_is_caught(oracle):
    m_m, m_v, m_k, x, q = _hand_case()
    d = x.shape[-1]
    zeros_v = np.zeros((1, d))
    y = _run(oracle, x[None], q[None], (m_m[None], m_v[None], m_k[None], zeros_v, zeros_v), 1,
             mutation=1)
    assert not np.allclose(y[0, 1], _chunk_one_by_hand(m_m, m_v, m_k, x, q), rtol=1e-6)


def test_mutation_dropped_difference_term_is_caught(oracle):
    m_m, m_v, m_k, x, q = _hand_case()
    d = x.shape[-1]
    zeros_v = np.zeros((1, d))
    y = _run(oracle, x[None], q[None], (m_m[None], m_v[None], m_k[None], zeros_v, zeros_v), 1,
             mutation=2)
    assert not np.allclose(y[0, 1], _chunk_one_by_hand(m_m, m_v, m_k, x, q), rtol=1e-6)


def test_mutation_wrong_sign_is_caught(oracle):
    m_m, m_v, m_k, x, q = _hand_case()
    d = x.shape[-1]
    zeros_v = np.zeros((1, d))
    y = _run(oracle, x[None], q[None], (m_m[None], m_v[None], m_k[None], zeros_v, zeros_v), 1,
             mutation=3)
    assert not np.allclose(y[0, 1], _chunk_one_by_hand(m_m, m_v, m_k, x, q), rtol=1e-6)
    mems = _flat(memories(1, 2, 16, kind="strong", seed=31))
    xs, qs = _lines(11, 2, 64, 16)
    ref = oracle.srnl_lines_numpy(xs, qs, mems, np.arange(2), np.full(2, 16))
    assert not np.allclose(_run(oracle, xs, qs, mems, 16, mutation=3), ref, rtol=1e-6)


def test_mutation_unnormalised_query_is_caught(oracle):
    d = 8
    mems = _flat(memories(1, 1, d, kind="strong", seed=41))
    x, q = _lines(12, 1, 33, d)
    a = _run(oracle, x, q, mems, 5, mutation=4)
    b = _run(oracle, x, q * 3.0, mems, 5, mutation=4)
    assert not np.allclose(a, b, rtol=1e-6)
