"""The block (UT) form of the SRNL gain recurrence, as the head_dim-16 scan kernel evaluates
it, checked in float64 against the token-by-token update of the reference
(``models/srnl_core/csrc/inference_recurrence.cuh:92-106``):

    G <- alpha_t G - eta^_t (G k_t + k_t - v_t) k_t^T        (one token at a time)

The kernel cuts a chunk into blocks of 16 token slots (slots past the chunk are the
identity: alpha = 1, eta^ = 0, k = v = 0) and forms, per block, with a_t the block-local
prefix product of alpha:

    L[s][t] = eta^_s (a_{t-1} / a_s) (k_s . k_t)    (s < t),  Z = (I + L)^-1 W K^T,
    W = diag(eta^_s a_15 / a_s),  X_b = a_15 I - K D_a Z,  Y_b = -Delta Z,
    G_{b+1} = G_b X_b + Y_b,

with the ratios built exactly as the kernel builds them: cl = inclusive prefix sum of
log2 alpha, clx = cl - log2 alpha, rho_s = eta^_s 2^(m - cl_s), kappa_t = 2^(clx_t - m)
about the midpoint m = cl_15 / 2, so L = diag(rho) K^T K diag(kappa), -a_{t-1} = -2^clx_t
and w_s = eta^_s 2^(cl_15 - cl_s).  The checks run at chunks 7, 14, 28 and 56 (the Tiny
row lengths: one, one, two and four blocks, ragged last blocks), with retention factors
spread over the whole gate range sigma(-10) .. sigma(10), and a planted mistake (a_t in
place of a_{t-1}) must fail them.
"""

import numpy as np
import pytest

BLOCK = 16
ALPHA_LO, ALPHA_HI = 1.0 / (1.0 + np.exp(10.0)), 1.0 / (1.0 + np.exp(-10.0))


def _tokens(rng, count, d=16):
    """Keys of norm below 1, values, retention factors over sigma(-10)..sigma(10) (log-spaced
    in 1 - alpha and in alpha, so both ends are hit), step sizes up to the spectral bound."""
    k = rng.standard_normal((count, d))
    k *= (rng.uniform(0.2, 0.999, count) / np.linalg.norm(k, axis=1))[:, None]
    v = rng.standard_normal((count, d)) * 0.5
    pick = rng.integers(0, 3, count)
    alpha = np.where(pick == 0, np.exp(rng.uniform(np.log(ALPHA_LO), np.log(0.5), count)),
                     np.where(pick == 1, 1.0 - np.exp(rng.uniform(np.log(1.0 - ALPHA_HI), np.log(0.5), count)),
                              rng.uniform(0.5, 0.95, count)))
    alpha[:2] = (ALPHA_LO, ALPHA_HI)[:count]
    eta = rng.uniform(0.0, 1.0, count) * 2.0 * alpha / np.sum(k * k, axis=1)
    return k, v, alpha, eta


def _serial(G, k, v, alpha, eta, with_delta=True):
    """Token-by-token gain update (inference_recurrence.cuh:92-106), columns of G as rows here
    follow the reference: G[i][j], r = G k + (k - v), G <- alpha G - eta r k^T."""
    G = G.copy()
    for t in range(len(alpha)):
        r = G @ k[t] + ((k[t] - v[t]) if with_delta else 0.0)
        G = alpha[t] * G - eta[t] * np.outer(r, k[t])
    return G


def _pad(k, v, alpha, eta):
    n = len(alpha)
    pad = (-n) % BLOCK
    if pad:
        d = k.shape[1]
        k = np.vstack([k, np.zeros((pad, d))])
        v = np.vstack([v, np.zeros((pad, d))])
        alpha = np.concatenate([alpha, np.ones(pad)])
        eta = np.concatenate([eta, np.zeros(pad)])
    return k, v, alpha, eta


def _block_maps(k, v, alpha, eta, *, planted=False):
    """X_b, Y_b, Z and L of one 16-slot block, built the way the kernel builds them."""
    la = np.log2(alpha)
    cl = np.cumsum(la)
    clx = cl - la if not planted else cl          # planted mistake: a_t instead of a_{t-1}
    tot = cl[-1]
    mid = 0.5 * tot
    rho = eta * np.exp2(mid - cl)
    kappa = np.exp2(clx - mid)
    neg_a_prev = -np.exp2(clx)
    w = eta * np.exp2(tot - cl)
    gram = k @ k.T
    L = np.triu(rho[:, None] * gram * kappa[None, :], 1)
    Z = np.linalg.solve(np.eye(BLOCK) + L, w[:, None] * k)          # 16 slots x d features
    K = k.T                                                           # d x 16
    delta = (k - v).T
    X = np.exp2(tot) * np.eye(k.shape[1]) + (K * neg_a_prev[None, :]) @ Z
    Y = -delta @ Z
    return X, Y, Z, L


def _back_substitution(L, rhs):
    """Z = (I + L)^-1 rhs for strictly upper L, last row first, as the kernel's lanes solve
    it (Z[s] = rhs[s] - sum_{v > s} L[s][v] Z[v])."""
    Z = np.zeros_like(rhs)
    for s in range(BLOCK - 1, -1, -1):
        Z[s] = rhs[s] - L[s, s + 1:] @ Z[s + 1:]
    return Z


def _chunk_gain(k, v, alpha, eta, *, planted=False):
    k, v, alpha, eta = _pad(k, v, alpha, eta)
    G = np.eye(k.shape[1])
    for b0 in range(0, len(alpha), BLOCK):
        sl = slice(b0, b0 + BLOCK)
        X, Y, _, _ = _block_maps(k[sl], v[sl], alpha[sl], eta[sl], planted=planted)
        G = G @ X + Y
    return G


@pytest.mark.parametrize("chunk", [7, 14, 28, 56, 16, 33])
@pytest.mark.parametrize("seed", [0, 1, 2])
def test_chunk_gain_matches_token_by_token(chunk, seed):
    rng = np.random.default_rng(100 * chunk + seed)
    k, v, alpha, eta = _tokens(rng, chunk)
    want = _serial(np.eye(16), k, v, alpha, eta)
    got = _chunk_gain(k, v, alpha, eta)
    assert np.abs(got - want).max() <= 1e-12 * max(1.0, np.abs(want).max())


@pytest.mark.parametrize("count", [16, 9, 1])
def test_block_maps_match_serial_linear_and_affine_parts(count):
    """X_b is the serial map of the block from G = I without the (k - v) term; Y_b is the
    serial map from G = 0 with it; ragged blocks are padded with identity slots."""
    rng = np.random.default_rng(7 + count)
    k, v, alpha, eta = _pad(*_tokens(rng, count))
    X, Y, Z, L = _block_maps(k, v, alpha, eta)
    assert np.allclose(X, _serial(np.eye(16), k, v, alpha, eta, with_delta=False), rtol=0, atol=1e-13)
    assert np.allclose(Y, _serial(np.zeros((16, 16)), k, v, alpha, eta), rtol=0, atol=1e-13)
    # the kernel's back substitution gives the same Z as the dense solve
    a_ratio = np.exp2(np.cumsum(np.log2(alpha))[-1] - np.cumsum(np.log2(alpha)))
    assert np.allclose(_back_substitution(L, (eta * a_ratio)[:, None] * k), Z, rtol=0, atol=1e-13)


def test_correction_vectors_satisfy_the_triangular_system():
    """R (I + L) = G_b K D_a + Delta for the serial correction vectors r_t = G_{t-1} k_t +
    delta_t from an arbitrary entry gain G_b, and G_{b+1} = a_15 G_b - R W K^T."""
    rng = np.random.default_rng(11)
    k, v, alpha, eta = _pad(*_tokens(rng, 13))
    Gb = rng.standard_normal((16, 16)) * 0.3
    G = Gb.copy()
    R = np.zeros((16, BLOCK))
    for t in range(BLOCK):
        R[:, t] = G @ k[t] + (k[t] - v[t])
        G = alpha[t] * G - eta[t] * np.outer(R[:, t], k[t])
    _, _, _, L = _block_maps(k, v, alpha, eta)
    a = np.cumprod(alpha)
    a_prev = np.concatenate([[1.0], a[:-1]])
    lhs = R @ (np.eye(BLOCK) + L)
    rhs = Gb @ (k.T * a_prev[None, :]) + (k - v).T
    assert np.allclose(lhs, rhs, rtol=0, atol=1e-12)
    w = eta * a[-1] / a
    assert np.allclose(G, a[-1] * Gb - (R * w[None, :]) @ k, rtol=0, atol=1e-12)
    X, Y, _, _ = _block_maps(k, v, alpha, eta)
    assert np.allclose(G, Gb @ X + Y, rtol=0, atol=1e-12)


def test_ratio_factors_stay_finite_at_the_gate_extremes():
    """Sixteen slots at sigma(-10): a_15 = sigma(-10)^16 ~ 1e-69 underflows FP32, but the
    kernel only ever forms the split factors rho and kappa (exponents within |cl_15| / 2)
    and ratios <= 1, all finite in FP32."""
    alpha = np.full(BLOCK, ALPHA_LO)
    la = np.log2(alpha).astype(np.float32)
    cl = np.cumsum(la, dtype=np.float32)
    clx, mid = cl - la, np.float32(0.5) * cl[-1]
    with np.errstate(over="raise", under="ignore"):
        rho = np.exp2(mid - cl)
        kappa = np.exp2(clx - mid)
    assert np.isfinite(rho).all() and np.isfinite(kappa).all()
    # only s < t is used (the lower triangle, where the product may overflow, is masked
    # out by a select in the kernel); there a_{t-1} / a_s <= 1 up to FP32 rounding
    s_idx, t_idx = np.triu_indices(BLOCK, 1)
    ratio = rho[s_idx] * kappa[t_idx]
    assert np.isfinite(ratio).all() and (ratio <= 1.0 + 1e-5).all()


def test_planted_index_mistake_is_caught():
    rng = np.random.default_rng(3)
    k, v, _, _ = _tokens(rng, 14)
    alpha = rng.uniform(0.6, 0.95, 14)   # gains far from zero, so the mistake shows
    eta = rng.uniform(0.2, 1.0, 14) * 2.0 * alpha / np.sum(k * k, axis=1)
    want = _serial(np.eye(16), k, v, alpha, eta)
    wrong = _chunk_gain(k, v, alpha, eta, planted=True)
    assert np.abs(wrong - want).max() > 1e-3 * np.abs(want).max()
