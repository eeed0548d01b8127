"""Differentiable CPU oracle of the SRNL recurrence — TEST INFRASTRUCTURE ONLY.

Only ``tests/`` may import this module, as the checker of the backward kernels: the
gradients of this float64 PyTorch restatement (autograd) are what the HIP backward is
compared against.  Nothing in ``visionhope_amd`` imports it.

``srnl_lines_torch`` restates the training forward of the reference (the math spec of
``models/srnl_core/csrc/chunk.cu:252-509`` with ``memory.cuh:219-233``) with the
subgradient conventions of its backward (``chunk.cu:511-1057``, ``memory.cuh:253-352``):

* the pre-activation clamps pass the gradient when ``|pre| <= 10`` (``chunk.cu:394-395``);
* the spectral clamp ``min(eta_eff, nextafter(F alpha / max(||k||^2, 1e-20), 0))`` takes
  the limit only when ``eta_eff`` exceeds it, and its gradient flows to alpha and, when
  ``||k||^2 > 1e-20``, to ``||k||^2`` (``memory.cuh:333-344``); nextafter's one-ulp step is
  treated as the identity;
* the query normalisation ``q / max(||q||, 1e-12)`` drops the projection term below the
  epsilon (``chunk.cu:1042-1043``).

The operator tail (``direction_fusion_torch``, ``grn_torch``, ``layernorm2d_torch``,
``qnorm_torch``, ``residual_add_torch``) restates the forwards of
``utils/csrc/direction_fusion.cu:11-65``, ``utils/grn.py:26-38``, ``models/layers.py:25-35``,
``utils/csrc/query_normalization.cu:10-40`` and ``utils/residual.py:31-52``; their
gradients are the checker of the tail backward kernels.

Pinning (``tests/test_oracle_backward.py``): every forward equals the C oracle and/or the
NumPy formulation of ``oracle.py`` on the same inputs, and ``torch.autograd.gradcheck``
checks every gradient against central finite differences in float64.
"""

from __future__ import annotations

import torch

from .oracle import Consts, restore_index


def _line(x, q, mm, mv, mk, ev, av, c_len, q_raw, k):
    """One line: x, q ``[L, d]`` float64 tensors, state ``mm, mv, mk [d, d]``, ``ev, av [d]``."""
    length, d = x.shape
    n_chunks = -(-length // c_len)
    pad = n_chunks * c_len - length
    if pad:
        x = torch.cat([x, x.new_zeros(pad, d)])
        q = torch.cat([q, x.new_ones(pad, d)])
    eye = torch.eye(d, dtype=x.dtype)
    outs = []
    for c in range(n_chunks):
        xc = x[c * c_len:(c + 1) * c_len]
        qc = q[c * c_len:(c + 1) * c_len]
        if q_raw:
            qc = qc / torch.clamp_min(qc.norm(dim=1, keepdim=True), 1e-12)
        outs.append(qc @ mm.T)
        if c == n_chunks - 1:
            break
        kraw = xc @ mk.T
        vals = xc @ mv.T
        keys = kraw / torch.sqrt((kraw * kraw).sum(1, keepdim=True) + 1e-6)
        ep = torch.clamp(xc @ ev, -10.0, 10.0)
        ap = torch.clamp(xc @ av + k.retention_bias, -10.0, 10.0)
        eta = k.step_scale * torch.where(ep > 20, ep, torch.log1p(torch.exp(ep)))
        alpha = k.min_retention + (1 - k.min_retention) * torch.sigmoid(ap)
        dn = torch.sqrt(((keys - vals) ** 2).sum(1) + 1e-12)
        cap = k.injection_margin * (1 - alpha) / (dn + 1e-6)
        eff = -cap * torch.expm1(-eta / cap)
        if k.spectral_clamp:
            lim = 2 * k.spectral_margin * alpha / torch.clamp_min((keys * keys).sum(1), 1e-20)
            lim = lim + (torch.nextafter(lim, torch.zeros_like(lim)) - lim).detach()
            eff = torch.where(eff > lim, lim, eff)
        gain = eye
        for t in range(c_len):
            kt = keys[t]
            r = gain @ kt + (kt - vals[t])
            gain = alpha[t] * gain - eff[t] * torch.outer(r, kt)
        mm, mv, mk = mm @ gain, mv @ gain, mk @ gain
        ev, av = gain.T @ ev, gain.T @ av
    return torch.cat(outs)[:length]


def srnl_lines_torch(x, q, memories, state_index, chunks, *, q_raw=True, consts=None):
    """Differentiable float64 SRNL over independent lines.

    x, q: ``[n_lines, L, d]`` tensors; memories ``(M_m, M_v, M_k, M_eta, M_alpha)`` with
    shapes ``[S, d, d]`` x3 and ``[S, d]`` x2, shared by the lines whose ``state_index``
    selects them; ``chunks[n]`` the chunk length of line n.  Returns y ``[n_lines, L, d]``.
    """
    k = consts or Consts.from_env()
    mm, mv, mk, me, ma = memories
    ys = [_line(x[n], q[n], mm[s], mv[s], mk[s], me[s], ma[s], int(chunks[n]), q_raw, k)
          for n, s in enumerate(int(v) for v in state_index)]
    return torch.stack(ys)


def sequence_forward_torch(x_packed, q, memories, chunks, *, q_raw=True, consts=None):
    """Packed layout of ``oracle.sequence_forward``: x ``[B,R,heads,N,d]``; q raw ``[B,R,N,C]``
    or normalized ``[B,R,heads,N,d]``; memories ``[R,heads,d,d]`` / ``[R,heads,d]``."""
    b, r, heads, length, d = x_packed.shape
    if q_raw:
        q_lines = q.reshape(b, r, length, heads, d).permute(0, 1, 3, 2, 4).reshape(b * r * heads, length, d)
    else:
        q_lines = q.reshape(b * r * heads, length, d)
    n_lines = b * r * heads
    mems = [m.reshape((r * heads,) + tuple(m.shape[2:])) for m in memories]
    line_r = [(n // heads) % r for n in range(n_lines)]
    y = srnl_lines_torch(x_packed.reshape(n_lines, length, d), q_lines, mems,
                         [n % (r * heads) for n in range(n_lines)], [chunks[lr] for lr in line_r],
                         q_raw=q_raw, consts=consts)
    return y.reshape(b, r, heads, length, d)


def direction_fusion_torch(y, x, d_skip, scale, height, width):
    """``out[b, c, pixel] = sum_r scale[r, c] (y_r + skip_r[c] x_r)[t_r(pixel)]``, NCHW.

    y, x ``[B, 4, heads, L, d]``; d_skip ``[heads, d]`` or ``[4, heads, d]``; scale ``[4, C]``.
    """
    b, _, heads, length, d = y.shape
    c = heads * d
    skip = d_skip.reshape(-1, c)
    out = 0
    for r in range(4):
        k = skip[r if skip.shape[0] == 4 else 0].reshape(heads, 1, d)
        seq = (y[:, r] + k * x[:, r]).permute(0, 2, 1, 3).reshape(b, length, c)
        idx = torch.as_tensor(restore_index(r, height, width), dtype=torch.long)
        # restored[:, idx[t]] = seq[:, t]  <=>  restored = seq[:, inverse(idx)]
        inv = torch.empty_like(idx)
        inv[idx] = torch.arange(length)
        out = out + scale[r] * seq[:, inv]
    return out.reshape(b, height, width, c).permute(0, 3, 1, 2)


def grn_torch(x, gamma, beta, eps=1e-6):
    """``x (1 + gamma nx) + beta``, nx = ||x_c|| / (mean_c ||x_c|| + eps), NCHW."""
    c = x.shape[1]
    gx = torch.linalg.vector_norm(x, dim=(2, 3), keepdim=True)   # subgradient 0 at a zero channel
    nx = gx / (gx.mean(dim=1, keepdim=True) + eps)
    return x * (1 + gamma.reshape(1, c, 1, 1) * nx) + beta.reshape(1, c, 1, 1)


def layernorm2d_torch(x, weight, bias, eps=1e-6):
    """LayerNorm over channels per pixel, biased variance, NCHW."""
    c = x.shape[1]
    mean = x.mean(dim=1, keepdim=True)
    var = ((x - mean) ** 2).mean(dim=1, keepdim=True)
    return (x - mean) / torch.sqrt(var + eps) * weight.reshape(1, c, 1, 1) + bias.reshape(1, c, 1, 1)


def qnorm_torch(q_raw, heads, head_dim):
    """``[B, R, N, heads d]`` -> ``q / max(|q|, 1e-12)`` as ``[B, R, heads, N, d]``."""
    b, r, length, _ = q_raw.shape
    q = q_raw.reshape(b, r, length, heads, head_dim).permute(0, 1, 3, 2, 4)
    return q / torch.clamp_min(q.norm(dim=-1, keepdim=True), 1e-12)


def residual_add_torch(residual, branch, gamma, drop_scale):
    """``residual + branch gamma_c drop_scale_b`` on NCHW tensors."""
    c = branch.shape[1]
    return residual + branch * gamma.reshape(1, c, 1, 1) * drop_scale.reshape(-1, 1, 1, 1)
