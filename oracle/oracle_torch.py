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

Pinning (``tests/test_oracle_backward.py``): the forward equals the C oracle and the
independent NumPy formulation of ``oracle.py`` on the same inputs, and
``torch.autograd.gradcheck`` checks every gradient against central finite differences in
float64.
"""

from __future__ import annotations

import torch

from .oracle import Consts


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
