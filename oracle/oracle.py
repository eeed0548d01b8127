"""CPU oracle for the VisionHOPE SRNL hot path — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import this module, and only as the checker (or as the timed CPU
baseline).  Nothing in ``visionhope_amd`` imports it: the product path has no
CPU fallback.

Contents and the reference code each function restates:

* ``srnl_lines`` — ctypes front end of ``liboracle_srnl.so`` (C, fp32/fp64),
  the SRNL recurrence of ``models/srnl_core/csrc/inference_recurrence.cuh:3-137``
  and ``memory.cuh:219-233``.
* ``srnl_lines_numpy`` — an independent fp64 NumPy formulation of the same
  recurrence (chunk-level matrix algebra instead of per-thread loops), used to
  cross-check the C code on small inputs.
* ``restore_index`` / ``serialize`` — the four scan orders of
  ``models/operator.py:79-86`` and the restoration of
  ``models/srnl_core/csrc/parallel_line.cuh:16-23``.
* ``operator_forward`` — four scans + restoration + weighted fusion, the fast
  spatial path ``operator.py:159-193`` / ``fused.cu:307-351``.
* ``sequence_forward`` — packed sequence inference ``fused.cu:63-179``.
* ``direction_fusion`` — ``utils/csrc/direction_fusion.cu:11-65`` (and the
  PyTorch fallback ``operator.py:121-139``).
* ``grn`` — ``utils/grn.py:26-38``.  ``layernorm2d`` — ``models/layers.py:25-35``
  and ``utils/layer_norm_cuda.py:44-57``.  ``qnorm`` —
  ``utils/csrc/query_normalization.cu:135-177``.  ``residual_add`` —
  ``utils/residual.py:31-52``.

Pinning: ``tests/test_oracle_srnl.py`` and ``tests/test_oracle_elementwise.py``
check every function here against closed forms, invariants, the independent
formulation, textbook routines and planted mistakes.  The reference ships no
golden vectors and cannot be run here (CUDA-only, needs ``timm``), so no
reference-produced fixture exists.
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from dataclasses import dataclass
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
_LIB_PATH = _HERE / "liboracle_srnl.so"
_LIB = None


def _env_float(name, default):
    raw = os.environ.get(name)
    return float(default) if raw is None else float(raw)


@dataclass(frozen=True)
class Consts:
    """Stability constants; defaults and env names from ``models/srnl_core/chunk.py:44-49``."""

    step_scale: float = 0.025
    min_retention: float = 0.0
    retention_bias: float = 2.197224577
    injection_margin: float = 0.999
    spectral_clamp: int = 1
    spectral_margin: float = 0.999999

    @classmethod
    def from_env(cls):
        return cls(
            step_scale=_env_float("VISIONHOPE_STEP_SCALE", 0.025),
            min_retention=_env_float("VISIONHOPE_MIN_RETENTION", 0.0),
            retention_bias=_env_float("VISIONHOPE_RETENTION_BIAS", 2.197224577),
            injection_margin=_env_float("VISIONHOPE_INJECTION_MARGIN", 0.999),
            spectral_clamp=1,
            spectral_margin=_env_float("VISIONHOPE_SPECTRAL_MARGIN", 0.999999),
        )


class _CConsts(ctypes.Structure):
    _fields_ = [
        ("step_scale", ctypes.c_double),
        ("min_retention", ctypes.c_double),
        ("retention_bias", ctypes.c_double),
        ("injection_margin", ctypes.c_double),
        ("spectral_clamp", ctypes.c_int),
        ("spectral_margin", ctypes.c_double),
    ]


def build():
    """Compile ``liboracle_srnl.so`` with the committed Makefile."""
    subprocess.run(["make", "-s", "-C", str(_HERE)], check=True)


def _lib():
    global _LIB
    if _LIB is None:
        if not _LIB_PATH.exists():
            build()
        lib = ctypes.CDLL(str(_LIB_PATH))
        for suffix in ("f32", "f64"):
            fn = getattr(lib, f"oracle_srnl_lines_{suffix}")
            fn.restype = None
            fn.argtypes = [ctypes.c_void_p] * 2 + [ctypes.c_int] + [ctypes.c_void_p] * 7 + [
                ctypes.c_int64, ctypes.c_int64, ctypes.c_int, ctypes.POINTER(_CConsts), ctypes.c_int,
                ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64]
        _LIB = lib
    return _LIB


def _ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def srnl_lines(x, q, memories, state_index, chunks, *, q_raw=True, dtype=np.float32,
               consts=None, mutation=0, want_final=False, want_gains=False):
    """Run the C oracle over independent lines.

    x, q: ``[n_lines, L, d]``; memories: ``(M_m, M_v, M_k, M_eta, M_alpha)`` with
    shapes ``[S, d, d]`` x3 and ``[S, d]`` x2; ``state_index[n]`` selects the
    memory set of line n (``chunk.cu:287``: ``state_pid = pid % StateCount``);
    ``chunks[n]`` is its chunk length.  Returns y ``[n_lines, L, d]`` (and the
    final states / per-chunk gains when asked).
    """
    consts = consts or Consts.from_env()
    x = np.ascontiguousarray(x, dtype=dtype)
    q = np.ascontiguousarray(q, dtype=dtype)
    n_lines, length, d = x.shape
    if q.shape != x.shape:
        raise ValueError("x and q must have the same [n_lines, L, d] shape")
    mm, mv, mk, me, ma = (np.ascontiguousarray(m, dtype=dtype) for m in memories)
    state_index = np.ascontiguousarray(state_index, dtype=np.int64)
    chunks = np.ascontiguousarray(chunks, dtype=np.int32)
    if state_index.shape != (n_lines,) or chunks.shape != (n_lines,):
        raise ValueError("state_index and chunks need one entry per line")
    if chunks.min() <= 0:
        raise ValueError("chunk lengths must be positive")
    y = np.zeros_like(x)
    final = np.zeros((n_lines, 3 * d * d + 2 * d), dtype=dtype) if want_final else None
    gpl = int(max((length + c - 1) // c for c in chunks)) if want_gains else 0
    gains = np.zeros((n_lines, gpl, d, d), dtype=dtype) if want_gains else None
    cc = _CConsts(consts.step_scale, consts.min_retention, consts.retention_bias,
                  consts.injection_margin, int(consts.spectral_clamp), consts.spectral_margin)
    fn = _lib().oracle_srnl_lines_f32 if dtype == np.float32 else _lib().oracle_srnl_lines_f64
    fn(_ptr(x), _ptr(q), int(bool(q_raw)), _ptr(mm), _ptr(mv), _ptr(mk), _ptr(me), _ptr(ma),
       _ptr(state_index), _ptr(chunks), n_lines, length, d, ctypes.byref(cc), int(mutation),
       _ptr(y), _ptr(final) if final is not None else None,
       _ptr(gains) if gains is not None else None, gpl)
    out = [y]
    if want_final:
        out.append(final)
    if want_gains:
        out.append(gains)
    return out[0] if len(out) == 1 else tuple(out)


def srnl_lines_numpy(x, q, memories, state_index, chunks, *, q_raw=True, consts=None):
    """Independent fp64 formulation: chunk-level matrix algebra, no shared code with the C file."""
    consts = consts or Consts.from_env()
    x = np.asarray(x, dtype=np.float64)
    q = np.asarray(q, dtype=np.float64)
    n_lines, length, d = x.shape
    mems = [np.asarray(m, dtype=np.float64) for m in memories]
    y = np.zeros_like(x)
    for n in range(n_lines):
        s = int(state_index[n])
        c_len = int(chunks[n])
        mm, mv, mk = (mems[i][s].copy() for i in range(3))
        ev, av = mems[3][s].copy(), mems[4][s].copy()
        n_chunks = -(-length // c_len)
        pad = n_chunks * c_len - length
        xp = np.concatenate([x[n], np.zeros((pad, d))])
        qp = np.concatenate([q[n], np.ones((pad, d))])
        for c in range(n_chunks):
            xc = xp[c * c_len:(c + 1) * c_len]
            qc = qp[c * c_len:(c + 1) * c_len]
            if q_raw:
                qc = qc / np.maximum(np.linalg.norm(qc, axis=1, keepdims=True), 1e-12)
            yc = qc @ mm.T
            keep = min(c_len, length - c * c_len)
            y[n, c * c_len:c * c_len + keep] = yc[:keep]
            kraw = xc @ mk.T
            vals = xc @ mv.T
            keys = kraw / np.sqrt((kraw ** 2).sum(1, keepdims=True) + 1e-6)
            ep = np.clip(xc @ ev, -10, 10)
            ap = np.clip(xc @ av + consts.retention_bias, -10, 10)
            eta = consts.step_scale * np.where(ep > 20, ep, np.log1p(np.exp(ep)))
            alpha = consts.min_retention + (1 - consts.min_retention) / (1 + np.exp(-ap))
            dn = np.sqrt(((keys - vals) ** 2).sum(1) + 1e-12)
            cap = consts.injection_margin * (1 - alpha) / (dn + 1e-6)
            eff = -cap * np.expm1(-eta / cap)
            if consts.spectral_clamp:
                lim = 2 * consts.spectral_margin * alpha / np.maximum((keys ** 2).sum(1), 1e-20)
                eff = np.minimum(eff, lim)
            gain = np.eye(d)
            for t in range(c_len):
                k = keys[t]
                # G <- G (alpha I - eta k k^T) - eta (k - v) k^T
                gain = gain @ (alpha[t] * np.eye(d) - eff[t] * np.outer(k, k)) \
                    - eff[t] * np.outer(k - vals[t], k)
            mm, mv, mk = mm @ gain, mv @ gain, mk @ gain
            ev, av = gain.T @ ev, gain.T @ av
    return y


# --------------------------------------------------------------------------------------
# Four-direction spatial operator
# --------------------------------------------------------------------------------------

def restore_index(direction, height, width):
    """Spatial position (h*W + w) of serialized token t, for every t (parallel_line.cuh:16-23)."""
    length = height * width
    t = np.arange(length)
    orig = length - 1 - t if direction & 1 else t
    if direction < 2:
        return orig
    return (orig % height) * width + orig // height


def serialize(x_nhwc):
    """[B,H,W,C] -> [B,4,L,C] in the four scan orders (operator.py:79-86)."""
    b, h, w, c = x_nhwc.shape
    flat = x_nhwc.reshape(b, h * w, c)
    return np.stack([flat[:, restore_index(r, h, w)] for r in range(4)], axis=1)


def _to_lines(seq, heads, d):
    """[B,R,L,C] -> [B*R*heads, L, d] (line order b, r, head)."""
    b, r, length, _ = seq.shape
    return seq.reshape(b, r, length, heads, d).transpose(0, 1, 3, 2, 4).reshape(b * r * heads, length, d)


def operator_forward(x_nhwc, q_nhwc, memories, d_skip, weights, head_dim, chunks=None, *,
                     dtype=np.float32, consts=None):
    """Fast spatial operator: out[b,h,w,c] = sum_r w[r,c] (y_r + skip_r[c] x) in NHWC fp32.

    ``chunks`` defaults to the row/column lengths (W, W, H, H) of ``srnl.py:128-139``.
    Summation order follows ``parallel_line.cuh:20-22`` then ``fused.cu:47-59``.
    """
    b, h, w, c = x_nhwc.shape
    heads, d = c // head_dim, head_dim
    if chunks is None:
        chunks = (w, w, h, h)
    xs = serialize(np.asarray(x_nhwc, dtype=dtype))
    qs = serialize(np.asarray(q_nhwc, dtype=dtype))
    n_lines = b * 4 * heads
    line_r = (np.arange(n_lines) // heads) % 4
    state_index = (np.arange(n_lines) % (4 * heads))
    y = srnl_lines(_to_lines(xs, heads, d), _to_lines(qs, heads, d), memories, state_index,
                   np.asarray(chunks)[line_r], q_raw=True, dtype=dtype, consts=consts)
    y = y.reshape(b, 4, heads, h * w, d).transpose(0, 1, 3, 2, 4).reshape(b, 4, h * w, c)
    skip = np.asarray(d_skip, dtype=dtype).reshape(-1, c)
    if skip.shape[0] == 1:
        skip = np.repeat(skip, 4, axis=0)
    wts = np.asarray(weights, dtype=dtype).reshape(4, c)
    xflat = np.asarray(x_nhwc, dtype=dtype).reshape(b, h * w, c)
    out = None
    for r in range(4):
        restored = np.empty_like(y[:, r])
        restored[:, restore_index(r, h, w)] = y[:, r]
        contrib = wts[r] * (restored + skip[r] * xflat)
        out = contrib if out is None else out + contrib
    return out.reshape(b, h, w, c)


def sequence_forward(x_packed, q, memories, chunks, *, q_raw=True, dtype=np.float32, consts=None):
    """Packed SRNL: x ``[B,R,heads,N,d]``; q raw ``[B,R,N,C]`` or normalized ``[B,R,heads,N,d]``.

    Memories ``[R,heads,d,d]``/``[R,heads,d]`` shared over the batch (chunk.py:193-196).
    Returns y ``[B,R,heads,N,d]`` (fused.cu:63-109; chunk.cu:252-509).
    """
    b, r, heads, length, d = x_packed.shape
    if q_raw:
        q_lines = _to_lines(np.asarray(q, dtype=dtype), heads, d)
    else:
        q_lines = np.asarray(q, dtype=dtype).reshape(b * r * heads, length, d)
    n_lines = b * r * heads
    mems = [np.asarray(m, dtype=dtype).reshape((r * heads,) + tuple(m.shape[2:])) for m in memories]
    line_r = (np.arange(n_lines) // heads) % r
    y = srnl_lines(np.asarray(x_packed, dtype=dtype).reshape(n_lines, length, d), q_lines, mems,
                   np.arange(n_lines) % (r * heads), np.asarray(chunks)[line_r], q_raw=q_raw,
                   dtype=dtype, consts=consts)
    return y.reshape(b, r, heads, length, d)


# --------------------------------------------------------------------------------------
# Elementwise tail
# --------------------------------------------------------------------------------------

def direction_fusion(y, x, d_skip, scale, height, width):
    """``visionhope_postprocess_scale_forward`` (direction_fusion.cu:11-65): NCHW fp32 output.

    y, x: ``[B,4,heads,L,d]``; d_skip ``[heads,d]`` or ``[4,heads,d]``; scale ``[4,C]``.
    """
    y = np.asarray(y, dtype=np.float32)
    x = np.asarray(x, dtype=np.float32)
    b, _, heads, length, d = y.shape
    c = heads * d
    skip = np.asarray(d_skip, dtype=np.float32).reshape(-1, c)
    if skip.shape[0] == 1:
        skip = np.repeat(skip, 4, axis=0)
    scale = np.asarray(scale, dtype=np.float32).reshape(4, c)
    out = None
    for r in range(4):
        seq = (y[:, r] + skip[r].reshape(heads, 1, d) * x[:, r])          # [B,heads,L,d]
        seq = seq.transpose(0, 2, 1, 3).reshape(b, length, c)
        restored = np.empty_like(seq)
        restored[:, restore_index(r, height, width)] = seq
        term = scale[r] * restored
        out = term if out is None else out + term
    return out.reshape(b, height, width, c).transpose(0, 3, 1, 2)


def grn(x_nchw, gamma, beta, eps=1e-6):
    """``grn_reference`` (utils/grn.py:26-38), fp32."""
    x = np.asarray(x_nchw, dtype=np.float32)
    c = x.shape[1]
    g = np.asarray(gamma, dtype=np.float32).reshape(1, c, 1, 1)
    bt = np.asarray(beta, dtype=np.float32).reshape(1, c, 1, 1)
    gx = np.sqrt((x.astype(np.float64) ** 2).sum(axis=(2, 3), keepdims=True)).astype(np.float32)
    nx = gx / (gx.mean(axis=1, keepdims=True) + np.float32(eps))
    return x * (np.float32(1) + g * nx) + bt


def layernorm2d(x_nchw, weight, bias, eps=1e-6):
    """LayerNorm over C per pixel, biased variance, fp32 out (layers.py:25-35)."""
    x = np.asarray(x_nchw, dtype=np.float64)
    mean = x.mean(axis=1, keepdims=True)
    var = ((x - mean) ** 2).mean(axis=1, keepdims=True)
    c = x.shape[1]
    w = np.asarray(weight, dtype=np.float64).reshape(1, c, 1, 1)
    b = np.asarray(bias, dtype=np.float64).reshape(1, c, 1, 1)
    return ((x - mean) / np.sqrt(var + eps) * w + b).astype(np.float32)


def qnorm(q_raw, heads, head_dim):
    """[B,4,L,C] -> normalized [B,4,heads,L,d] fp32 and 1/max(|q|,1e-12) [B,4,heads,L]."""
    q = np.asarray(q_raw, dtype=np.float32)
    b, r, length, _ = q.shape
    q = q.reshape(b, r, length, heads, head_dim).transpose(0, 1, 3, 2, 4)
    inv = np.float32(1) / np.maximum(np.sqrt((q.astype(np.float64) ** 2).sum(-1)), 1e-12).astype(np.float32)
    return q * inv[..., None], inv


def residual_add(residual, branch, gamma, drop_scale):
    """out = residual + branch * gamma_c * drop_scale_b on NHWC-ordered data (residual.py:31-52)."""
    res = np.asarray(residual, dtype=np.float32)
    br = np.asarray(branch, dtype=np.float32)
    b = res.shape[0]
    c = res.shape[-1]
    return res + br * np.asarray(gamma, dtype=np.float32).reshape(c) * \
        np.asarray(drop_scale, dtype=np.float32).reshape((b,) + (1,) * (res.ndim - 1))
