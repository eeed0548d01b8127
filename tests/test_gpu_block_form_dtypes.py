"""The block-form scans (srnl_ut.hip, srnl_utw.hip, srnl_utw32.hip) on fp16 and FP32
activations, through the spatial operator (``vh_srnl_spatial_forward``, FP32 output) and
the sequence entry, against the C oracle on the same inputs.

Each shape selects one kernel of the library's own dispatch: the one-wave block form with
its 2 x 2 and 1 x 4 packings (4096 and 1024 lines, head_dim 16), the few-line form with a
chunk's blocks over 1 or 2 waves (head_dim 16, fewer than 1024 lines) and the head_dim-32
form with chunks of 14 and 56 tokens (1 and 4 waves).  fp16 values are exact as bf16 hi + lo
operands and FP32 values enter within 2^-16 of their value, so both are held to the bound of
the bf16 block form, 2e-5 (about one hi + lo rounding of the output, five times inside the
FP32 contract of 1e-4; observed on MI355X: 5e-8 normwise with default-scale memories, up to
9e-7 elementwise with strong ones).  The observed errors are printed (``pytest -s``).
"""

import pytest
import torch

from tests.helpers import max_rel_err, memories, randn, rel_err

pytestmark = pytest.mark.gpu

BLOCK_TOL = 2e-5     # FP32 output: the block form's own arithmetic
FP32_TOL = 1e-4      # the FP32 parity contract (the stepped and wide kernels under an override)
FP16_OUT_TOL = 2e-3  # fp16 output of the sequence entry: one fp16 rounding (2^-11) on top

# (batch, H = W, heads, head_dim): kernel chosen by the default dispatch
SHAPES = [
    (64, 14, 16, 16),   # 4096 lines: one-wave block form, 2 x 2 packing
    (32, 14, 8, 16),    # 1024 lines: one-wave block form, 1 x 4 packing
    (4, 28, 4, 16),     # 64 lines, chunks of 28: few-line form, 2 waves per line
    (8, 14, 4, 32),     # head_dim 32, chunks of 14: one wave per line
    (2, 56, 2, 32),     # head_dim 32, chunks of 56: four waves per line
]


def _spatial_case(batch, hw, heads, d, dtype, kind):
    channels = heads * d
    seed = batch * 1000 + hw * 10 + heads + d
    mems = memories(4, heads, d, kind=kind, seed=seed)
    x = randn(batch, hw, hw, channels, seed=seed + 1).to(dtype)
    q = randn(batch, hw, hw, channels, seed=seed + 2).to(dtype)
    skip = randn(channels, seed=seed + 3, scale=0.1)
    wts = 1 + randn(4, channels, seed=seed + 4, scale=0.1)
    return mems, x, q, skip, wts


@pytest.mark.parametrize("batch,hw,heads,d", SHAPES)
@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("kind", ["perturbed", "strong"])
def test_block_form_spatial_fp16_fp32(oracle, device, batch, hw, heads, d, dtype, kind):
    from visionhope_amd.models.srnl_core.fused import srnl_spatial_inference

    mems, x, q, skip, wts = _spatial_case(batch, hw, heads, d, dtype, kind)
    print(f"\n[case] spatial {dtype} B={batch} {hw}x{hw} heads={heads} d={d} lines={batch * 4 * heads} {kind}",
          flush=True)
    got = srnl_spatial_inference(tuple(torch.from_numpy(m).to(device) for m in mems), x.to(device), q.to(device),
                                 skip.to(device), wts.to(device), (hw,) * 4).cpu().numpy()
    expected = oracle.operator_forward(x.float().numpy(), q.float().numpy(), mems, skip.numpy(), wts.numpy(), d)
    r, m = rel_err(got, expected), max_rel_err(got, expected)
    print(f"[err] {dtype} {hw}x{hw} d={d} {kind}: normwise {r:.2e} elementwise {m:.2e}", flush=True)
    assert r <= BLOCK_TOL and m <= BLOCK_TOL, f"{dtype} {hw}x{hw} d={d} {kind}: normwise {r:.3e}, elementwise {m:.3e}"


@pytest.mark.parametrize("head_dim,chunk", [(16, 14), (16, 64), (32, 14), (32, 49)])
@pytest.mark.parametrize("dtype,tol", [(torch.float16, FP16_OUT_TOL), (torch.float32, BLOCK_TOL)])
def test_block_form_sequence_fp16_fp32(oracle, device, head_dim, chunk, dtype, tol):
    """Packed sequences (the SRNL module's inference entry) of 196 tokens, 2 sequences, one
    direction, 2 heads (config 1's shape at head_dim 32), raw queries; y comes back in the
    input dtype (fp16: one rounding, 2^-11 relative, on top of the scan's error)."""
    from visionhope_amd.models.srnl_core.chunk import srnl_packed_forward

    batch, directions, heads, length = 2, 1, 2, 196
    seed = 7 * head_dim + chunk
    mems = memories(directions, heads, head_dim, kind="perturbed", seed=seed)
    x = randn(batch, directions, heads, length, head_dim, seed=seed + 1).to(dtype)
    q = randn(batch, directions, length, heads * head_dim, seed=seed + 2).to(dtype)
    print(f"\n[case] sequence {dtype} d={head_dim} chunk={chunk}", flush=True)
    got = srnl_packed_forward(tuple(torch.from_numpy(m).to(device) for m in mems), x.to(device), q.to(device),
                              [chunk], q_raw=True)
    assert got.dtype == dtype
    expected = oracle.sequence_forward(x.float().numpy(), q.float().numpy(), mems, [chunk])
    got = got.float().cpu().numpy()
    r, m = rel_err(got, expected), max_rel_err(got, expected)
    print(f"[err] sequence {dtype} d={head_dim} chunk={chunk}: normwise {r:.2e} elementwise {m:.2e}", flush=True)
    assert r <= tol and m <= tol, f"{dtype} d={head_dim} chunk={chunk}: normwise {r:.3e}, elementwise {m:.3e}"


@pytest.mark.parametrize("batch,hw,heads,d,forced", [
    (32, 14, 8, 16, {"scan_ut": 0}),      # stepped form, 1024 lines
    (4, 28, 4, 16, {"scan_wide": 2}),     # wide scan, 64 lines
    (8, 14, 4, 32, {"scan_utw": 0}),      # head_dim 32: wide scan
])
def test_fp32_forced_stepped_and_wide_forms(oracle, device, dispatch, batch, hw, heads, d, forced):
    """The kernels the block form replaced stay reachable for FP32 maps under an override."""
    from visionhope_amd.models.srnl_core.fused import srnl_spatial_inference

    dispatch(**forced)
    mems, x, q, skip, wts = _spatial_case(batch, hw, heads, d, torch.float32, "strong")
    print(f"\n[case] forced {forced} FP32 B={batch} {hw}x{hw} d={d}", flush=True)
    got = srnl_spatial_inference(tuple(torch.from_numpy(m).to(device) for m in mems), x.to(device), q.to(device),
                                 skip.to(device), wts.to(device), (hw,) * 4).cpu().numpy()
    expected = oracle.operator_forward(x.numpy(), q.numpy(), mems, skip.numpy(), wts.numpy(), d)
    r, m = rel_err(got, expected), max_rel_err(got, expected)
    print(f"[err] forced {forced}: normwise {r:.2e} elementwise {m:.2e}", flush=True)
    assert r <= FP32_TOL and m <= FP32_TOL, f"{forced}: normwise {r:.3e}, elementwise {m:.3e}"
