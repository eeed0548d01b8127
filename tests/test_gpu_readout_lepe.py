"""The spatial readout with the block's local position encoding computed in the same pass
(``vh_srnl_spatial_readout_lepe``), against

* the two-pass form it replaces, bit for bit: the 5x5 depthwise kernel (plain epilogue,
  ``vh_dwconv2d_nhwc_forward``) writes the encoding in the map's dtype and the readout adds
  it (``vh_srnl_spatial_readout`` with aux).  Both accumulate each output from the bias in
  tap-row order, left to right, with the same FP32 fused multiply-adds, so any difference
  is a defect (a halo pixel read from the wrong place, a lost tap or edge);
* an independent reference: the C oracle's operator output plus torch's CPU FP32
  ``conv2d`` of the same map rounded to the map's dtype, within one rounding of the
  output (bf16: 2^-8 relative on the largest value, fp16 and FP32 tighter).

Shapes cover both readout tiles (16 x 16 pixels, and 8 x 8 on maps of at most 8 x 8,
each also forced onto the other map size), head_dim 16 and 32 (two workgroups per tile),
ragged and non-square maps whose last tiles are partial, the three activation dtypes, and
the per-element readout that fp16 maps with head_dim 32 and head_dim 8 take (encoding in
place through the output).  The observed errors are printed (``pytest -s``).
"""

import copy

import pytest
import torch
from torch.nn import functional as F

from tests.helpers import max_rel_err, memories, randn, rel_err

pytestmark = pytest.mark.gpu

OUT_TOL = {torch.bfloat16: 5e-3, torch.float16: 1e-3, torch.float32: 1e-4}

# (batch, H, W, heads, head_dim, dtype, dispatch override)
CASES = [
    (8, 56, 56, 2, 16, torch.bfloat16, {}),                     # Tiny stage 1 shape, 16 x 16 tiles
    (16, 14, 14, 8, 16, torch.bfloat16, {}),                    # stage 3: one partial tile per image
    (32, 7, 7, 16, 16, torch.bfloat16, {}),                     # stage 4: 8 x 8 tiles
    (4, 20, 13, 4, 16, torch.bfloat16, {}),                     # non-square, partial tiles on both axes
    (4, 28, 28, 3, 32, torch.bfloat16, {}),                     # head_dim 32: two halves per tile
    (8, 14, 14, 8, 16, torch.bfloat16, {"readout_tile": 8}),    # 8 x 8 tiles on a 14 x 14 map
    (16, 7, 7, 16, 16, torch.bfloat16, {"readout_tile": 16}),   # 16 x 16 tiles on a 7 x 7 map
    (8, 14, 14, 4, 16, torch.float16, {}),
    (8, 14, 14, 4, 16, torch.float32, {}),
    (4, 9, 11, 2, 32, torch.float32, {}),
    (4, 14, 14, 2, 32, torch.float16, {}),                      # per-element readout (fp16, head_dim 32)
    (4, 14, 14, 4, 8, torch.bfloat16, {}),                      # per-element readout (head_dim 8)
]


def _case(batch, h, w, heads, d, dtype):
    channels = heads * d
    seed = batch * 7 + h * 3 + w + heads + d
    mems = memories(4, heads, d, kind="strong", seed=seed)
    x = randn(batch, h, w, channels, seed=seed + 1).to(dtype)
    q = randn(batch, h, w, channels, seed=seed + 2).to(dtype)
    skip = randn(channels, seed=seed + 3, scale=0.1)
    wts = 1 + randn(4, channels, seed=seed + 4, scale=0.1)
    conv = torch.nn.Conv2d(channels, channels, 5, padding=2, groups=channels)
    with torch.no_grad():
        conv.weight.copy_(randn(channels, 1, 5, 5, seed=seed + 5, scale=0.2))
        conv.bias.copy_(randn(channels, seed=seed + 6, scale=0.1))
    return mems, x, q, skip, wts, conv


@pytest.mark.parametrize("batch,h,w,heads,d,dtype,forced", CASES)
def test_readout_with_position_encoding(oracle, device, dispatch, batch, h, w, heads, d, dtype, forced):
    from visionhope_amd.models.srnl_core.fused import srnl_spatial_readout, srnl_spatial_scan
    from visionhope_amd.utils import dwconv

    if forced:
        dispatch(**forced)
    mems, x, q, skip, wts, conv = _case(batch, h, w, heads, d, dtype)
    print(f"\n[case] readout+lepe {dtype} B={batch} {h}x{w} heads={heads} d={d} {forced}", flush=True)
    chunks = (w, w, h, h)
    xd, qd = x.to(device), q.to(device)
    conv_d = copy.deepcopy(conv).to(device)
    skip_d, wts_d = skip.to(device), wts.to(device)
    ws = srnl_spatial_scan(tuple(torch.from_numpy(m).to(device) for m in mems), xd, chunks)
    taps, bias = dwconv.depthwise_taps(conv_d)
    fused = srnl_spatial_readout(ws, xd, qd, skip_d, wts_d, chunks, d, out_dtype=dtype, lepe=(taps, bias))
    lepe = dwconv.depthwise_conv(xd.permute(0, 3, 1, 2), conv_d, dwconv.EPI_PLAIN)
    two_pass = srnl_spatial_readout(ws, xd, qd, skip_d, wts_d, chunks, d, aux=lepe.permute(0, 2, 3, 1),
                                    out_dtype=dtype)
    torch.cuda.synchronize()
    assert fused.dtype == dtype and fused.shape == x.shape
    differ = (fused != two_pass).sum().item()
    print(f"[bits] {differ} of {fused.numel()} outputs differ from the two-pass form", flush=True)
    assert differ == 0, f"{differ} outputs differ from the depthwise pass + readout"

    with torch.no_grad():
        enc = F.conv2d(x.float().permute(0, 3, 1, 2), conv.weight.float(), conv.bias.float(), padding=2,
                       groups=x.shape[-1]).to(dtype).float().permute(0, 2, 3, 1).numpy()
    expected = oracle.operator_forward(x.float().numpy(), q.float().numpy(), mems, skip.numpy(), wts.numpy(), d) + enc
    got = fused.float().cpu().numpy()
    r, m = rel_err(got, expected), max_rel_err(got, expected)
    print(f"[err] readout+lepe {dtype} {h}x{w} d={d}: normwise {r:.2e} elementwise {m:.2e}", flush=True)
    tol = OUT_TOL[dtype]
    assert r <= tol and m <= tol, f"normwise {r:.3e}, elementwise {m:.3e}"


def test_position_encoding_arguments_are_checked(device):
    from visionhope_amd.models.srnl_core.fused import srnl_spatial_readout, srnl_spatial_scan

    mems, x, q, skip, wts, conv = _case(2, 14, 14, 2, 16, torch.bfloat16)
    xd = x.to(device)
    ws = srnl_spatial_scan(tuple(torch.from_numpy(m).to(device) for m in mems), xd, (14,) * 4)
    taps = torch.zeros(25, 32, device=device)
    with pytest.raises(ValueError):   # FP32 output is not offered with the encoding
        srnl_spatial_readout(ws, xd, q.to(device), skip.to(device), wts.to(device), (14,) * 4, 16,
                             out_dtype=torch.float32, lepe=(taps, None))
    with pytest.raises(ValueError):   # taps of the wrong size
        srnl_spatial_readout(ws, xd, q.to(device), skip.to(device), wts.to(device), (14,) * 4, 16,
                             out_dtype=torch.bfloat16, lepe=(taps[:9], None))
