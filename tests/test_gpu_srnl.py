"""GPU parity of the SRNL kernels (through the C ABI) against the CPU oracle.

Tolerances: fp32 I/O 1e-4 normwise and
elementwise-on-scale; bf16/fp16 I/O 2e-2 with the oracle fed the same rounded
inputs.
"""

import math

import numpy as np
import pytest
import torch

from tests.helpers import assert_close, memories, randn

pytestmark = pytest.mark.gpu

FP32_TOL = 1e-4
HALF_TOL = 2e-2


def _packed_case(batch, directions, heads, length, head_dim, dtype, seed):
    x = randn(batch, directions, heads, length, head_dim, seed=seed).to(dtype)
    q = randn(batch, directions, length, heads * head_dim, seed=seed + 1).to(dtype)
    return x, q


@pytest.mark.parametrize("head_dim", [4, 8, 16, 32, 64])
@pytest.mark.parametrize("kind", ["default", "perturbed", "strong"])
def test_sequence_forward_fp32_head_dims(oracle, device, head_dim, kind):
    from visionhope_amd.models.srnl_core.chunk import srnl_packed_forward

    batch, directions, heads, length, chunk = 2, 2, 2, 45, 7   # 45 = 6*7 + 3: padded last chunk
    mems = memories(directions, heads, head_dim, kind=kind, seed=head_dim)
    x, q = _packed_case(batch, directions, heads, length, head_dim, torch.float32, seed=head_dim + 7)
    y = srnl_packed_forward(tuple(torch.from_numpy(m).to(device) for m in mems), x.to(device),
                            q.to(device), [chunk, chunk + 2], q_raw=True)
    expected = oracle.sequence_forward(x.numpy(), q.numpy(), mems, [chunk, chunk + 2])
    assert_close(y.cpu().numpy(), expected, FP32_TOL, f"d={head_dim} {kind}")


SCAN16_PACKINGS = ["1x4", "2x4", "4x4", "1x2", "2x2"]   # <lines per wave>x<16-slot tiles per wave>


@pytest.mark.parametrize("packing", SCAN16_PACKINGS)
@pytest.mark.parametrize("height,width", [(7, 7), (14, 14), (6, 9), (19, 37)])
@pytest.mark.parametrize("dtype,tol", [(torch.float32, FP32_TOL), (torch.bfloat16, HALF_TOL)])
def test_spatial_scan16_packing(oracle, device, dispatch, packing, height, width, dtype, tol):
    """head_dim 16 scan with 1, 2 or 4 lines and 2 or 4 token tiles per wave (forced; the
    library picks a packing by itself from the line count): short and long chunks (more
    than one tile per chunk), rectangular images."""
    dispatch(scan_pack=packing)
    heads = 4
    channels = heads * 16
    mems = memories(4, heads, 16, kind="strong", seed=height * 31 + width)
    x = randn(2, height, width, channels, seed=71).to(dtype)
    q = randn(2, height, width, channels, seed=72).to(dtype)
    skip = randn(channels, seed=73, scale=0.1)
    wts = 1 + randn(4, channels, seed=74, scale=0.1)
    got = _spatial(device, x, q, mems, skip, wts, (width, width, height, height))
    expected = oracle.operator_forward(x.float().numpy(), q.float().numpy(), mems, skip.numpy(), wts.numpy(), 16)
    assert_close(got, expected, tol, f"scan16 packing {packing} {height}x{width} {dtype}")


@pytest.mark.parametrize("packing", ["2x4", "4x4", "1x2", "2x2"])
@pytest.mark.parametrize("chunks", [(5, 16), (17, 33)])
def test_sequence_scan16_packing(oracle, device, dispatch, packing, chunks):
    """Packed sequences with head_dim 16 and 4 heads, lines and tiles packed per wave,
    padded chunks."""
    from visionhope_amd.models.srnl_core.chunk import srnl_packed_forward

    dispatch(scan_pack=packing)
    batch, directions, heads, length = 2, 2, 4, 83
    mems = memories(directions, heads, 16, kind="perturbed", seed=int(packing[0]))
    x, q = _packed_case(batch, directions, heads, length, 16, torch.float32, seed=81)
    y = srnl_packed_forward(tuple(torch.from_numpy(m).to(device) for m in mems), x.to(device),
                            q.to(device), list(chunks), q_raw=True)
    expected = oracle.sequence_forward(x.numpy(), q.numpy(), mems, list(chunks))
    assert_close(y.cpu().numpy(), expected, FP32_TOL, f"sequence packing {packing} chunks={chunks}")


def test_config1_standalone_srnl(oracle, device):
    """Standalone SRNL workload: B=2, 14x14 tokens (L=196), C=64 in 2 heads, chunk 14, fp32."""
    from visionhope_amd.models import SRNL

    torch.manual_seed(1234)
    module = SRNL(64, head_dim=32, chunk_size=14).to(device).eval()
    with torch.no_grad():
        module.M_eta_0.normal_(0, 0.1)
        module.M_alpha_0.normal_(0, 0.1)
    x = randn(2, 196, 64, seed=1234)
    with torch.no_grad():
        y = module(x.to(device)).cpu().numpy()
    mems = tuple(p.detach().cpu().numpy() for p in module.initial_memories)
    packed = x.view(2, 1, 196, 2, 32).transpose(2, 3).numpy()
    # ordinary path for one direction: queries normalised per head (srnl.py:153-157)
    expected = oracle.sequence_forward(packed, x.view(2, 1, 196, 64).numpy(), mems, [14], q_raw=True)
    expected = expected[:, 0].transpose(0, 2, 1, 3).reshape(2, 196, 64)
    assert_close(y, expected, FP32_TOL, "config 1")


@pytest.mark.parametrize("dtype,tol", [(torch.float32, FP32_TOL), (torch.bfloat16, HALF_TOL),
                                       (torch.float16, HALF_TOL)])
@pytest.mark.parametrize("head_dim", [16, 32])
def test_srnl_module_fast_inference_sequence_path(oracle, device, dtype, tol, head_dim):
    """SRNL(fast_inference=True) in eval mode without gradients takes the sequence inference
    entry (reference ``fused.py:211-219`` via ``srnl.py:_inference_path``): config 1's
    standalone shape, and the packed four-direction call with spatial chunks."""
    from visionhope_amd.models import SRNL

    torch.manual_seed(1234)
    module = SRNL(64, head_dim=head_dim, chunk_size=14, fast_inference=True).to(device).eval()
    with torch.no_grad():
        module.M_eta_0.normal_(0, 0.1)
        module.M_alpha_0.normal_(0, 0.1)
    x = randn(2, 196, 64, seed=1234).to(dtype)
    with torch.no_grad():
        assert module.inference_status(x.to(device))["path"] == "sequence"
        y = module(x.to(device))
    assert y.dtype == dtype
    mems = tuple(p.detach().cpu().numpy() for p in module.initial_memories)
    heads = 64 // head_dim
    packed = x.float().view(2, 1, 196, heads, head_dim).transpose(2, 3).numpy()
    expected = oracle.sequence_forward(packed, x.float().view(2, 1, 196, 64).numpy(), mems, [14], q_raw=True)
    expected = expected[:, 0].transpose(0, 2, 1, 3).reshape(2, 196, 64)
    assert_close(y.float().cpu().numpy(), expected, tol, f"fast inference standalone {dtype} d={head_dim}")

    four = SRNL(32, head_dim=head_dim, directions=4, fast_inference=True).to(device).eval()
    with torch.no_grad():
        four.M_eta_0.normal_(0, 0.1)
        four.M_alpha_0.normal_(0, 0.1)
    height, width = 6, 9
    xp = randn(2, 4, 32 // head_dim, height * width, head_dim, seed=5).to(dtype)
    qp = randn(2, 4, height * width, 32, seed=6).to(dtype)
    with torch.no_grad():
        yp = four(xp.to(device), qp.to(device), spatial_shape=(height, width))
    mems = tuple(p.detach().cpu().numpy() for p in four.initial_memories)
    expected = oracle.sequence_forward(xp.float().numpy(), qp.float().numpy(), mems, [width, width, height, height])
    assert_close(yp.float().cpu().numpy(), expected, tol, f"fast inference packed {dtype} d={head_dim}")


@pytest.mark.parametrize("dtype,tol", [(torch.bfloat16, HALF_TOL), (torch.float16, HALF_TOL)])
def test_sequence_forward_half(oracle, device, dtype, tol):
    from visionhope_amd.models.srnl_core.chunk import srnl_packed_forward

    mems = memories(4, 3, 16, kind="perturbed", seed=3)
    x, q = _packed_case(2, 4, 3, 100, 16, dtype, seed=11)
    y = srnl_packed_forward(tuple(torch.from_numpy(m).to(device) for m in mems), x.to(device),
                            q.to(device), [10] * 4, q_raw=True)
    assert y.dtype == dtype
    expected = oracle.sequence_forward(x.float().numpy(), q.float().numpy(), mems, [10] * 4)
    assert_close(y.float().cpu().numpy(), expected, tol, str(dtype))


def test_normalized_query_path(oracle, device):
    from visionhope_amd.models.srnl_core.chunk import srnl_packed_forward

    mems = memories(1, 2, 16, kind="strong", seed=5)
    x = randn(3, 1, 2, 64, 16, seed=21)
    q = randn(3, 1, 2, 64, 16, seed=22)
    q = q / q.norm(dim=-1, keepdim=True)
    y = srnl_packed_forward(tuple(torch.from_numpy(m).to(device) for m in mems), x.to(device),
                            q.to(device), [16], q_raw=False)
    expected = oracle.sequence_forward(x.numpy(), q.numpy(), mems, [16], q_raw=False)
    assert_close(y.cpu().numpy(), expected, FP32_TOL, "normalized q")


def _spatial(device, x_nhwc, q_nhwc, mems, skip, wts, chunks):
    from visionhope_amd.models.srnl_core.fused import srnl_spatial_inference

    return srnl_spatial_inference(tuple(torch.from_numpy(m).to(device) for m in mems),
                                  x_nhwc.to(device), q_nhwc.to(device), skip.to(device),
                                  wts.to(device), chunks).cpu().numpy()


@pytest.mark.parametrize("height,width,head_dim,heads", [(7, 7, 16, 2), (6, 9, 16, 3), (12, 5, 32, 1),
                                                         (4, 4, 8, 2), (5, 3, 64, 1), (3, 6, 4, 4)])
@pytest.mark.parametrize("skip_per_direction", [False, True])
def test_spatial_forward_fp32(oracle, device, height, width, head_dim, heads, skip_per_direction):
    channels = heads * head_dim
    mems = memories(4, heads, head_dim, kind="strong", seed=height * width)
    x = randn(2, height, width, channels, seed=31)
    q = randn(2, height, width, channels, seed=32)
    skip = randn(4 if skip_per_direction else 1, channels, seed=33, scale=0.1).reshape(-1)
    wts = 1 + randn(4, channels, seed=34, scale=0.1)
    chunks = (width, width, height, height)
    got = _spatial(device, x, q, mems, skip, wts, chunks)
    expected = oracle.operator_forward(x.numpy(), q.numpy(), mems, skip.numpy(), wts.numpy(), head_dim)
    assert_close(got, expected, FP32_TOL, f"spatial {height}x{width} d={head_dim}")


@pytest.mark.parametrize("height,width,heads", [(19, 37, 2), (16, 32, 1), (33, 17, 3), (56, 56, 2)])
@pytest.mark.parametrize("dtype,tol", [(torch.float32, FP32_TOL), (torch.bfloat16, HALF_TOL),
                                       (torch.float16, HALF_TOL)])
def test_spatial_readout_tiles(oracle, device, height, width, heads, dtype, tol):
    """head_dim 16 with row/column chunks: 16x16 tile readout, full and ragged edge tiles."""
    channels = heads * 16
    mems = memories(4, heads, 16, kind="strong", seed=height + width)
    x = randn(1, height, width, channels, seed=51).to(dtype)
    q = randn(1, height, width, channels, seed=52).to(dtype)
    skip = randn(4 * channels, seed=53, scale=0.1)
    wts = 1 + randn(4, channels, seed=54, scale=0.1)
    got = _spatial(device, x, q, mems, skip, wts, (width, width, height, height))
    expected = oracle.operator_forward(x.float().numpy(), q.float().numpy(), mems, skip.numpy(), wts.numpy(), 16)
    assert_close(got, expected, tol, f"tiled readout {height}x{width} {dtype}")


def test_spatial_forward_other_chunks(oracle, device):
    """Chunk lengths other than the row/column lengths take the per-element readout."""
    heads, height, width = 2, 6, 9
    mems = memories(4, heads, 16, kind="perturbed", seed=5)
    x = randn(2, height, width, 32, seed=61)
    q = randn(2, height, width, 32, seed=62)
    skip = randn(32, seed=63, scale=0.1)
    wts = 1 + randn(4, 32, seed=64, scale=0.1)
    chunks = (5, 7, 3, 4)
    got = _spatial(device, x, q, mems, skip, wts, chunks)
    expected = oracle.operator_forward(x.numpy(), q.numpy(), mems, skip.numpy(), wts.numpy(), 16, chunks)
    assert_close(got, expected, FP32_TOL, "spatial other chunks")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_spatial_forward_half_config3_shape(oracle, device, dtype):
    """Operator workload shape at reduced batch (B=2, 56x56, C=96, 3 heads of 32), bf16 and
    fp16 activations (the reference builds every kernel for both, cuda_source.py:50-68)."""
    heads, head_dim, hw = 3, 32, 56
    channels = heads * head_dim
    mems = memories(4, heads, head_dim, kind="perturbed", seed=9)
    x = randn(2, hw, hw, channels, seed=41).to(dtype)
    q = randn(2, hw, hw, channels, seed=42).to(dtype)
    skip = randn(channels, seed=43, scale=0.1)
    wts = 1 + randn(4, channels, seed=44, scale=0.1)
    got = _spatial(device, x, q, mems, skip, wts, (hw, hw, hw, hw))
    expected = oracle.operator_forward(x.float().numpy(), q.float().numpy(), mems, skip.numpy(),
                                       wts.numpy(), head_dim)
    assert_close(got, expected, HALF_TOL, f"config3 {dtype}")


@pytest.mark.parametrize("height,width,head_dim,heads", [(7, 7, 16, 2), (6, 9, 16, 3), (12, 5, 32, 1),
                                                         (14, 14, 32, 2), (4, 4, 8, 2), (5, 3, 64, 1)])
def test_spatial_forward_fp16(oracle, device, height, width, head_dim, heads):
    """fp16 activations through the spatial operator at every head_dim path (the per-element
    readout at head_dim 32, the matrix-core tile readout at 16)."""
    channels = heads * head_dim
    mems = memories(4, heads, head_dim, kind="strong", seed=height * width + 1)
    x = randn(2, height, width, channels, seed=35).half()
    q = randn(2, height, width, channels, seed=36).half()
    skip = randn(channels, seed=37, scale=0.1)
    wts = 1 + randn(4, channels, seed=38, scale=0.1)
    got = _spatial(device, x, q, mems, skip, wts, (width, width, height, height))
    expected = oracle.operator_forward(x.float().numpy(), q.float().numpy(), mems, skip.numpy(), wts.numpy(), head_dim)
    assert_close(got, expected, HALF_TOL, f"spatial fp16 {height}x{width} d={head_dim}")


def test_line_forward_seq_noatomic_reference_layout(oracle, device):
    """The reference's own entry (serialized stacks [B,4,L,C]) through the C ABI."""
    from visionhope_amd.models.srnl_core.fused import load_fused_cuda

    heads, head_dim, height, width = 2, 16, 8, 8
    channels = heads * head_dim
    mems = memories(4, heads, head_dim, kind="perturbed", seed=77)
    x = randn(2, height, width, channels, seed=51)
    q = randn(2, height, width, channels, seed=52)
    xs = torch.from_numpy(oracle.serialize(x.numpy()))
    qs = torch.from_numpy(oracle.serialize(q.numpy()))
    skip = randn(channels, seed=53, scale=0.1)
    wts = 1 + randn(4, channels, seed=54, scale=0.1)
    ops = load_fused_cuda(torch.float32)
    got = ops.srnl_line_forward_seq_noatomic(
        *(torch.from_numpy(m).to(device) for m in mems), xs.to(device), qs.to(device),
        skip.to(device), wts.to(device), height, width, head_dim).cpu().numpy()
    expected = oracle.operator_forward(x.numpy(), q.numpy(), mems, skip.numpy(), wts.numpy(), head_dim)
    assert_close(got, expected, FP32_TOL, "line_forward_seq_noatomic")


def test_long_chunk_base512_like(oracle, device):
    """Chunks longer than 64 tokens (Base-512 stage 1 rows are 128 tokens)."""
    from visionhope_amd.models.srnl_core.lines import srnl_long_chunk

    heads, head_dim, length, chunk = 3, 16, 128 * 4, 128
    mems = memories(4, heads, head_dim, kind="perturbed", seed=88)
    x, q = _packed_case(1, 4, heads, length, head_dim, torch.float32, seed=61)
    dev = tuple(torch.from_numpy(m).to(device) for m in mems)
    with torch.no_grad():
        y = srnl_long_chunk(*dev, x.to(device), q.to(device), chunk, heads, head_dim)
    expected = oracle.sequence_forward(x.numpy(), q.numpy(), mems, [chunk] * 4)
    assert_close(y.cpu().numpy(), expected, FP32_TOL, "long chunk")


def test_zero_length_rejected(device):
    from visionhope_amd.models.srnl_core.chunk import srnl_packed_forward

    mems = tuple(torch.from_numpy(m).to(device) for m in memories(1, 1, 16))
    x = torch.zeros(1, 1, 1, 0, 16, device=device)
    q = torch.zeros(1, 1, 0, 16, device=device)
    with pytest.raises(RuntimeError, match="nonempty"):
        srnl_packed_forward(mems, x, q, [4], q_raw=True)


def test_full_config3_properties(device):
    """Full operator workload (B=32, 56x56, C=96, d=32, bf16) is too large for the oracle
    in seconds; check the closed form that fixes it exactly: with M_k = M_v = 0 and zero
    gate vectors every gain is 0.9^56 I, so y_r of a pixel in chunk c is
    0.9^(56 c) M_m q_hat (first-chunk GEMM, then pure decay)."""
    from visionhope_amd.models.srnl_core.fused import srnl_spatial_inference

    batch, hw, heads, head_dim = 32, 56, 3, 32
    channels = heads * head_dim
    gen = torch.Generator().manual_seed(5)
    m_m = torch.randn(4, heads, head_dim, head_dim, generator=gen) * 0.05
    zeros_m = torch.zeros_like(m_m)
    zeros_v = torch.zeros(4, heads, head_dim)
    x = torch.randn(batch, hw, hw, channels, generator=gen).bfloat16()
    q = torch.randn(batch, hw, hw, channels, generator=gen).bfloat16()
    mems = tuple(t.to(device) for t in (m_m, zeros_m, zeros_m, zeros_v, zeros_v))
    skip = torch.zeros(channels, device=device)
    wts = torch.ones(4, channels, device=device)
    out = srnl_spatial_inference(mems, x.to(device), q.to(device), skip, wts, (hw,) * 4)
    # expected: sum_r 0.9^(56*chunk_r) * M_m[r] q_hat, evaluated on the GPU in fp32 by torch
    qd = q.to(device).float().view(batch, hw, hw, heads, head_dim)
    qh = qd / qd.norm(dim=-1, keepdim=True).clamp_min(1e-12)
    mm = m_m.to(device)
    rows = torch.arange(hw, device=device, dtype=torch.float64)
    expected = torch.zeros(batch, hw, hw, heads, head_dim, device=device)
    alpha = 1.0 / (1.0 + math.exp(-2.197224577))
    for r in range(4):
        y = torch.matmul(qh.unsqueeze(-2), mm[r].transpose(-1, -2).contiguous()).squeeze(-2)
        if r == 0:
            chunk = rows.view(hw, 1).expand(hw, hw)
        elif r == 1:
            chunk = (hw - 1 - rows).view(hw, 1).expand(hw, hw)
        elif r == 2:
            chunk = rows.view(1, hw).expand(hw, hw)
        else:
            chunk = (hw - 1 - rows).view(1, hw).expand(hw, hw)
        decay = torch.pow(torch.tensor(alpha, dtype=torch.float64, device=device), hw * chunk).float()
        expected += y * decay.view(1, hw, hw, 1, 1)
    got = out.view(batch, hw, hw, heads, head_dim)
    assert torch.isfinite(got).all()
    err = (got - expected).norm() / expected.norm()
    assert err.item() < 1e-4, err.item()


# (head_dim, waves per line, mode): "rows" splits the rows of the gain over the waves,
# "blocks" also splits each segment's tokens into blocks composed afterwards.
WIDE_CASES = [(16, 1, "rows"), (16, 2, "rows"), (16, 2, "blocks"), (16, 4, "rows"), (16, 4, "blocks"),
              (32, 2, "rows"), (32, 4, "rows"), (32, 4, "blocks")]


def _wide_env(dispatch, waves, mode):
    dispatch(scan_wide=waves, scan_tb="1" if mode == "rows" else "2")


@pytest.mark.parametrize("head_dim,waves,mode", WIDE_CASES)
@pytest.mark.parametrize("height,width", [(7, 7), (14, 14), (19, 37), (56, 56)])
@pytest.mark.parametrize("dtype,tol", [(torch.float32, FP32_TOL), (torch.bfloat16, HALF_TOL)])
def test_spatial_scan_wide(oracle, device, dispatch, head_dim, waves, mode, height, width, dtype, tol):
    """The scan with one line per workgroup of 1, 2 or 4 waves (rows of the gain split over
    the waves): square and rectangular maps, chunks of 7 to 56 (one to four 16-token tiles,
    ragged last tiles), strong memories (active soft cap and spectral clamp)."""
    _wide_env(dispatch, waves, mode)
    heads = 2
    channels = heads * head_dim
    mems = memories(4, heads, head_dim, kind="strong", seed=height * 7 + width + head_dim)
    x = randn(2, height, width, channels, seed=91).to(dtype)
    q = randn(2, height, width, channels, seed=92).to(dtype)
    skip = randn(channels, seed=93, scale=0.01)   # small: the recurrence's output dominates
    wts = 1 + randn(4, channels, seed=94, scale=0.1)
    got = _spatial(device, x, q, mems, skip, wts, (width, width, height, height))
    expected = oracle.operator_forward(x.float().numpy(), q.float().numpy(), mems, skip.numpy(), wts.numpy(),
                                       head_dim)
    assert_close(got, expected, tol, f"wide scan d={head_dim} W={waves} {mode} {height}x{width} {dtype}")


@pytest.mark.parametrize("head_dim,waves,mode", WIDE_CASES)
@pytest.mark.parametrize("chunks", [(5, 16, 64, 3), (65, 128, 100, 200)])
@pytest.mark.parametrize("dtype,tol", [(torch.float32, FP32_TOL), (torch.bfloat16, HALF_TOL)])
def test_sequence_scan_wide(oracle, device, dispatch, head_dim, waves, mode, chunks, dtype, tol):
    """Packed sequences through the wide scan: chunks shorter than a tile, spanning several
    64-token segments, and ragged last chunks (length 263 = 2*128 + 7)."""
    from visionhope_amd.models.srnl_core.chunk import srnl_packed_forward

    _wide_env(dispatch, waves, mode)
    batch, directions, heads, length = 1, 4, 2, 263
    mems = memories(directions, heads, head_dim, kind="perturbed", seed=head_dim + waves)
    x, q = _packed_case(batch, directions, heads, length, head_dim, dtype, seed=95)
    y = srnl_packed_forward(tuple(torch.from_numpy(m).to(device) for m in mems), x.to(device),
                            q.to(device), list(chunks), q_raw=True)
    expected = oracle.sequence_forward(x.float().numpy(), q.float().numpy(), mems, list(chunks))
    assert_close(y.float().cpu().numpy(), expected, tol, f"wide sequence d={head_dim} W={waves} {mode} {chunks}")


# bf16 head_dim-16 scans with fewer lines than SIMDs take the block form with one workgroup
# per line and the chunk's 16-token blocks spread over 1, 2, 4 or 8 waves (chunks of at most
# 128 tokens; longer chunks keep the wide scan).  FP32 output of a bf16 scan: the block form's
# hi + lo products put it within about 2^-16 of the oracle.
FEW_LINES_TOL = 2e-5


@pytest.mark.parametrize("height,width,heads", [(56, 56, 2), (28, 28, 4), (9, 6, 3), (16, 128, 1), (32, 100, 1),
                                                (7, 7, 2), (128, 128, 1)])
@pytest.mark.parametrize("kind", ["perturbed", "strong"])
def test_spatial_few_lines_block_form(oracle, device, height, width, heads, kind):
    channels = heads * 16
    mems = memories(4, heads, 16, kind=kind, seed=height * 3 + width)
    x = randn(2, height, width, channels, seed=height + 101).bfloat16()
    q = randn(2, height, width, channels, seed=width + 102).bfloat16()
    skip = randn(channels, seed=103, scale=0.1)
    wts = 1 + randn(4, channels, seed=104, scale=0.1)
    got = _spatial(device, x, q, mems, skip, wts, (width, width, height, height))
    expected = oracle.operator_forward(x.float().numpy(), q.float().numpy(), mems, skip.numpy(), wts.numpy(), 16)
    assert_close(got, expected, FEW_LINES_TOL, f"few-line block form {height}x{width} heads={heads} {kind}")


@pytest.mark.parametrize("height,width,heads", [(56, 56, 3), (28, 28, 2), (14, 14, 2), (9, 6, 3), (7, 40, 1),
                                                (64, 64, 1), (65, 20, 1)])
@pytest.mark.parametrize("kind", ["perturbed", "strong"])
def test_spatial_head_dim32_block_form(oracle, device, height, width, heads, kind):
    """head_dim 32, bf16: the block form with one workgroup per line and the chunk's blocks
    over 1, 2 or 4 waves (chunks of up to 64 tokens; the 65-row map sends its column scans'
    launch to the wide scan)."""
    channels = heads * 32
    mems = memories(4, heads, 32, kind=kind, seed=height * 5 + width)
    x = randn(2, height, width, channels, seed=height + 111).bfloat16()
    q = randn(2, height, width, channels, seed=width + 112).bfloat16()
    skip = randn(channels, seed=113, scale=0.1)
    wts = 1 + randn(4, channels, seed=114, scale=0.1)
    got = _spatial(device, x, q, mems, skip, wts, (width, width, height, height))
    expected = oracle.operator_forward(x.float().numpy(), q.float().numpy(), mems, skip.numpy(), wts.numpy(), 32)
    assert_close(got, expected, FEW_LINES_TOL, f"d=32 block form {height}x{width} heads={heads} {kind}")


@pytest.mark.parametrize("chunks", [(5, 16, 64, 3), (64, 33, 17, 48), (65, 7, 30, 12)])
def test_sequence_head_dim32_block_form(oracle, device, chunks):
    """Packed bf16 sequences with head_dim 32 (157 tokens, ragged last chunks) through the
    block form; a chunk of 65 tokens sends the launch to the wide scan."""
    from visionhope_amd.models.srnl_core.chunk import srnl_packed_forward

    batch, directions, heads, length = 2, 4, 2, 157
    mems = memories(directions, heads, 32, kind="strong", seed=sum(chunks) + 1)
    x, q = _packed_case(batch, directions, heads, length, 32, torch.bfloat16, seed=117)
    y = srnl_packed_forward(tuple(torch.from_numpy(m).to(device) for m in mems), x.to(device),
                            q.to(device), list(chunks), q_raw=True)
    expected = oracle.sequence_forward(x.float().numpy(), q.float().numpy(), mems, list(chunks))
    # bf16 output: one rounding of the result on top of the scan's error
    assert_close(y.float().cpu().numpy(), expected, 5e-3, f"d=32 sequence {chunks}")


@pytest.mark.parametrize("chunks", [(5, 16, 64, 3), (65, 128, 100, 17), (128, 128, 128, 128), (200, 40, 7, 33)])
def test_sequence_few_lines_block_form(oracle, device, chunks):
    """Packed bf16 sequences (263 tokens, ragged last chunks) through the few-line block form;
    a chunk of 200 tokens (more than 8 blocks) sends the launch to the wide scan."""
    from visionhope_amd.models.srnl_core.chunk import srnl_packed_forward

    batch, directions, heads, length = 1, 4, 2, 263
    mems = memories(directions, heads, 16, kind="strong", seed=sum(chunks))
    x, q = _packed_case(batch, directions, heads, length, 16, torch.bfloat16, seed=107)
    y = srnl_packed_forward(tuple(torch.from_numpy(m).to(device) for m in mems), x.to(device),
                            q.to(device), list(chunks), q_raw=True)
    expected = oracle.sequence_forward(x.float().numpy(), q.float().numpy(), mems, list(chunks))
    # bf16 output: one rounding of the result on top of the scan's error
    assert_close(y.float().cpu().numpy(), expected, 5e-3, f"few-line sequence {chunks}")


@pytest.mark.parametrize("head_dim,batch,heads,length,chunks", [
    (16, 2, 2, 70, (16, 33, 64, 7)),      # few lines: one workgroup per line
    (16, 64, 4, 24, (8, 16, 12, 24)),     # 1024 lines: lines packed per wave
    (32, 2, 2, 70, (16, 33, 64, 7)),      # head_dim 32 block form
])
def test_sequence_per_line_memories_block_form(oracle, device, head_dim, batch, heads, length, chunks):
    """5-D memories (one state per line, chunk.cu:287) through the bf16 block-form scans;
    the oracle runs each line as a problem of its own with that line's memories."""
    from visionhope_amd.models.srnl_core.chunk import srnl_packed_forward

    directions = 4
    shared = memories(directions, heads, head_dim, kind="perturbed", seed=head_dim + batch)
    gen = np.random.default_rng(head_dim * 7 + batch)
    mems = tuple(np.ascontiguousarray(np.stack([m + 0.05 * gen.standard_normal(m.shape).astype(np.float32)
                                                for _ in range(batch)]), dtype=np.float32) for m in shared)
    x, q = _packed_case(batch, directions, heads, length, head_dim, torch.bfloat16, seed=127 + head_dim)
    y = srnl_packed_forward(tuple(torch.from_numpy(m).to(device) for m in mems), x.to(device), q.to(device),
                            list(chunks), q_raw=True)
    xf, qf = x.float().numpy(), q.float().numpy()
    expected = np.empty((batch, directions, heads, length, head_dim), np.float32)
    for b in range(batch):
        for r in range(directions):
            for h in range(heads):
                line_mems = [m[b, r, h][None, None] for m in mems]
                expected[b, r, h] = oracle.sequence_forward(
                    xf[b:b + 1, r:r + 1, h:h + 1], qf[b:b + 1, r:r + 1, :, h * head_dim:(h + 1) * head_dim],
                    line_mems, [chunks[r]])[0, 0, 0]
    assert_close(y.float().cpu().numpy(), expected, 5e-3, f"per-line memories d={head_dim} lines={batch * directions * heads}")
