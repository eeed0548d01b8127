"""GPU parity of the matrix-core 1x1 convolution (``vh_pointwise_conv_nhwc_forward``) and
of the GRN statistics entry (``vh_grn_scale_forward``).

The GEMM is checked against the FP64 product of the same bf16 operands, with each fused
step applied to the bf16-rounded value as the reference's autocast graph does; outputs
are bf16, so the bar is a few bf16 roundings (normwise and elementwise 5e-3).  A second
check runs the reference expression itself (``F.linear`` under bf16 autocast).
"""

import pytest
import torch
from torch import nn
from torch.nn import functional as F

from tests.helpers import assert_close, randn

pytestmark = pytest.mark.gpu


def _bf16(t):
    return t.to(torch.bfloat16)


def _linear_ref(x, module):
    """bf16(x W^T + b) in FP64 from the bf16 operands (CPU)."""
    w = module.weight.detach().reshape(module.weight.shape[0], -1).cpu()
    b = module.bias.detach().cpu()
    y = x.double() @ _bf16(w).double().t() + _bf16(b).double()
    return _bf16(y)


@pytest.mark.parametrize("m", [1, 37, 256, 1000])
@pytest.mark.parametrize("k,n", [(64, 32), (32, 32), (128, 64), (96, 128), (256, 128), (64, 256),
                                 (1024, 256), (256, 1024), (512, 384), (2048, 512),
                                 # widths that are multiples of 32 or 64 but not of 128 (Base: 96, 192,
                                 # 224, 320, 448), shallow and deep
                                 (192, 96), (384, 96), (96, 96), (96, 192), (768, 192), (448, 224),
                                 (224, 224), (224, 448), (1792, 448), (640, 320), (320, 320)])
def test_pointwise_bias(device, m, k, n):
    from visionhope_amd.utils import pointwise

    conv = nn.Conv2d(k, n, 1)
    with torch.no_grad():
        conv.weight.copy_(randn(*conv.weight.shape, seed=1, scale=k ** -0.5))
        conv.bias.copy_(randn(n, seed=2, scale=0.5))
    x = _bf16(randn(m, k, seed=3))
    got = pointwise.pointwise_conv(x.to(device), conv.to(device))
    assert got.dtype == torch.bfloat16 and got.shape == (m, n)
    assert_close(got.double().cpu().numpy(), _linear_ref(x, conv).double().numpy(), 5e-3, f"pw M={m} K={k} N={n}")


@pytest.mark.parametrize("k,n", [(64, 256), (256, 1024), (128, 64)])
def test_pointwise_gelu(device, k, n):
    from visionhope_amd.utils import pointwise

    lin = nn.Linear(k, n)
    x = _bf16(randn(3, 7, 11, k, seed=4))
    got = pointwise.pointwise_conv(x.to(device), lin.to(device), pointwise.EPI_GELU)
    expected = _bf16(F.gelu(_linear_ref(x, lin.cpu()).double()))
    assert got.shape == (3, 7, 11, n)
    assert_close(got.double().cpu().numpy(), expected.double().numpy(), 5e-3, "pw gelu")


@pytest.mark.parametrize("k,n,m", [(64, 256, 98309), (128, 512, 40007), (256, 1024, 25088), (192, 128, 70001),
                                   (256, 128, 64 * 512 * 5), (128, 256, 129)])
@pytest.mark.parametrize("epilogue", [0, 1, 3])
def test_pointwise_resident_weights_match_tiled_kernel(device, dispatch, k, n, m, epilogue):
    """The resident-weight kernel (shallow products: weights held in registers, pixel
    tiles streamed through an LDS ring, several tiles per block at these sizes, a ragged
    last tile) accumulates k in the order of the LDS-tiled kernels, so the bf16 outputs
    are identical; both match the FP64 reference."""
    from visionhope_amd.utils import pointwise

    lin = nn.Linear(k, n)
    with torch.no_grad():
        lin.weight.copy_(randn(n, k, seed=71, scale=k ** -0.5))
        lin.bias.copy_(randn(n, seed=72, scale=0.5))
    lin = lin.to(device)
    x = _bf16(randn(m, k, seed=73)).to(device)
    dispatch(pw_resident="2")
    got = pointwise.pointwise_conv(x, lin, epilogue)
    dispatch(pw_resident="0")
    other = pointwise.pointwise_conv(x, lin, epilogue)
    torch.cuda.synchronize()
    assert torch.equal(got, other)
    rows = torch.arange(0, m, max(1, m // 997), device=device)   # a sample of rows against FP64
    ref = _linear_ref(x[rows].cpu(), lin.cpu())
    if epilogue == pointwise.EPI_GELU:
        ref = _bf16(F.gelu(ref.double()))
    elif epilogue == pointwise.EPI_SILU:
        ref = _bf16(F.silu(ref.double()))
    assert_close(got[rows].double().cpu().numpy(), ref.double().numpy(), 5e-3, f"resident K={k} N={n} M={m}")


@pytest.mark.parametrize("k,n", [(256, 64), (1024, 256), (64, 32), (512, 128), (128, 512), (384, 96), (768, 192),
                                 (1792, 448)])
@pytest.mark.parametrize("with_grn", [False, True])
@pytest.mark.parametrize("hw", [(5, 7), (7, 7), (8, 10), (16, 20)])
def test_pointwise_residual_and_grn(device, k, n, with_grn, hw):
    """fc2 of the FFN: r + fc2(GRN(h)), the GRN applied to the operand as it is loaded:
    staged in LDS per k tile with the scale rows of the two images a block can span (320
    pixels; 80 with 64-row blocks) or of three (35, 49 and 80 pixels per image with blocks
    of up to 2x the image), per chunk from global memory when images are smaller still."""
    from visionhope_amd.utils import pointwise

    images, (h, w) = 3, hw
    lin = nn.Linear(k, n)
    x = _bf16(randn(images, h, w, k, seed=5))
    r = _bf16(randn(images, h, w, n, seed=6))
    grn = None
    operand = x
    if with_grn:
        scale = 1 + randn(images, k, seed=7, scale=0.3)
        beta = randn(k, seed=8, scale=0.2)
        grn = (scale.to(device), beta.to(device))
        # The kernel computes x * scale + beta in fp32 with one fused multiply-add; compare
        # against that single rounding (the product is exact in float64), not against
        # torch.addcmul on the CPU, which fuses or not depending on the host's vector path.
        fused = x.double() * scale.double()[:, None, None, :] + beta.double()
        operand = _bf16(fused.float())
    got = pointwise.pointwise_conv(x.to(device), lin.to(device), pointwise.EPI_ADD, residual=r.to(device), grn=grn)
    expected = _bf16(r.double() + _linear_ref(operand, lin.cpu()).double())
    assert_close(got.double().cpu().numpy(), expected.double().numpy(), 5e-3, f"pw add grn={with_grn}")


def test_pointwise_matches_autocast_linear(device):
    """The reference expression: F.linear under bf16 autocast (hipBLASLt), then GELU."""
    from visionhope_amd.utils import pointwise

    lin = nn.Linear(128, 512).to(device)
    x = randn(4, 14, 14, 128, seed=9).to(device)
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        ref = F.gelu(lin(x))
    got = pointwise.pointwise_conv(_bf16(x), lin, pointwise.EPI_GELU)
    assert ref.dtype == got.dtype == torch.bfloat16
    assert_close(got.double().cpu().numpy(), ref.double().cpu().numpy(), 1e-2, "pw vs autocast linear")


def test_pointwise_rejects_unsupported(device):
    from visionhope_amd.utils import pointwise

    with pytest.raises(ValueError):
        pointwise.pointwise_conv(_bf16(randn(4, 48)).to(device), nn.Linear(48, 64).to(device))
    with pytest.raises(ValueError):
        pointwise.pointwise_conv(_bf16(randn(4, 64)).to(device), nn.Linear(64, 48).to(device))
    with pytest.raises(ValueError):
        pointwise.pointwise_conv(randn(4, 64).to(device), nn.Linear(64, 64).to(device))   # fp32 x


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_grn_scale_matches_grn(oracle, device, dtype):
    """x * scale + beta reproduces the GRN output (oracle: utils/grn.py:26-38)."""
    from visionhope_amd.utils.grn_cuda import grn_scale

    x = randn(3, 64, 6, 5, seed=10).to(dtype).contiguous(memory_format=torch.channels_last)
    gamma = randn(64, seed=11, scale=0.2)
    beta = randn(64, seed=12, scale=0.2)
    scale = grn_scale(x.to(device), gamma.to(device), 1e-6)
    assert scale.shape == (3, 64) and scale.dtype == torch.float32
    y = x.float() * scale.cpu()[:, :, None, None] + beta[None, :, None, None]
    expected = oracle.grn(x.float().numpy(), gamma.numpy(), beta.numpy())
    assert_close(y.numpy(), expected, 2e-5, "GRN scale")


@pytest.mark.parametrize("batch,channels,hw", [(8, 384, 64), (2, 1792, 32), (63, 64, 12), (64, 64, 12), (1, 2048, 9)])
def test_grn_scale_few_and_many_images(oracle, device, batch, channels, hw):
    """The statistics of few images (fewer than 64: slab sums spread over channel blocks,
    up to 256 slabs per image) and of many (one workgroup per image) against the oracle."""
    from visionhope_amd.utils.grn_cuda import grn_scale

    x = randn(batch, channels, hw, hw, seed=13).bfloat16().contiguous(memory_format=torch.channels_last)
    gamma = randn(channels, seed=14, scale=0.2)
    beta = randn(channels, seed=15, scale=0.2)
    scale = grn_scale(x.to(device), gamma.to(device), 1e-6)
    y = x.float() * scale.cpu()[:, :, None, None] + beta[None, :, None, None]
    expected = oracle.grn(x.float().numpy(), gamma.numpy(), beta.numpy())
    assert_close(y.numpy(), expected, 2e-5, f"GRN scale B={batch} C={channels} {hw}x{hw}")


@pytest.mark.parametrize("m,k,n", [(25088, 256, 128), (1000, 256, 128), (37, 128, 128), (1, 64, 128),
                                   (100352, 128, 64), (1000, 64, 64), (300, 512, 64),
                                   (401408, 64, 32), (1000, 64, 32), (37, 32, 32), (1, 32, 32)])
def test_pointwise_chain_matches_two_projections(device, m, k, n):
    """``vh_pointwise_chain_nhwc_forward``: out = proj_in(x) and out2 = local_gate(out) in one
    launch.  out has the bits of a separate projection (same tiles, same k order); at
    N = 128 and 32 so does out2 (the separate launch of the N x N product takes the same
    64 x 128 tiles, or the same LDS-free kernel), at N = 64 the separate launch takes the
    LDS-free kernel and the chain 128 x 64 tiles, so out2 is also held to the FP64 product
    of the bf16 operands (one bf16 rounding, 5e-3)."""
    from visionhope_amd.utils import pointwise

    first, second = nn.Linear(k, n), nn.Linear(n, n)
    with torch.no_grad():
        for lin, seed in ((first, 31), (second, 32)):
            lin.weight.copy_(randn(*lin.weight.shape, seed=seed, scale=lin.weight.shape[1] ** -0.5))
            lin.bias.copy_(randn(lin.bias.shape[0], seed=seed + 1, scale=0.1))
    x = _bf16(randn(m, k, seed=33))
    first_d, second_d = first.to(device), second.to(device)
    print(f"\n[case] chain M={m} K={k} N={n}", flush=True)
    xd = x.to(device)
    out, out2 = pointwise.pointwise_chain(xd, first_d, second_d)
    ref1 = pointwise.pointwise_conv(xd, first_d)
    ref2 = pointwise.pointwise_conv(ref1, second_d)
    torch.cuda.synchronize()
    assert torch.equal(out, ref1), "first product differs from the separate projection"
    if n in (32, 128):
        assert torch.equal(out2, ref2), "second product differs from the separate projection"
    expected = _linear_ref(out.cpu(), second)
    assert_close(out2.double().cpu().numpy(), expected.double().numpy(), 5e-3, "chained second product")


def test_pointwise_chain_declines_other_widths(device):
    from visionhope_amd.utils import pointwise

    assert not pointwise.chain_supported(nn.Linear(256, 256), nn.Linear(256, 256))   # N = 256
    assert not pointwise.chain_supported(nn.Linear(96, 128), nn.Linear(128, 128))    # K % 64
    assert not pointwise.chain_supported(nn.Linear(128, 32), nn.Linear(32, 32))      # N = 32 needs K <= 64
    assert not pointwise.chain_supported(nn.Linear(256, 128), nn.Linear(128, 64))    # second not N x N
    assert pointwise.chain_supported(nn.Linear(256, 128), nn.Linear(128, 128))
    with pytest.raises(ValueError):
        pointwise.pointwise_chain(torch.zeros(4, 96, device=device, dtype=torch.bfloat16), nn.Linear(96, 128).to(device),
                                  nn.Linear(128, 128).to(device))


@pytest.mark.parametrize("m,k,n", [(401408, 32, 64), (1000, 64, 64), (100352, 64, 128), (37, 128, 128),
                                   (25088, 128, 256), (1000, 64, 256), (1, 128, 256)])
def test_pointwise_add_layernorm_matches_separate_kernels(device, m, k, n):
    """``vh_pointwise_add_layernorm_nhwc_forward`` (proj_out + residual add + norm2) against
    the projection followed by the channels-last add + LayerNorm kernel: the same bits,
    the LayerNorm sums running in that kernel's order; and against FP64 (two bf16
    roundings of the sum and of the output)."""
    from visionhope_amd.utils import pointwise
    from visionhope_amd.utils.layer_norm_cuda import visionhope_add_layernorm2d

    lin = nn.Linear(k, n)
    with torch.no_grad():
        lin.weight.copy_(randn(n, k, seed=41, scale=k ** -0.5))
        lin.bias.copy_(randn(n, seed=42, scale=0.1))
    x = _bf16(randn(m, k, seed=43))
    res = _bf16(randn(m, n, seed=44))
    lw = 1 + randn(n, seed=45, scale=0.2)
    lb = randn(n, seed=46, scale=0.2)
    lin_d = lin.to(device)
    print(f"\n[case] proj + add + LayerNorm M={m} K={k} N={n}", flush=True)
    xd, rd, lwd, lbd = x.to(device), res.to(device), lw.to(device), lb.to(device)
    s, h = pointwise.pointwise_add_layernorm(xd, lin_d, rd, lwd, lbd, 1e-6)
    branch = pointwise.pointwise_conv(xd, lin_d)
    # the add + LayerNorm kernel on [1, N, 1, M] channels-last views of the same rows
    as_map = lambda t: t.reshape(1, 1, m, n).permute(0, 3, 1, 2)
    s_ref, h_ref = visionhope_add_layernorm2d(as_map(rd), as_map(branch), lwd, lbd, 1e-6, out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    s_ref = s_ref.permute(0, 2, 3, 1).reshape(m, n)
    h_ref = h_ref.permute(0, 2, 3, 1).reshape(m, n)
    ds, dh = (s != s_ref).sum().item(), (h != h_ref).sum().item()
    print(f"[bits] sum differs in {ds}, norm in {dh} of {m * n}", flush=True)
    assert ds == 0 and dh == 0
    s64 = (res.double() + _linear_ref(x, lin).double()).to(torch.bfloat16).double()
    mu = s64.mean(-1, keepdim=True)
    var = ((s64 - mu) ** 2).mean(-1, keepdim=True)
    expected = (s64 - mu) / torch.sqrt(var + 1e-6) * lw.double() + lb.double()
    assert_close(h.double().cpu().numpy(), expected.numpy(), 1e-2, "fused add + LayerNorm")
