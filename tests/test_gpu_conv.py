"""GPU parity of the 3x3 implicit-GEMM convolution (stem and downsample layers) against
an FP64 convolution of the same bf16-rounded operands."""

import pytest
import torch
from torch import nn
from torch.nn import functional as F

from tests.helpers import assert_close, randn

pytestmark = pytest.mark.gpu

BF16_TOL = 8e-3   # one bf16 rounding of the sum (2^-9 relative) plus one of the GELU output


def _reference(x, weight, bias, stride, act):
    """FP64 conv of bf16-rounded x and weight, + bias, rounded to bf16 after the sum and
    after the activation (the kernel's rounding points)."""
    xr = x.to(torch.bfloat16).double()
    wr = weight.to(torch.bfloat16).double()
    y = F.conv2d(xr, wr, None, stride, 1) + bias.double()[None, :, None, None]
    y = y.to(torch.bfloat16).double()
    if act:
        y = F.gelu(y).to(torch.bfloat16).double()
    return y


@pytest.mark.parametrize("cin,cout,stride,hw,act,in_dtype", [
    (3, 32, 2, (32, 32), 1, torch.float32),     # first stem conv, fp32 image
    (3, 32, 2, (17, 23), 1, torch.bfloat16),    # odd map, bf16 image
    (3, 64, 2, (9, 12), 0, torch.float32),
    (32, 32, 1, (16, 16), 1, torch.bfloat16),
    (32, 64, 2, (15, 13), 1, torch.bfloat16),
    (64, 64, 1, (14, 14), 0, torch.bfloat16),
    (64, 128, 2, (14, 14), 0, torch.bfloat16),  # downsample 1
    (96, 128, 1, (7, 9), 1, torch.bfloat16),    # Cin % 64 != 0 with k tiles of 32
    (128, 256, 2, (10, 10), 0, torch.bfloat16),
    (256, 512, 2, (7, 7), 0, torch.bfloat16),   # downsample 3 at 14 -> 7 shape class
    (3, 96, 2, (20, 18), 1, torch.float32),     # N = 96: BN = 32 tiles
    (96, 96, 1, (11, 10), 0, torch.bfloat16),   # Base stem, last conv
    (96, 192, 2, (12, 12), 0, torch.bfloat16),  # Base downsamples: N % 64 == 0 (BN = 64)
    (192, 448, 2, (8, 9), 0, torch.bfloat16),
    (448, 640, 2, (6, 6), 0, torch.bfloat16),
])
def test_conv3x3(device, cin, cout, stride, hw, act, in_dtype):
    from visionhope_amd.utils.conv_bn import conv3x3_bias_act

    conv = nn.Conv2d(cin, cout, 3, stride=stride, padding=1)
    x = randn(3, cin, *hw, seed=61)
    weight = randn(cout, cin, 3, 3, seed=62, scale=(9 * cin) ** -0.5)
    bias = randn(cout, seed=63, scale=0.5)
    xd = x.to(in_dtype).to(device).contiguous(memory_format=torch.channels_last)
    wd = weight.to(device).contiguous(memory_format=torch.channels_last)
    got = conv3x3_bias_act(xd, conv, wd, bias.to(device), act)
    expected = _reference(x, weight, bias, stride, act)
    assert got.dtype == torch.bfloat16 and got.shape == expected.shape
    assert got.is_contiguous(memory_format=torch.channels_last)
    assert_close(got.double().cpu().numpy(), expected.numpy(), BF16_TOL,
                 f"conv3x3 cin={cin} cout={cout} s={stride} hw={hw} act={act}")


@pytest.mark.parametrize("batch,cin,cout,stride,hw,act,in_dtype", [
    (2, 3, 32, 2, (224, 224), 1, torch.float32),    # Tiny stem, first convolution
    (2, 3, 64, 2, (9, 12), 0, torch.bfloat16),
    (2, 32, 32, 1, (112, 112), 1, torch.bfloat16),  # stem convolution 2
    (2, 32, 64, 2, (112, 112), 1, torch.bfloat16),  # stem convolution 3
    (2, 64, 64, 1, (56, 56), 0, torch.bfloat16),    # stem convolution 4
    (2, 64, 128, 2, (56, 56), 0, torch.bfloat16),   # downsample 1
    (3, 32, 32, 1, (13, 29), 0, torch.bfloat16),    # tiles across row ends, partial last band
    (3, 64, 96, 2, (15, 17), 1, torch.bfloat16),    # odd map at stride 2, three 32-channel slices
    (2, 32, 64, 1, (1, 1), 1, torch.bfloat16),      # one pixel: every neighbour in the padding
    (1, 64, 64, 1, (97, 5), 0, torch.bfloat16),     # narrow, tall map
])
def test_conv3x3_band_kernel_matches_tiled_kernel(device, dispatch, batch, cin, cout, stride, hw, act, in_dtype):
    """The band kernel (input rows staged in LDS once per band, weights in registers) runs
    the products in the tiled kernel's k order with the same operands, so both give the
    same bits; the conv_band override "0" selects the tiled kernel."""
    from visionhope_amd.utils.conv_bn import conv3x3_bias_act

    conv = nn.Conv2d(cin, cout, 3, stride=stride, padding=1)
    x = randn(batch, cin, *hw, seed=81).to(in_dtype).to(device).contiguous(memory_format=torch.channels_last)
    wd = randn(cout, cin, 3, 3, seed=82, scale=(9 * cin) ** -0.5).to(device).contiguous(memory_format=torch.channels_last)
    bias = randn(cout, seed=83, scale=0.5).to(device)
    dispatch(conv_band="1")
    band = conv3x3_bias_act(x, conv, wd, bias, act)
    dispatch(conv_band="0")
    tiled = conv3x3_bias_act(x, conv, wd, bias, act)
    assert torch.equal(band, tiled), f"band vs tiled: max diff {(band.float() - tiled.float()).abs().max().item()}"
    if hw[0] * hw[1] <= 4096:
        expected = _reference(x.float().cpu(), wd.float().cpu(), bias.cpu(), stride, act)
        assert_close(band.double().cpu().numpy(), expected.numpy(), BF16_TOL, "band kernel vs fp64")


def test_conv3x3_cached_weight_follows_the_folded_weight(device):
    """The GEMM operand is rebuilt when the folded weight changes."""
    from visionhope_amd.utils.conv_bn import conv3x3_bias_act

    conv = nn.Conv2d(32, 32, 3, padding=1)
    x = randn(1, 32, 8, 8, seed=64).to(torch.bfloat16).to(device).contiguous(memory_format=torch.channels_last)
    bias = torch.zeros(32, device=device)
    w1 = randn(32, 32, 3, 3, seed=65, scale=0.05).to(device).contiguous(memory_format=torch.channels_last)
    w2 = -w1
    y1 = conv3x3_bias_act(x, conv, w1, bias)
    y2 = conv3x3_bias_act(x, conv, w2, bias)
    assert torch.equal(y1.float(), -y2.float())


def test_conv3x3_rejects(device):
    from visionhope_amd.utils import hip

    lib = hip.load_library()
    x = torch.zeros(1, 8, 8, 48, device=device, dtype=torch.bfloat16)
    w = torch.zeros(64, 9 * 48, device=device, dtype=torch.bfloat16)
    b = torch.zeros(64, device=device)
    out = torch.zeros(1, 8, 8, 64, device=device, dtype=torch.bfloat16)
    s = hip.stream_of(x)
    bf16 = hip.VH_DTYPE_BF16
    # in_channels 48 is neither 3 nor a multiple of 32
    assert lib.vh_conv3x3_nhwc_forward(hip.ptr(x), bf16, hip.ptr(w), hip.ptr(b), 0, hip.ptr(out),
                                       1, 8, 8, 48, 64, 1, s) != 0
    # stride 3
    assert lib.vh_conv3x3_nhwc_forward(hip.ptr(x), bf16, hip.ptr(w), hip.ptr(b), 0, hip.ptr(out),
                                       1, 8, 8, 32, 64, 3, s) != 0
    # out_channels 48 (not a multiple of 32)
    assert lib.vh_conv3x3_nhwc_forward(hip.ptr(x), bf16, hip.ptr(w), hip.ptr(b), 0, hip.ptr(out),
                                       1, 8, 8, 32, 48, 1, s) != 0
    # fp32 map with 32 channels
    assert lib.vh_conv3x3_nhwc_forward(hip.ptr(x), hip.VH_DTYPE_F32, hip.ptr(w), hip.ptr(b), 0, hip.ptr(out),
                                       1, 8, 8, 32, 64, 1, s) != 0
    assert "conv3x3" in lib.vh_last_error().decode()


def test_prepared_stem_uses_native_conv(device, monkeypatch):
    """Under bf16 autocast the folded stem and downsample run every 3x3 convolution through
    the native kernel (no library convolution)."""
    from visionhope_amd.models.layers import Downsample, PatchEmbedding

    calls = []
    real_conv2d = F.conv2d
    monkeypatch.setattr(F, "conv2d", lambda *a, **k: calls.append(1) or real_conv2d(*a, **k))
    for mod, x in ((PatchEmbedding(3, 64), randn(2, 3, 32, 32, seed=66)),
                   (Downsample(64, 128), randn(2, 64, 14, 14, seed=67))):
        mod = mod.to(device).to(memory_format=torch.channels_last).eval()
        mod._vh_fold_bn = True
        xd = x.to(device).contiguous(memory_format=torch.channels_last)
        if isinstance(mod, Downsample):
            xd = xd.to(torch.bfloat16)
        with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
            y = mod(xd)
        assert y.dtype == torch.bfloat16
    assert not calls


def test_fused_classifier_head(device):
    """LayerNorm -> 1x1 conv -> BatchNorm -> SiLU -> mean with the BatchNorm folded and the
    SiLU in the GEMM epilogue, against the same modules run one by one under autocast."""
    from visionhope_amd.models.hierarchical import HierarchicalVisionHOPE

    torch.manual_seed(7)
    model = HierarchicalVisionHOPE(embed_dims=(32, 32, 64, 128), mixer_dims=(32, 32, 32, 64),
                                   depths=(1, 1, 1, 1), projection_dim=256, num_classes=10)
    bn = model.head_norm
    with torch.no_grad():
        bn.running_mean.copy_(randn(256, seed=68, scale=0.5))
        bn.running_var.copy_(randn(256, seed=69).abs() + 0.5)
        bn.weight.copy_(1 + randn(256, seed=70, scale=0.2))
        bn.bias.copy_(randn(256, seed=71, scale=0.2))
        model.norm.weight.copy_(1 + randn(128, seed=72, scale=0.1))
    model = model.to(device).to(memory_format=torch.channels_last).eval()
    x = randn(3, 128, 7, 7, seed=73).to(device).to(torch.bfloat16).contiguous(memory_format=torch.channels_last)
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        expected = model.head_act(model.head_norm(model.head_pre_logits(model.norm(x)))).mean(dim=[2, 3])
        model._vh_fold_head = True
        assert model._fused_head_ok(x)
        got = model._fused_head(x)
    assert got.dtype == expected.dtype and got.shape == expected.shape
    assert_close(got.double().cpu().numpy(), expected.double().cpu().numpy(), 2e-2, "fused head")


@pytest.mark.parametrize("embed_dim", [96, 80])
def test_prepared_base_stem_pads_narrow_widths(device, monkeypatch, embed_dim):
    """A stem whose inner widths are not multiples of 32 (Base: 48, here also 40) runs every
    convolution natively on zero-padded channels when its output width allows (96), or
    falls back to the library for the convolutions it cannot pad (80); either way it matches
    the unfolded stem under bf16 autocast."""
    import copy

    from visionhope_amd.models.layers import PatchEmbedding

    torch.manual_seed(3)
    ref = PatchEmbedding(3, embed_dim).to(device).to(memory_format=torch.channels_last).eval()
    with torch.no_grad():
        for m in ref.modules():
            if isinstance(m, nn.BatchNorm2d):
                m.running_mean.normal_(0, 0.1)
                m.running_var.uniform_(0.5, 1.5)
                m.weight.normal_(1, 0.1)
                m.bias.normal_(0, 0.1)
    folded = copy.deepcopy(ref)
    folded._vh_fold_bn = True
    x = randn(2, 3, 40, 36, seed=71).to(device).contiguous(memory_format=torch.channels_last)
    calls = []
    real_conv2d = F.conv2d
    monkeypatch.setattr(F, "conv2d", lambda *a, **k: calls.append(1) or real_conv2d(*a, **k))
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        got = folded(x)
    monkeypatch.setattr(F, "conv2d", real_conv2d)
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        want = ref(x)
    assert got.shape == want.shape == (2, embed_dim, 10, 9)
    if embed_dim == 96:
        assert not calls, "the padded Base stem should not call the library convolution"
    assert_close(got.float().cpu().numpy(), want.float().cpu().numpy(), 2e-2, f"stem {embed_dim}")
