"""GPU parity of the fused depthwise kernels and of the fused inference path of a prepared
VisionHOPE block.

The depthwise kernels are checked against PyTorch's FP64 CPU convolution on the same
(rounded) inputs.  The fused block is checked against the same block run on the CPU in
FP32 with the operator computed by the CPU oracle in FP64.
"""

import copy

import pytest
import torch
from torch.nn import functional as F

from tests.helpers import assert_close, oracle_operator, perturb_block, randn

pytestmark = pytest.mark.gpu


def _dw_reference(x, conv, epilogue, gate=None, acc=None):
    """FP64 CPU composition of the fused epilogues on NCHW ``x``."""
    from visionhope_amd.utils import dwconv

    x = x.double().cpu()
    y = F.conv2d(x, conv.weight.detach().double().cpu(),
                 None if conv.bias is None else conv.bias.detach().double().cpu(),
                 padding=conv.padding, groups=conv.groups)
    if epilogue == dwconv.EPI_ADD_INPUT:
        y = x + y
    elif epilogue == dwconv.EPI_GATE:
        y = x + torch.sigmoid(gate.double().cpu()) * y
    elif epilogue == dwconv.EPI_ADD_GELU:
        y = F.gelu(x + y)
    elif epilogue in (dwconv.EPI_ACCUM_F32, dwconv.EPI_ADD_F32_AUX):
        y = acc.double().cpu().permute(0, 3, 1, 2) + y
    return y


@pytest.mark.parametrize("ksize", [3, 5, 7])
@pytest.mark.parametrize("epilogue", [0, 1, 2, 3, 4, 5])
@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-5), (torch.bfloat16, 1e-2)])
@pytest.mark.parametrize("tile", ["0", "2"])
@pytest.mark.parametrize("hw", [(9, 13), (6, 14)])
def test_depthwise_epilogues(device, dispatch, ksize, epilogue, dtype, tol, tile, hw):
    """Both kernels (the per-thread window one, dw_tile="0", and the LDS-tiled one
    wherever it applies, dw_tile="2"; FP32 maps always take the first), on a ragged map
    and on one whose width 7 divides (7 pixels per thread in the window kernel)."""
    from visionhope_amd.utils import dwconv

    dispatch(dw_tile=tile)

    channels = 24
    conv = torch.nn.Conv2d(channels, channels, ksize, padding=ksize // 2, groups=channels)
    with torch.no_grad():
        conv.weight.copy_(randn(*conv.weight.shape, seed=11, scale=0.3))
        conv.bias.copy_(randn(channels, seed=12, scale=0.1))
    conv = conv.to(device)
    h, w = hw
    x = randn(2, channels, h, w, seed=13).to(dtype)
    gate = randn(2, channels, h, w, seed=14).to(dtype)
    acc = randn(2, h, w, channels, seed=15)
    x_dev = x.to(device).contiguous(memory_format=torch.channels_last)
    gate_dev = gate.to(device).contiguous(memory_format=torch.channels_last)
    acc_dev = acc.to(device).contiguous()
    aux = gate_dev if epilogue == 2 else acc_dev if epilogue == 5 else None
    out = dwconv.depthwise_conv(x_dev, conv, epilogue, aux=aux, out=acc_dev if epilogue == 4 else None)
    expected = _dw_reference(x, conv, epilogue, gate=gate, acc=acc)
    if epilogue == dwconv.EPI_ACCUM_F32:
        assert out is acc_dev and out.dtype == torch.float32
        got = out.permute(0, 3, 1, 2)
    else:
        assert out.dtype == dtype and out.is_contiguous(memory_format=torch.channels_last)
        got = out
    assert_close(got.double().cpu().numpy(), expected.numpy(), tol, f"dwconv K={ksize} epi={epilogue}")


@pytest.mark.parametrize("ksize", [3, 5, 7])
@pytest.mark.parametrize("epilogue", [0, 1, 2, 3, 4, 5])
@pytest.mark.parametrize("shape", [(3, 40, 14, 14), (2, 16, 28, 28), (1, 64, 7, 7), (2, 8, 5, 19), (1, 128, 9, 16)])
def test_depthwise_tiled_kernel_matches_window_kernel(device, dispatch, ksize, epilogue, shape):
    """The LDS-tiled kernel accumulates each window in the order of the per-thread one,
    so on bf16 maps the two give identical bits (shapes: Tiny-like maps, a map narrower
    than one segment, rows that do not fill the last band, several channel slabs)."""
    from visionhope_amd.utils import dwconv

    b, c, h, w = shape
    conv = torch.nn.Conv2d(c, c, ksize, padding=ksize // 2, groups=c)
    with torch.no_grad():
        conv.weight.copy_(randn(*conv.weight.shape, seed=61, scale=0.3))
        conv.bias.copy_(randn(c, seed=62, scale=0.1))
    conv = conv.to(device)
    x = randn(b, c, h, w, seed=63).bfloat16().to(device).contiguous(memory_format=torch.channels_last)
    gate = randn(b, c, h, w, seed=64).bfloat16().to(device).contiguous(memory_format=torch.channels_last)
    acc = randn(b, h, w, c, seed=65).to(device)
    aux = gate if epilogue == dwconv.EPI_GATE else acc if epilogue == dwconv.EPI_ADD_F32_AUX else None
    results = []
    for tile in ("0", "2"):
        dispatch(dw_tile=tile)
        out = acc.clone() if epilogue == dwconv.EPI_ACCUM_F32 else None
        results.append(dwconv.depthwise_conv(x, conv, epilogue, aux=aux, out=out))
    torch.cuda.synchronize()
    assert torch.equal(results[0], results[1])


@pytest.mark.parametrize("ksize,epilogue", [(3, 3), (7, 2), (5, 5)])
def test_depthwise_split_launches_match_one_launch(device, dispatch, ksize, epilogue):
    """Inputs above the per-launch buffer limit go in several launches of whole images;
    the result is bit-identical to one launch (the limit is lowered to one image here)."""
    from visionhope_amd.utils import dwconv

    channels, h, w = 16, 6, 11
    conv = torch.nn.Conv2d(channels, channels, ksize, padding=ksize // 2, groups=channels)
    with torch.no_grad():
        conv.weight.copy_(randn(*conv.weight.shape, seed=41, scale=0.3))
        conv.bias.copy_(randn(channels, seed=42, scale=0.1))
    conv = conv.to(device)
    dispatch(dw_tile="0")   # the split applies to the per-thread window kernel
    x = randn(5, channels, h, w, seed=43).bfloat16().to(device).contiguous(memory_format=torch.channels_last)
    gate = randn(5, channels, h, w, seed=44).bfloat16().to(device).contiguous(memory_format=torch.channels_last)
    acc = randn(5, h, w, channels, seed=45).to(device)
    aux = gate if epilogue == dwconv.EPI_GATE else acc if epilogue == dwconv.EPI_ADD_F32_AUX else None
    whole = dwconv.depthwise_conv(x, conv, epilogue, aux=aux)
    dispatch(dw_launch_bytes=str(h * w * channels * 2 + 7))
    split = dwconv.depthwise_conv(x, conv, epilogue, aux=aux)
    torch.cuda.synchronize()
    assert torch.equal(split, whole)


def test_depthwise_without_bias_and_noncontiguous_input(device):
    from visionhope_amd.utils import dwconv

    conv = torch.nn.Conv2d(16, 16, 5, padding=2, groups=16, bias=False)
    with torch.no_grad():
        conv.weight.copy_(randn(*conv.weight.shape, seed=21, scale=0.3))
    conv = conv.to(device)
    x = randn(1, 16, 7, 5, seed=22)
    out = dwconv.depthwise_conv(x.to(device), conv)       # NCHW input is relaid out
    assert_close(out.cpu().numpy(), _dw_reference(x, conv, 0).numpy(), 1e-5, "dwconv no bias")


def test_depthwise_taps_cache_follows_weight_updates(device):
    from visionhope_amd.utils import dwconv

    conv = torch.nn.Conv2d(8, 8, 3, padding=1, groups=8).to(device)
    x = randn(1, 8, 4, 4, seed=31).to(device).contiguous(memory_format=torch.channels_last)
    first = dwconv.depthwise_conv(x, conv)
    with torch.no_grad():
        conv.weight.mul_(2.0)
    second = dwconv.depthwise_conv(x, conv)
    bias = conv.bias.detach().view(1, -1, 1, 1)
    assert_close((second - bias).cpu().numpy(), (2 * (first - bias)).cpu().numpy(), 1e-6, "cache refresh")


def _cpu_block_reference(block, x, oracle):
    """The prepared block on the CPU in FP32, with the operator from the FP64 CPU oracle."""
    with oracle_operator(oracle), torch.no_grad():
        return block(x)


@pytest.mark.parametrize("local_mode", ["gated_dwconv7", "residual_dwconv"])
@pytest.mark.parametrize("autocast", [None, torch.bfloat16, torch.float16])
def test_fused_block_matches_oracle(oracle, device, local_mode, autocast):
    """The fused inference path of a block (FP32, bf16 and fp16 autocast; fp16 takes the
    library GEMM for the 1x1 projections and the fp16 scan and readout kernels) against
    the prepared block on the CPU with the FP64 oracle operator."""
    from visionhope_amd.inference.prepare import prepare_for_inference
    from visionhope_amd.models.block import VisionHOPEBlock

    torch.manual_seed(7)
    block = VisionHOPEBlock(32, head_dim=16, local_mode=local_mode)
    perturb_block(block, seed=8)
    reference = copy.deepcopy(block)
    prepare_for_inference(reference)
    gpu = block.to(device).to(memory_format=torch.channels_last)
    prepare_for_inference(gpu)
    x = randn(2, 32, 9, 11, seed=9)
    expected = _cpu_block_reference(reference, x, oracle).numpy()

    x_dev = x.to(device).contiguous(memory_format=torch.channels_last)
    with torch.no_grad(), torch.autocast("cuda", dtype=autocast or torch.bfloat16, enabled=autocast is not None):
        if autocast is not None:
            x_dev = x_dev.to(autocast)
        assert gpu._fused_eligible(x_dev)
        out = gpu(x_dev)
    assert out.dtype == (autocast or torch.float32)
    assert out.is_contiguous(memory_format=torch.channels_last)
    # FP32 tolerance 1e-4; bf16 / fp16 autocast tolerance 2e-2, both normwise and elementwise.
    assert_close(out.double().cpu().numpy(), expected, 2e-2 if autocast is not None else 1e-4,
                 f"fused block {local_mode} autocast={autocast}")


@pytest.mark.parametrize("dim", [32, 64, 128])
@pytest.mark.parametrize("native_gemm", [False, True])
def test_fused_block_bf16_gemm_paths(oracle, device, monkeypatch, dim, native_gemm):
    """bf16 autocast through either 1x1 path: the native matrix-core kernel for every
    projection (fc1 + GELU, fc2 with the GRN apply and the residual add fused), or the
    library GEMM with separate elementwise passes (the path of shapes the kernel does not
    cover)."""
    from visionhope_amd.inference.prepare import prepare_for_inference
    from visionhope_amd.models import block as block_mod
    from visionhope_amd.models.block import VisionHOPEBlock

    if not native_gemm:
        monkeypatch.setattr(block_mod, "_matrix_core_ok", lambda t, module, grn_prologue=False: False)
    torch.manual_seed(17)
    block = VisionHOPEBlock(dim, head_dim=16)
    perturb_block(block, seed=18)
    reference = copy.deepcopy(block)
    prepare_for_inference(reference)
    gpu = block.to(device).to(memory_format=torch.channels_last)
    prepare_for_inference(gpu)
    x = randn(3, dim, 7, 12, seed=19)
    expected = _cpu_block_reference(reference, x, oracle).numpy()
    x_dev = x.to(device).contiguous(memory_format=torch.channels_last).bfloat16()
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        out = gpu(x_dev)
    assert out.dtype == torch.bfloat16
    assert_close(out.double().cpu().numpy(), expected, 2e-2, f"fused block dim={dim} native={native_gemm}")


def test_fused_block_falls_back_for_odd_layouts(device):
    from visionhope_amd.inference.prepare import prepare_for_inference
    from visionhope_amd.models.block import VisionHOPEBlock

    block = VisionHOPEBlock(32, head_dim=16)
    perturb_block(block, seed=10)
    block = block.to(device)
    prepare_for_inference(block)
    x = torch.randn(1, 32, 6, 6, device=device)                 # NCHW storage
    assert not block._fused_eligible(x)
    assert block._fused_eligible(x.contiguous(memory_format=torch.channels_last))
    with torch.no_grad():
        a = block(x)
        b = block(x.contiguous(memory_format=torch.channels_last))
    assert_close(a.cpu().numpy(), b.cpu().numpy(), 1e-4, "fused vs ordinary block")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("shape", [(2, 64, 16, 16), (3, 256, 8, 24), (2, 1024, 14, 14)])
@pytest.mark.parametrize("ksize,tile", [(3, "1"), (7, "1"), (3, "2")])
def test_depthwise_gelu_grn_statistics(device, dispatch, dtype, shape, ksize, tile):
    """The FFN middle with GRN statistics taken in the depthwise pass: the map equals the
    plain fused depthwise + GELU (same arithmetic) and the scale matches the separate GRN
    statistics pass on that map (FP32 sums in another order)."""
    from visionhope_amd.utils import dwconv
    from visionhope_amd.utils.grn_cuda import grn_scale

    dispatch(dw_tile=tile)
    b, c, h, w = shape
    conv = torch.nn.Conv2d(c, c, ksize, padding=ksize // 2, groups=c)
    with torch.no_grad():
        conv.weight.copy_(randn(*conv.weight.shape, seed=51, scale=0.3))
        conv.bias.copy_(randn(c, seed=52, scale=0.1))
    conv = conv.to(device)
    gamma = randn(c, seed=53, scale=0.3).to(device)
    x = randn(b, c, h, w, seed=54).to(dtype).to(device).contiguous(memory_format=torch.channels_last)
    fused = dwconv.depthwise_conv_gelu_grn(x, conv, gamma, 1e-6)
    assert fused is not None
    out, scale = fused
    plain = dwconv.depthwise_conv(x, conv, dwconv.EPI_ADD_GELU)
    assert torch.equal(out, plain)
    assert_close(scale.cpu().numpy(), grn_scale(plain, gamma, 1e-6).cpu().numpy(), 1e-5, "fused GRN scale")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("shape", [(2, 768, 16, 16), (2, 1792, 8, 8), (2, 768, 64, 64), (3, 384, 10, 16),
                                   (2, 384, 128, 128), (1, 256, 14, 14), (2, 96, 8, 8)])
def test_depthwise_gelu_grn_statistics_whole_group_blocks(device, dtype, shape):
    """Blocks of whole channel groups other than 256 threads (Base: 768, 1792 and 384 FFN
    channels in blocks of 192, 224 and 192 threads; 256 channels on 14 x 14 in blocks of 7
    segments; 96 channels), and few images with many slabs (the spread statistics: 256 and
    512 slabs per image): the map equals the plain fused depthwise + GELU and the scale
    matches the separate GRN statistics pass."""
    from visionhope_amd.utils import dwconv
    from visionhope_amd.utils.grn_cuda import grn_scale

    b, c, h, w = shape
    conv = torch.nn.Conv2d(c, c, 3, padding=1, groups=c)
    with torch.no_grad():
        conv.weight.copy_(randn(*conv.weight.shape, seed=61, scale=0.3))
        conv.bias.copy_(randn(c, seed=62, scale=0.1))
    conv = conv.to(device)
    gamma = randn(c, seed=63, scale=0.3).to(device)
    x = randn(b, c, h, w, seed=64).to(dtype).to(device).contiguous(memory_format=torch.channels_last)
    print(f"\n[case] dwconv + GRN sums {dtype} {shape}", flush=True)
    fused = dwconv.depthwise_conv_gelu_grn(x, conv, gamma, 1e-6)
    assert fused is not None
    out, scale = fused
    plain = dwconv.depthwise_conv(x, conv, dwconv.EPI_ADD_GELU)
    assert torch.equal(out, plain)
    assert_close(scale.cpu().numpy(), grn_scale(plain, gamma, 1e-6).cpu().numpy(), 1e-5, "fused GRN scale")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("shape", [(2, 64, 56, 56), (3, 128, 28, 28), (2, 256, 14, 14), (4, 256, 7, 7),
                                   (2, 128, 9, 13), (2, 8, 5, 6), (1, 32, 1, 17)])
def test_depthwise_add_layernorm_matches_separate_kernels(device, dtype, shape):
    """The block's CPE with norm1 in one pass gives the bits of the depthwise CPE kernel
    followed by the channels-last LayerNorm kernel (same sums in the same lane order)."""
    from visionhope_amd.utils import dwconv
    from visionhope_amd.utils.layer_norm_cuda import visionhope_layernorm2d

    b, c, h, w = shape
    conv = torch.nn.Conv2d(c, c, 3, padding=1, groups=c)
    with torch.no_grad():
        conv.weight.copy_(randn(*conv.weight.shape, seed=91, scale=0.3))
        conv.bias.copy_(randn(c, seed=92, scale=0.1))
    conv = conv.to(device)
    weight = (1 + randn(c, seed=93, scale=0.2)).to(device)
    bias = randn(c, seed=94, scale=0.1).to(device)
    x = randn(b, c, h, w, seed=95, scale=2.0).to(dtype).to(device).contiguous(memory_format=torch.channels_last)
    fused = dwconv.depthwise_conv_add_layernorm(x, conv, weight, bias, 1e-6)
    assert fused is not None
    y, yn = fused
    ref_y = dwconv.depthwise_conv(x, conv, dwconv.EPI_ADD_INPUT)
    with torch.no_grad():
        ref_n = visionhope_layernorm2d(ref_y, weight, bias, 1e-6, force_channels_last=True, out_dtype=dtype)
    assert y.dtype == yn.dtype == dtype
    assert torch.equal(y, ref_y)
    assert torch.equal(yn, ref_n), (yn.float() - ref_n.float()).abs().max().item()


def test_depthwise_add_layernorm_declines_uncovered_shapes(device):
    from visionhope_amd.utils import dwconv

    for c in (96, 512):
        conv = torch.nn.Conv2d(c, c, 3, padding=1, groups=c).to(device)
        x = torch.zeros(1, c, 4, 4, device=device, dtype=torch.bfloat16).contiguous(memory_format=torch.channels_last)
        ones = torch.ones(c, device=device)
        assert dwconv.depthwise_conv_add_layernorm(x, conv, ones, ones, 1e-6) is None


def test_depthwise_gelu_grn_declines_uncovered_shapes(device):
    from visionhope_amd.utils import dwconv

    # 2,560 channels: 320 groups of 8, more than one block of 256 threads holds
    conv = torch.nn.Conv2d(2560, 2560, 3, padding=1, groups=2560).to(device)
    x = torch.randn(1, 2560, 7, 7, device=device).contiguous(memory_format=torch.channels_last)
    assert dwconv.depthwise_conv_gelu_grn(x, conv, torch.ones(2560, device=device), 1e-6) is None
