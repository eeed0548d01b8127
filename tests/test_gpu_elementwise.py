"""GPU parity of the elementwise kernels (direction fusion, GRN, LayerNorm2d, qnorm,
residual) against the CPU oracle, including the full B=128 elementwise workload."""

import numpy as np
import pytest
import torch

from tests.helpers import assert_close, randn

pytestmark = pytest.mark.gpu

FP32_TOL = 1e-5


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("channels_last", [False, True])
@pytest.mark.parametrize("per_direction", [False, True])
@pytest.mark.parametrize("heads,head_dim,height,width", [(3, 16, 6, 9), (5, 8, 13, 17), (2, 64, 16, 8),
                                                         (1, 4, 5, 3), (8, 16, 7, 10), (4, 32, 5, 6)])
def test_direction_fusion(oracle, device, dtype, channels_last, per_direction, heads, head_dim, height, width):
    """Every fusion kernel (tiled 4x4 channels-last with partial edge tiles and a last chunk
    of fewer heads than the others (8 heads of 16, 4 of 32), scalar NCHW,
    head_dim 4 below the 8-channel vectors) against the oracle."""
    from visionhope_amd.utils.direction_fusion import visionhope_postprocess_scale

    batch = 2
    y = randn(batch, 4, heads, height * width, head_dim, seed=1).to(dtype)
    x = randn(batch, 4, heads, height * width, head_dim, seed=2).to(dtype)
    skip = randn(*((4, heads, head_dim) if per_direction else (heads, head_dim)), seed=3, scale=0.1)
    scale = 1 + randn(4, heads * head_dim, seed=4, scale=0.1)
    out = visionhope_postprocess_scale(y.to(device), x.to(device), skip.to(device), scale.to(device),
                                       height, width, channels_last)
    assert out.dtype == torch.float32
    assert out.is_contiguous(memory_format=torch.channels_last if channels_last else torch.contiguous_format)
    expected = oracle.direction_fusion(y.float().numpy(), x.float().numpy(), skip.numpy(), scale.numpy(),
                                       height, width)
    assert_close(out.cpu().numpy(), expected, FP32_TOL, "fusion")


@pytest.mark.parametrize("shape", [(128, 96, 56, 56), (128, 192, 28, 28)])
def test_config2_full_size(oracle, device, shape):
    """Full-size elementwise workload (B=128, 56x56x96 and 28x28x192): fusion, GRN, LN in bf16."""
    from visionhope_amd.utils.direction_fusion import visionhope_postprocess_scale
    from visionhope_amd.utils.grn_cuda import visionhope_grn
    from visionhope_amd.utils.layer_norm_cuda import visionhope_layernorm2d

    batch, channels, height, width = shape
    heads, head_dim = channels // 16, 16
    gen = torch.Generator(device=device).manual_seed(1234)
    x = torch.randn(batch, height, width, channels, device=device, generator=gen).bfloat16()
    x_nchw = x.permute(0, 3, 1, 2)
    gamma = torch.randn(channels, device=device, generator=gen) * 0.1
    beta = torch.randn(channels, device=device, generator=gen) * 0.1
    w = 1 + torch.randn(channels, device=device, generator=gen) * 0.1
    b = torch.randn(channels, device=device, generator=gen) * 0.1

    y = visionhope_grn(x_nchw, gamma, beta, 1e-6)
    exp = oracle.grn(x_nchw.float().cpu().numpy(), gamma.cpu().numpy(), beta.cpu().numpy())
    assert_close(y.cpu().numpy(), exp, 1e-5, "GRN config 2")
    del y, exp

    y = visionhope_layernorm2d(x_nchw, w, b, 1e-6)
    exp = oracle.layernorm2d(x_nchw.float().cpu().numpy(), w.cpu().numpy(), b.cpu().numpy())
    assert_close(y.cpu().numpy(), exp, 1e-5, "LN config 2")
    del y, exp

    ys = torch.randn(batch, 4, heads, height * width, head_dim, device=device, generator=gen).bfloat16()
    xs = torch.randn(batch, 4, heads, height * width, head_dim, device=device, generator=gen).bfloat16()
    skip = torch.randn(heads, head_dim, device=device, generator=gen) * 0.1
    scale = 1 + torch.randn(4, channels, device=device, generator=gen) * 0.1
    out = visionhope_postprocess_scale(ys, xs, skip, scale, height, width, True)
    exp = oracle.direction_fusion(ys.float().cpu().numpy(), xs.float().cpu().numpy(), skip.cpu().numpy(),
                                  scale.cpu().numpy(), height, width)
    assert_close(out.cpu().numpy(), exp, 1e-5, "fusion config 2")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("channels,height,width", [(96, 7, 5), (256, 14, 14), (7, 3, 3), (2048, 7, 7), (1792, 16, 16), (2560, 9, 7)])
@pytest.mark.parametrize("channels_last", [True, False])
def test_grn(oracle, device, dtype, channels, height, width, channels_last):
    from visionhope_amd.utils.grn import global_response_norm

    x = randn(3, channels, height, width, seed=5).to(dtype)
    if channels_last:
        x = x.contiguous(memory_format=torch.channels_last)
    gamma = randn(1, channels, 1, 1, seed=6, scale=0.1)
    beta = randn(1, channels, 1, 1, seed=7, scale=0.1)
    y = global_response_norm(x.to(device), gamma.to(device), beta.to(device))
    assert y.dtype == torch.float32
    expected = oracle.grn(x.float().numpy(), gamma.numpy(), beta.numpy())
    assert_close(y.cpu().numpy(), expected, 2e-5, "GRN")


def _grn_abi(lib, x, gamma, beta, ws):
    """vh_grn_forward through the C-ABI on a channels-last [B, H, W, C] tensor: y, gx, inv_den."""
    from visionhope_amd.utils import hip

    batch, height, width, channels = x.shape
    y = torch.empty(x.shape, device=x.device, dtype=torch.float32)
    gx = torch.empty(batch, channels, device=x.device)
    inv_den = torch.empty(batch, device=x.device)
    hip.check(lib.vh_grn_forward(hip.ptr(x), hip.dtype_code(x.dtype), hip.ptr(gamma), hip.ptr(beta), hip.ptr(y),
                                 hip.VH_DTYPE_F32, hip.ptr(gx), hip.ptr(inv_den), batch, channels, height, width,
                                 1e-6, hip.ptr(ws), ws.numel() * 4, hip.stream_of(x)), "vh_grn_forward")
    return y, gx, inv_den


def _grn_stats(x):
    """float64 gx and inv_den of a channels-last numpy map (utils/grn.py:26-38)."""
    gx = np.sqrt((x.astype(np.float64) ** 2).sum(axis=(1, 2)))
    return gx, 1.0 / (gx.mean(axis=1) + 1e-6)


@pytest.mark.parametrize("batch,channels,height,width", [(16, 96, 100, 100), (5, 256, 14, 14), (3, 2048, 7, 7),
                                                         (4, 96, 7, 5)])
def test_grn_one_pass_pieces(oracle, device, batch, channels, height, width):
    """The one-pass GRN (x held in registers while the pieces of an image exchange their
    sums of squares) at 60, 4, 7 and 1 pieces per image through the C-ABI: y, gx and
    inv_den against float64, and the workspace's 32 KiB synchronisation header is zero
    again after the call (the contract that lets the next call reuse the workspace)."""
    from visionhope_amd.utils import hip

    lib = hip.load_library()
    gen = torch.Generator(device=device).manual_seed(channels + height)
    x = torch.randn(batch, height, width, channels, device=device, generator=gen).bfloat16()
    gamma = torch.randn(channels, device=device, generator=gen) * 0.1
    beta = torch.randn(channels, device=device, generator=gen) * 0.1
    nbytes = lib.vh_grn_workspace_bytes(batch, channels, height, width)
    ws = torch.zeros((nbytes + 3) // 4, device=device)
    for _ in range(2):   # the second call runs on the counters the first one left
        y, gx, inv_den = _grn_abi(lib, x, gamma, beta, ws)
        torch.cuda.synchronize()
        words = ws[:8192].view(torch.int32)
        assert int(words.abs().sum()) == 0, "synchronisation words not left zero"
        xn = x.float().cpu().numpy()
        want_gx, want_inv = _grn_stats(xn)
        assert_close(gx.cpu().numpy(), want_gx, 1e-5, "gx")
        assert_close(inv_den.cpu().numpy(), want_inv, 1e-5, "inv_den")
        expected = oracle.grn(xn.transpose(0, 3, 1, 2), gamma.cpu().numpy(), beta.cpu().numpy()).transpose(0, 2, 3, 1)
        assert_close(y.cpu().numpy(), expected, 1e-5, "GRN one pass")


def test_grn_one_pass_back_to_back_shapes(oracle, device):
    """Calls with different batch, piece counts and dtypes in a row on one workspace, each
    checked: a small batch followed by a larger one (whose counters must not sit where the
    first call wrote partial sums), and a batch of 300 (two launches of at most 256
    images)."""
    from visionhope_amd.utils.grn_cuda import visionhope_grn

    shapes = [(3, 96, 40, 40, torch.bfloat16), (8, 96, 56, 56, torch.bfloat16), (2, 192, 28, 28, torch.float32),
              (33, 96, 20, 30, torch.float16), (1, 512, 9, 11, torch.bfloat16), (300, 64, 6, 6, torch.bfloat16)]
    for i, (batch, channels, height, width, dtype) in enumerate(shapes):
        x = randn(batch, channels, height, width, seed=40 + i).to(dtype).contiguous(memory_format=torch.channels_last)
        gamma = randn(channels, seed=50 + i, scale=0.1)
        beta = randn(channels, seed=60 + i, scale=0.1)
        y = visionhope_grn(x.to(device), gamma.to(device), beta.to(device), 1e-6)
        expected = oracle.grn(x.float().numpy(), gamma.numpy(), beta.numpy())
        assert_close(y.cpu().numpy(), expected, 2e-5, f"GRN call {i}")


def test_grn_one_pass_graph_replays(device):
    """The one-pass GRN captured in a HIP graph three times over: every replay, with eager
    GRN calls of another shape and synchronisations between replays, equals the eager
    result bit for bit."""
    from visionhope_amd.utils.grn_cuda import visionhope_grn

    gen = torch.Generator(device=device).manual_seed(77)
    x = torch.randn(32, 28, 28, 192, device=device, generator=gen).bfloat16().permute(0, 3, 1, 2)
    other = torch.randn(3, 14, 14, 256, device=device, generator=gen).bfloat16().permute(0, 3, 1, 2)
    gamma = torch.randn(192, device=device, generator=gen) * 0.1
    beta = torch.randn(192, device=device, generator=gen) * 0.1
    g2, b2 = gamma[:128].repeat(2), beta[:128].repeat(2)
    eager = visionhope_grn(x, gamma, beta, 1e-6)
    eager_other = visionhope_grn(other, g2, b2, 1e-6)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = [visionhope_grn(x, gamma, beta, 1e-6) for _ in range(3)]
    for replay in range(3):
        for o in outs:
            o.zero_()
        graph.replay()
        torch.cuda.synchronize()
        for o in outs:
            assert torch.equal(o, eager), f"replay {replay} differs from eager"
        assert torch.equal(visionhope_grn(other, g2, b2, 1e-6), eager_other)
        torch.cuda.synchronize()


def test_grn_one_pass_two_graphs_replayed_in_reverse(device):
    """Two graphs captured one after the other on the same capture stream: replaying the
    second one first, before the first graph ever ran, still gives the eager result (each
    capture creates its own GRN workspace, zeroed by a node of that graph), and so does a
    graph of three calls that share one workspace (each call leaves its words zero)."""
    from visionhope_amd.utils.grn_cuda import visionhope_grn

    gen = torch.Generator(device=device).manual_seed(79)
    x1 = torch.randn(8, 56, 56, 96, device=device, generator=gen).bfloat16().permute(0, 3, 1, 2)
    x2 = torch.randn(16, 28, 28, 192, device=device, generator=gen).bfloat16().permute(0, 3, 1, 2)
    g1, b1 = torch.randn(96, device=device, generator=gen) * 0.1, torch.randn(96, device=device, generator=gen) * 0.1
    g2, b2 = torch.randn(192, device=device, generator=gen) * 0.1, torch.randn(192, device=device, generator=gen) * 0.1
    stream = torch.cuda.Stream(device=device)
    graphs = [torch.cuda.CUDAGraph(), torch.cuda.CUDAGraph()]
    with torch.cuda.graph(graphs[0], stream=stream):
        out1 = visionhope_grn(x1, g1, b1, 1e-6)
    with torch.cuda.graph(graphs[1], stream=stream):
        out2 = [visionhope_grn(x2, g2, b2, 1e-6) for _ in range(3)]
    eager1, eager2 = visionhope_grn(x1, g1, b1, 1e-6), visionhope_grn(x2, g2, b2, 1e-6)
    for _ in range(2):
        for out in (out1, *out2):
            out.zero_()
        graphs[1].replay()
        torch.cuda.synchronize()
        for out in out2:
            assert torch.equal(out, eager2)
        graphs[0].replay()
        torch.cuda.synchronize()
        assert torch.equal(out1, eager1)


def test_grn_one_pass_wait_give_up_is_correct_and_counted(oracle, device, dispatch):
    """Forces every workgroup of the one-pass GRN to stop waiting, from the host and with
    every kernel exiting normally: the image counters are preset so that they never reach
    the piece count, and the wait is cut to 64 sleeps.  Each piece then computes its
    image's statistics from x itself: the output still matches the oracle, the give-ups
    are counted (vh_grn_workspace_fallbacks), and the counters are left zero, so the next
    call, with the default limit, runs the ordinary exchange and gives up nowhere."""
    from visionhope_amd.utils import hip
    from visionhope_amd.utils.grn_cuda import _stream_workspace, grn_wait_fallbacks, visionhope_grn

    batch, channels, height, width = 6, 96, 56, 56
    x = randn(batch, channels, height, width, seed=91).bfloat16().contiguous(memory_format=torch.channels_last)
    gamma, beta = randn(channels, seed=92, scale=0.1), randn(channels, seed=93, scale=0.1)
    expected = oracle.grn(x.float().numpy(), gamma.numpy(), beta.numpy())
    xd, gd, bd = x.to(device), gamma.to(device), beta.to(device)
    lib = hip.load_library()
    ws = _stream_workspace(lib.vh_grn_workspace_bytes(batch, channels, height, width), xd.device)
    before = grn_wait_fallbacks(xd.device)
    words = ws[:8192].view(torch.int32).view(256, 32)
    words[:batch, 0] = -1          # 2^32 - 1: after every piece has counted, pieces - 1 < pieces
    dispatch(grn_spin_limit=64)
    y = visionhope_grn(xd, gd, bd, 1e-6)
    torch.cuda.synchronize()
    assert_close(y.cpu().numpy(), expected, 2e-5, "GRN after give-up")
    gave_up = grn_wait_fallbacks(xd.device) - before
    print(f"[grn] give-ups counted: {gave_up}", flush=True)
    assert gave_up >= batch and gave_up % batch == 0, gave_up
    assert int(words[:, 0].abs().sum()) == 0 and int(words[:, 16].abs().sum()) == 0
    dispatch(grn_spin_limit=1 << 20)
    y = visionhope_grn(xd, gd, bd, 1e-6)
    torch.cuda.synchronize()
    assert_close(y.cpu().numpy(), expected, 2e-5, "GRN after the counters were restored")
    assert grn_wait_fallbacks(xd.device) - before == gave_up


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("channels", [3, 16, 64, 96, 128, 200, 512, 1024, 4096])
@pytest.mark.parametrize("channels_last", [True, False])
def test_layernorm2d(device, dtype, channels, channels_last):
    """Textbook check: torch.nn.functional.layer_norm on CPU in float64."""
    from visionhope_amd.utils.layer_norm_cuda import visionhope_layernorm2d

    x = randn(2, channels, 5, 7, seed=8).to(dtype)
    if channels_last:
        x = x.contiguous(memory_format=torch.channels_last)
    w = 1 + randn(channels, seed=9, scale=0.1)
    b = randn(channels, seed=10, scale=0.1)
    y = visionhope_layernorm2d(x.to(device), w.to(device), b.to(device), 1e-6)
    assert y.dtype == torch.float32
    assert y.is_contiguous(memory_format=torch.channels_last if channels_last else torch.contiguous_format)
    expected = torch.nn.functional.layer_norm(x.double().permute(0, 2, 3, 1), (channels,), w.double(),
                                              b.double(), 1e-6).permute(0, 3, 1, 2)
    assert_close(y.cpu().numpy(), expected.numpy(), 1e-5, "LN")


@pytest.mark.parametrize("head_dim", [4, 8, 16, 32, 64])
def test_qnorm(oracle, device, head_dim):
    from visionhope_amd.utils.query_normalization import visionhope_qnorm

    heads = 3
    q = randn(2, 4, 11, heads * head_dim, seed=12).bfloat16()
    out = visionhope_qnorm(q.to(device), heads, head_dim)
    expected, _ = oracle.qnorm(q.float().numpy(), heads, head_dim)
    assert_close(out.cpu().numpy(), expected, 1e-6, "qnorm")


def test_residual_add(oracle, device):
    from visionhope_amd.utils.residual import visionhope_residual_add

    res = randn(3, 32, 5, 6, seed=13).contiguous(memory_format=torch.channels_last)
    branch = randn(3, 32, 5, 6, seed=14).bfloat16().contiguous(memory_format=torch.channels_last)
    gamma = randn(32, 1, 1, seed=15, scale=0.1)
    out = visionhope_residual_add(res.to(device), branch.to(device), gamma.to(device), 0.0, False)
    expected = oracle.residual_add(res.permute(0, 2, 3, 1).numpy(), branch.float().permute(0, 2, 3, 1).numpy(),
                                   gamma.numpy(), np.ones(3, np.float32))
    assert_close(out.permute(0, 2, 3, 1).cpu().numpy(), expected, 1e-6, "residual")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("channels", [64, 96, 512])
def test_add_layernorm2d(device, dtype, channels):
    """Residual add + LayerNorm2d in one pass: the sum equals torch's add in the same dtype
    bit for bit; the norm matches F.layer_norm (float64) of that sum."""
    from visionhope_amd.utils.layer_norm_cuda import can_fuse_add_layernorm2d, visionhope_add_layernorm2d

    fmt = torch.channels_last
    x = randn(2, channels, 5, 7, seed=21).to(dtype).to(device).contiguous(memory_format=fmt)
    r = randn(2, channels, 5, 7, seed=22).to(dtype).to(device).contiguous(memory_format=fmt)
    w = (1 + randn(channels, seed=23, scale=0.1)).to(device)
    b = randn(channels, seed=24, scale=0.1).to(device)
    assert can_fuse_add_layernorm2d(x, r, w, b)
    s, y = visionhope_add_layernorm2d(x, r, w, b, 1e-6, out_dtype=torch.float32)
    assert torch.equal(s, x + r)
    assert y.is_contiguous(memory_format=fmt)
    expected = torch.nn.functional.layer_norm(s.double().cpu().permute(0, 2, 3, 1), (channels,), w.double().cpu(),
                                              b.double().cpu(), 1e-6).permute(0, 3, 1, 2)
    assert_close(y.cpu().numpy(), expected.numpy(), 1e-5, "add+LN")


@pytest.mark.parametrize("channels", [64, 96])
def test_layernorm2d_bf16_store_is_round_to_nearest_even(device, channels):
    """The kernels store bf16 through the hardware conversion: the bf16 output is the FP32
    output rounded by torch's conversion (nearest even), bit for bit, over a wide range of
    magnitudes (large |w| and tiny |b| put values at every exponent)."""
    from visionhope_amd.utils.layer_norm_cuda import visionhope_layernorm2d

    x = randn(4, channels, 6, 7, seed=31).to(device).contiguous(memory_format=torch.channels_last)
    w = (randn(channels, seed=32) * torch.logspace(-20, 20, channels)).to(device)
    b = (randn(channels, seed=33) * 1e-3).to(device)
    y32 = visionhope_layernorm2d(x, w, b, 1e-6)
    y16 = visionhope_layernorm2d(x, w, b, 1e-6, out_dtype=torch.bfloat16)
    assert y16.dtype == torch.bfloat16
    assert torch.equal(y16.view(torch.int16), y32.to(torch.bfloat16).view(torch.int16))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("act", [0, 1])
def test_bias_act(device, dtype, act):
    """act(round(x + b)) per channel: the folded BatchNorm output and its GELU."""
    from visionhope_amd.utils.conv_bn import bias_act

    x = randn(2, 24, 5, 7, seed=41).to(dtype).contiguous(memory_format=torch.channels_last)
    b = randn(24, seed=42)
    got = bias_act(x.to(device), b.to(device), act)
    y = (x.double() + b.double()[None, :, None, None]).to(dtype).double()
    expected = torch.nn.functional.gelu(y).to(dtype) if act else y.to(dtype)
    assert got.dtype == dtype
    assert_close(got.double().cpu().numpy(), expected.double().numpy(), 1e-5 if dtype == torch.float32 else 4e-3,
                 f"bias_act act={act}")


@pytest.mark.parametrize("autocast", [False, True])
def test_stem_and_downsample_fold_batchnorm(device, autocast):
    """Prepared stem / downsample (BatchNorm folded into the convolution) against the
    same modules unfolded, with BatchNorm statistics far from identity."""
    from visionhope_amd.models.layers import Downsample, PatchEmbedding

    torch.manual_seed(5)
    for mod, x in ((PatchEmbedding(3, 64), randn(2, 3, 32, 32, seed=43)),
                   (Downsample(64, 128), randn(2, 64, 14, 14, seed=44))):
        for m in mod.modules():
            if isinstance(m, torch.nn.BatchNorm2d):
                with torch.no_grad():
                    m.running_mean.copy_(randn(m.num_features, seed=45, scale=0.5))
                    m.running_var.copy_(randn(m.num_features, seed=46).abs() + 0.5)
                    m.weight.copy_(1 + randn(m.num_features, seed=47, scale=0.2))
                    m.bias.copy_(randn(m.num_features, seed=48, scale=0.2))
        mod = mod.to(device).to(memory_format=torch.channels_last).eval()
        xd = x.to(device).contiguous(memory_format=torch.channels_last)
        with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16, enabled=autocast):
            expected = mod(xd)
            mod._vh_fold_bn = True
            got = mod(xd)
            mod._vh_fold_bn = False
        assert got.dtype == expected.dtype and got.shape == expected.shape
        assert_close(got.double().cpu().numpy(), expected.double().cpu().numpy(), 2e-2 if autocast else 1e-5,
                     f"{type(mod).__name__} folded autocast={autocast}")
