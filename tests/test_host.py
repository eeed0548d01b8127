"""Host-side behaviour of the Python mirror: constructors, validation messages, path
selection, inference preparation, weight I/O, environment constants, CPU formulas."""

import os
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

from visionhope_amd.inference.prepare import prepare_for_inference
from visionhope_amd.models import SRNL, VisionHOPEBlock, VisionHOPEOperator, create_model
from visionhope_amd.models.factory import MODEL_CONFIGS, MODEL_REGISTRY
from visionhope_amd.models.layers import LayerNorm2d
from visionhope_amd.tools.checkpoint import load_checkpoint, read_weights, save_weights
from visionhope_amd.utils.grn import GlobalResponseNorm, global_response_norm, grn_reference

ROOT = Path(__file__).resolve().parents[1]


def test_srnl_constructor_validation():
    with pytest.raises(ValueError, match="divisible by head_dim"):
        SRNL(30, head_dim=16)
    with pytest.raises(ValueError, match="divisible by head_dim"):
        SRNL(24, head_dim=12)
    with pytest.raises(ValueError, match="directions must be 1, 2, or 4"):
        SRNL(32, directions=3)
    with pytest.raises(ValueError, match="chunk_size"):
        SRNL(32, chunk_size=0)
    with pytest.raises(TypeError, match="fast_inference"):
        SRNL(32, fast_inference=1)


def test_srnl_parameters_and_default_init():
    torch.manual_seed(0)
    m = SRNL(64, head_dim=16, directions=4)
    assert m.M_m_0.shape == (4, 4, 16, 16) and m.M_eta_0.shape == (4, 4, 16)
    assert torch.all(m.M_eta_0 == 0) and torch.all(m.M_alpha_0 == 0)
    assert 0.005 < m.M_m_0.std().item() < 0.015
    assert m.M_m_0.abs().max().item() <= 2.0
    assert "head_dim=16" in m.extra_repr()
    names = [n for n, _ in m.named_parameters()]
    assert names == ["M_m_0", "M_v_0", "M_k_0", "M_eta_0", "M_alpha_0"]


def test_srnl_path_selection_on_cpu():
    m = SRNL(32, fast_inference=True).eval()
    x = torch.randn(1, 10, 32)
    with torch.no_grad():
        assert m.inference_status(x) == {"path": "ordinary", "reason": "SRNL requires CUDA inputs"}
    assert m.inference_status(x)["reason"] == "Gradients are enabled"
    m.train()
    assert m.inference_status(x)["reason"] == "The module is in training mode"
    with pytest.raises(ValueError, match="same CUDA device"):
        m(x)


def test_srnl_shape_validation():
    m = SRNL(32, directions=1)
    with pytest.raises(ValueError, match=r"\[B, N, dim\]"):
        m(torch.randn(2, 5, 16))
    with pytest.raises(ValueError, match="same shape"):
        m(torch.randn(2, 5, 32), torch.randn(2, 6, 32))


def test_operator_validation_and_path():
    with pytest.raises(ValueError, match="direction_merge"):
        VisionHOPEOperator(32, direction_merge="max")
    with pytest.raises(TypeError):
        VisionHOPEOperator(32, share_direction_skip="yes")
    op = VisionHOPEOperator(32, 16, share_direction_skip=False, direction_merge="softmax")
    assert op.d_skip.shape == (4, 2, 16)
    w = op.direction_weights()
    assert torch.allclose(w.sum(0), torch.full((32,), 4.0))
    op_sum = VisionHOPEOperator(32, 16, direction_merge="sum")
    assert torch.all(op_sum.direction_weights() == 1)
    with pytest.raises(ValueError, match=r"\[B, 32, H, W\]"):
        op(torch.randn(1, 16, 4, 4))
    op.eval()
    with torch.no_grad():
        assert op.inference_status(torch.randn(1, 32, 4, 4))["path"] == "ordinary"


def test_operator_project_queries_and_serialize():
    op = VisionHOPEOperator(8, 4)
    x = torch.randn(2, 8, 3, 5)
    seq_hw = x.flatten(2).transpose(1, 2)
    q = op.project_queries(seq_hw, 3, 5)
    xs = VisionHOPEOperator.serialize(x, seq_hw)
    # every direction's query is W_q applied to that direction's serialized input
    with torch.no_grad():
        np.testing.assert_allclose(q.detach().numpy(), op.W_q(xs).detach().numpy(), rtol=1e-6, atol=1e-6)


def test_block_forces_scale_merge_and_local_modes():
    blk = VisionHOPEBlock(32, head_dim=16, mixer_dim=32)
    assert blk.operator.direction_merge == "scale"
    assert blk.gamma1.shape == (32, 1, 1)
    with pytest.raises(ValueError, match="local_mode"):
        VisionHOPEBlock(32, local_mode="conv")


@pytest.mark.parametrize("name,params_m", [("visionhope_tiny", 26.6), ("visionhope_small", 52.9),
                                           ("visionhope_base", 91.2)])
def test_model_configs_match_published_parameter_counts(name, params_m):
    """Parameter counts published in the reference README (README.md:331-333)."""
    model = create_model(name)
    n = sum(p.numel() for p in model.parameters()) / 1e6
    assert abs(n - params_m) < 0.05, n
    assert name in MODEL_REGISTRY and name in MODEL_CONFIGS


def test_create_model_validation():
    with pytest.raises(ValueError, match="Unknown model"):
        create_model("visionhope_huge")
    with pytest.raises(ValueError, match="checkpoint_path"):
        create_model("visionhope_tiny", pretrained=True)
    with pytest.raises(ValueError, match="Unsupported drop_rate"):
        create_model("visionhope_tiny", drop_rate=0.1)


def test_prepare_for_inference_counts_and_layerscale_fold():
    torch.manual_seed(1)
    model = create_model("visionhope_tiny")
    blk = model.stages[0][0]
    w_before = blk.proj_out.weight.detach().clone()
    g = blk.gamma1.detach().view(-1).clone()
    counts = prepare_for_inference(model)
    assert counts == dict(line_mixer=29, srnl=29, operator=29, layernorm2d=59, grn=29, layerscale=58)
    assert blk.gamma1 is None and blk._inference_prepared
    torch.testing.assert_close(blk.proj_out.weight, w_before * g.view(-1, 1))
    assert all(m.fast_inference for m in model.modules() if isinstance(m, SRNL))
    assert all(m.inference_layout for m in model.modules() if isinstance(m, LayerNorm2d))
    with pytest.raises(RuntimeError, match="folded inference weights"):
        model.train()


def test_checkpoint_roundtrip_native_names(tmp_path):
    torch.manual_seed(2)
    model = create_model("visionhope_tiny")
    path = tmp_path / "w.pth"
    save_weights(path, model.state_dict())
    state = read_weights(path)
    assert "stages.0.0.operator.srnl.M_m_0" in state
    other = create_model("visionhope_tiny")
    load_checkpoint(other, path)
    for (k, a), (_, b) in zip(model.state_dict().items(), other.state_dict().items()):
        assert torch.equal(a, b), k
    torch.save({"model": model.state_dict()}, tmp_path / "bad.pth")
    with pytest.raises(ValueError, match="only 'state_dict'"):
        read_weights(tmp_path / "bad.pth")


def test_environment_constants_are_validated():
    code = "import visionhope_amd.models.srnl_core.chunk"
    env = dict(os.environ, VISIONHOPE_MIN_RETENTION="1.5")
    proc = subprocess.run([sys.executable, "-c", code], cwd=ROOT, env=env, capture_output=True, text=True)
    assert proc.returncode != 0 and "MIN_RETENTION must be in [0, 1)" in proc.stderr
    env = dict(os.environ, VISIONHOPE_STEP_SCALE="abc")
    proc = subprocess.run([sys.executable, "-c", code], cwd=ROOT, env=env, capture_output=True, text=True)
    assert "VISIONHOPE_STEP_SCALE must be a float" in proc.stderr
    env = dict(os.environ, VISIONHOPE_STEP_SCALE="0.05", VISIONHOPE_SPECTRAL_MARGIN="0.5")
    proc = subprocess.run([sys.executable, "-c", code + " as c; c.srnl_consts(); "
                           "k=c.srnl_consts(); print(k.step_scale, k.spectral_factor)"],
                          cwd=ROOT, env=env, capture_output=True, text=True)
    assert proc.returncode == 0 and proc.stdout.split() == ["0.05000000074505806", "1.0"]


def test_grn_module_cpu_matches_oracle(oracle):
    torch.manual_seed(3)
    grn = GlobalResponseNorm(12)
    with torch.no_grad():
        grn.gamma.normal_(0, 0.1)
        grn.beta.normal_(0, 0.1)
    x = torch.randn(2, 12, 5, 4)
    expected = oracle.grn(x.numpy(), grn.gamma.detach().numpy(), grn.beta.detach().numpy())
    np.testing.assert_allclose(grn(x).detach().numpy(), expected, rtol=1e-5, atol=1e-6)
    assert torch.equal(global_response_norm(x, grn.gamma, grn.beta), grn_reference(x, grn.gamma, grn.beta))
    with pytest.raises(ValueError, match="one value per channel"):
        global_response_norm(x, torch.zeros(3), torch.zeros(12))


def test_layernorm2d_cpu_matches_oracle(oracle):
    ln = LayerNorm2d(20)
    with torch.no_grad():
        ln.weight.normal_(1, 0.1)
        ln.bias.normal_(0, 0.1)
    x = torch.randn(2, 20, 3, 3).contiguous(memory_format=torch.channels_last)
    y = ln(x)
    assert y.is_contiguous(memory_format=torch.channels_last)
    expected = oracle.layernorm2d(x.numpy(), ln.weight.detach().numpy(), ln.bias.detach().numpy())
    np.testing.assert_allclose(y.detach().numpy(), expected, rtol=1e-5, atol=1e-5)


def test_parameter_caches_follow_updates():
    from visionhope_amd.utils.cached_params import contiguous_fp32, linear_weights

    p = torch.nn.Parameter(torch.randn(4, 2, 3, 3)).to(memory_format=torch.channels_last)
    c1 = contiguous_fp32(p)
    assert c1.is_contiguous() and torch.equal(c1, p.detach())
    assert contiguous_fp32(p) is c1                 # cached while unchanged
    with torch.no_grad():
        p.mul_(2)
    c2 = contiguous_fp32(p)
    assert torch.equal(c2, p.detach()) and c2 is not c1
    lin = torch.nn.Linear(3, 5)
    w, b = linear_weights(lin, torch.bfloat16)
    assert w.dtype == torch.bfloat16 and torch.equal(w, lin.weight.detach().bfloat16())
    with torch.no_grad():
        lin.bias.add_(1)
    _, b2 = linear_weights(lin, torch.bfloat16)
    assert torch.equal(b2, lin.bias.detach().bfloat16())


def test_invariant_divisor_multiplication_is_exact():
    """The depthwise kernels divide thread indices by launch-invariant divisors with one
    multiplication: m = ceil(2^(32+l) / d), l = ceil(log2 d), floor(n/d) = (n*m) >> (32+l)
    for every n < 2^31.  Brute force over small divisors and dividends, and the extremes
    (the largest dividends, divisors at and around powers of two)."""
    rng = np.random.default_rng(5)

    def magic(d):
        l = (d - 1).bit_length()
        return -(-(1 << (32 + l)) // d), 32 + l

    divisors = list(range(1, 600)) + [(1 << k) + e for k in range(10, 31) for e in (-1, 0, 1)] + [(1 << 31) - 1]
    top = (1 << 31) - 1
    for d in divisors:
        m, shift = magic(d)
        assert m < (1 << 33) + 1
        ns = np.concatenate([np.arange(0, min(4 * d + 3, top), max(1, d // 7)), rng.integers(0, top, 200),
                             [top, top - 1, top - (top % d), top - (top % d) - 1]]).astype(object)
        for n in ns:
            n = int(n)
            assert 0 <= n <= top
            assert (n * m) >> shift == n // d, (n, d)
            assert n * m < (1 << 64)


def _bf16_round(x64):
    """float64 -> nearest-even bfloat16, returned as float64 (finite inputs)."""
    b = np.asarray(x64, dtype=np.float32).view(np.uint32).astype(np.uint64)
    b = (b + 0x7FFF + ((b >> 16) & 1)) >> 16 << 16
    return b.astype(np.uint32).view(np.float32).astype(np.float64)


def test_gelu_table_header_matches_generator(tmp_path):
    """gelu_table.h is what gen_gelu_table.py writes (the committed header is not stale)."""
    import subprocess
    import sys

    csrc = Path(__file__).resolve().parents[1] / "visionhope_amd" / "csrc"
    out = tmp_path / "gelu_table.h"
    subprocess.run([sys.executable, str(csrc / "gen_gelu_table.py"), str(out)], check=True)
    assert out.read_text() == (csrc / "gelu_table.h").read_text()


def _gelu_interp(x32, pairs):
    """gelu_qi in float32 (vh_common.h): s = min(128 |x|, 1024 - 2^-14), i = floor(s),
    f = s - i, Q = fma(f, step[i], value[i]), GELU = fma(-|x|, Q, max(x, 0))."""
    a = np.abs(x32)
    s = np.minimum(a * np.float32(128), np.float32(1024 - 2.0 ** -14)).astype(np.float32)
    i = s.astype(np.int64)
    f = (s - i.astype(np.float32)).astype(np.float32)
    # fma: the float64 product of two float32 values is exact; one rounding to float32
    q = (f.astype(np.float64) * pairs[i, 1] + pairs[i, 0]).astype(np.float32)
    return (np.maximum(x32, 0).astype(np.float64) - a.astype(np.float64) * q).astype(np.float32).astype(np.float64)


def test_gelu_interpolation_table_accuracy():
    """The interpolated GELU of the depthwise kernels (gelu_qi), emulated with the pairs
    parsed from gelu_table.h, against x Phi(x) in float64 (scipy's ndtr) on a dense grid
    of float32 inputs: within 2.3e-6 absolute everywhere and 2.1e-4 relative where
    |GELU| > 1e-6 (the bounds the header states), x/2 near 0, x at large positive x.
    A table shifted by one entry, or with the steps dropped, fails the bounds."""
    import re
    from scipy.special import ndtr

    src = (Path(__file__).resolve().parents[1] / "visionhope_amd" / "csrc" / "gelu_table.h").read_text()
    n = int(re.search(r"GELU_QI_N = ([0-9]+)u", src).group(1))
    body = src.split("gelu_interp_table[2 * GELU_QI_N]")[1].split("{")[1].split("};")[0]
    vals = [float.fromhex(v) for v in re.findall(r"(-?0x[0-9a-fp.+-]+)f,", body)]
    assert n == 1024 and len(vals) == 2 * n
    pairs = np.array(vals, dtype=np.float32).reshape(n, 2).astype(np.float64)
    x32 = np.concatenate([np.linspace(-12, 12, 600001), np.linspace(-1e-3, 1e-3, 2001),
                          np.array([0.0, 7.999, 8.0, 30.0, -7.999, -8.0])]).astype(np.float32)
    x = x32.astype(np.float64)
    exact = x * ndtr(x)

    def errors(table):
        err = np.abs(_gelu_interp(x32, table) - exact)
        big = np.abs(exact) > 1e-6
        return err.max(), (err[big] / np.abs(exact[big])).max()

    ab, rel = errors(pairs)
    assert ab < 2.3e-6 and rel < 2.1e-4, (ab, rel)
    small = (np.abs(x) < 1e-4) & (x != 0)
    assert np.allclose(_gelu_interp(x32[small], pairs), x[small] / 2, rtol=1e-4, atol=0)
    assert _gelu_interp(np.float32([30.0]), pairs)[0] == 30.0
    shifted = np.roll(pairs, 1, axis=0)
    assert errors(shifted)[0] > 1e-3
    no_step = pairs.copy()
    no_step[:, 1] = 0
    assert errors(no_step)[0] > 1e-4


def test_gelu_table_gives_the_bf16_gelu():
    """The device's tabulated GELU (gelu_bf16_tab: fma(-|x|, Q[clamp(|x|)], max(x, 0)) in
    float32 with Q(a) = Phi(-a), then the output rounding to bf16), emulated with the
    entries parsed from gelu_table.h, against the bf16 rounding of x Phi(x) in float64
    (scipy's ndtr) for every finite bf16 x with |x| < 64: equal except where the float64
    value lies within float32 rounding of a bf16 rounding boundary.  Tiny inputs give
    x/2 and |x| >= 8 gives x (positive) or a magnitude below 1e-15 |x| (negative; the
    exact value is below 7e-15)."""
    import re
    from scipy.special import ndtr

    src = (Path(__file__).resolve().parents[1] / "visionhope_amd" / "csrc" / "gelu_table.h").read_text()
    lo, hi, n = (int(v, 0) for v in re.search(r"GELU_TAB_LO = (0x[0-9A-F]+)u, GELU_TAB_HI = (0x[0-9A-F]+)u, "
                                               r"GELU_TAB_N = ([0-9]+)u", src).groups())
    body = src.split("gelu_tail_table[GELU_TAB_N] = {")[1].split("};")[0]
    vals = [float.fromhex(v) for v in re.findall(r"(-?0x[0-9a-fp.+-]+)f,", body)]
    assert n == hi - lo + 1 and len(vals) == n
    tab = np.array(vals, dtype=np.float32)

    def device(table):
        q = table[np.clip(bits & 0x7FFF, lo, hi) - lo].astype(np.float64)
        # fma: the float64 product of two float32 values is exact; one rounding to float32
        r = (np.maximum(x, 0) - np.abs(x) * q).astype(np.float32).astype(np.float64)
        return _bf16_round(r)

    bits = np.arange(0, 0x7F80, dtype=np.uint32)            # +0 .. largest finite bf16 magnitude
    bits = np.concatenate([bits, bits | 0x8000])
    x32 = (bits << 16).view(np.float32)
    keep = np.abs(x32) < 64
    bits, x32 = bits[keep], x32[keep]
    x = x32.astype(np.float64)
    got = device(tab)
    exact = x * ndtr(x)
    want = _bf16_round(exact)
    normal = (np.abs(x) >= 2.0 ** -100) & (x > -8)   # away from float32 subnormals and the far tail
    differ = (got != want) & normal
    # each difference is a one-unit flip at a near tie of the float64 value
    assert differ.mean() < 1e-4, differ.sum()
    gap = np.abs(exact[differ] - 0.5 * (got[differ] + want[differ]))
    assert (gap <= 1e-6 * np.abs(exact[differ]) + 1e-30).all()
    tiny = (np.abs(x) < 2.0 ** -10) & (np.abs(x) >= 2.0 ** -100)
    assert (got[tiny] == _bf16_round(x[tiny] / 2)).all()
    assert (got[x >= 8] == x[x >= 8]).all()
    far = x <= -8
    assert (np.abs(got[far]) <= 1e-15 * np.abs(x[far])).all() and (np.abs(exact[far]) < 7e-15).all()
    # a table shifted by one entry, or Phi(+a) in place of Phi(-a), fails
    assert (device(np.roll(tab, 1)) != want).mean() > 0.05
    assert (device((1 - tab).astype(np.float32)) != want).mean() > 0.05


def test_gelu_fit_accuracy():
    """The device GELU's erfc fit, evaluated step by step in float32 with the constants
    read from the kernel header, against x * Phi(x) in float64 (scipy's ndtr)."""
    import re
    from scipy.special import ndtr

    src = (Path(__file__).resolve().parents[1] / "visionhope_amd" / "csrc" / "vh_common.h").read_text()
    body = src[src.index("float gelu_fast(float x)"):]
    body = body[:body.index("\n}\n")]
    # p = c5; p = p * t -/+ c_k ...: the literals after the first `p = ` in order, with their signs
    lines = [ln.strip() for ln in body.splitlines() if ln.strip().startswith(("float p =", "p = p * t"))]
    coeffs = []
    for ln in lines:
        lit = float(re.search(r"([0-9]+\.[0-9]+)f", ln).group(1))
        coeffs.append(-lit if ("- " in ln.split("=")[1] and "p * t" in ln) else lit)
    assert len(coeffs) == 6
    f32 = np.float32
    x = np.concatenate([np.linspace(-12, 12, 200001), np.linspace(-1e-3, 1e-3, 2001)]).astype(f32)
    t = (f32(1) / (np.abs(x) * f32(0.35355339059327376) + f32(1))).astype(f32)
    p = f32(coeffs[0])
    for c in coeffs[1:]:
        p = (p * t + f32(c)).astype(f32)
    half_erfc = (t * np.exp2((p - (f32(0.72134752044448170) * x) * x).astype(f32))).astype(f32)
    g = (np.maximum(x, f32(0)) - np.abs(x) * half_erfc).astype(f32).astype(np.float64)
    exact = x.astype(np.float64) * ndtr(x.astype(np.float64))
    err = np.abs(g - exact)
    assert err.max() < 2e-6
    big = np.abs(exact) > 1e-6
    assert (err[big] / np.abs(exact[big])).max() < 1.2e-5
    # a dropped or mis-signed coefficient fails the same bound
    for k in range(6):
        bad = list(coeffs)
        bad[k] = -bad[k]
        p = f32(bad[0])
        for c in bad[1:]:
            p = (p * t + f32(c)).astype(f32)
        h = (t * np.exp2((p - (f32(0.72134752044448170) * x) * x).astype(f32))).astype(f32)
        gb = (np.maximum(x, f32(0)) - np.abs(x) * h).astype(f32).astype(np.float64)
        assert np.abs(gb - exact).max() > 1e-3


def test_audit_kernel_families_cover_every_scan_and_readout_kernel():
    """The launch audit counts kernels by name: every scan and readout kernel the library
    defines must belong to exactly one of its families."""
    import re
    from pathlib import Path

    from visionhope_amd.inference.audit import READOUT_KERNELS, SCAN_KERNELS

    csrc = Path(__file__).resolve().parents[1] / "visionhope_amd" / "csrc"
    names = set()
    for path in csrc.glob("*.hip"):
        names.update(re.findall(r"\bvoid\s+(srnl_\w+_kernel)\s*\(", path.read_text()))
    forward = {n for n in names if "backward" not in n}
    assert forward, "no kernels found"
    for name in forward:
        hits = [f for f in SCAN_KERNELS + READOUT_KERNELS if re.fullmatch(re.escape(f), name)]
        assert len(hits) == 1, (name, hits)
