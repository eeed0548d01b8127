"""The C ABI library: it loads, exports every symbol the public header declares, and
rejects invalid arguments on the host (before any GPU work) with status codes and
messages.  No kernel runs here: every call below fails validation first."""

import ctypes
import re
import subprocess
from pathlib import Path

import pytest

from visionhope_amd.utils import hip

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "visionhope_hip.h"


def _declared():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w[\w\s\*]*?\b(vh_\w+)\s*\(", text, re.M)))


@pytest.fixture(scope="module")
def lib():
    return hip.load_library()


def test_header_declares_expected_entry_points():
    assert set(_declared()) == set(hip.EXPORTED_SYMBOLS)


def test_library_exports_every_declared_symbol(lib):
    out = subprocess.run(["nm", "-D", "--defined-only", str(hip.LIB_PATH)], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r" T (vh_\w+)$", out, re.M))
    missing = set(_declared()) - exported
    assert not missing, missing
    for name in _declared():
        assert getattr(lib, name) is not None


def test_library_is_gfx950_and_links_one_hip_runtime():
    out = subprocess.run(["readelf", "-d", str(hip.LIB_PATH)], capture_output=True, text=True,
                         check=True).stdout
    assert "libamdhip64.so" in out
    blob = hip.LIB_PATH.read_bytes()
    assert b"gfx950" in blob


def test_abi_version_matches_header(lib):
    version = int(re.search(r"#define VH_ABI_VERSION (\d+)", HEADER.read_text()).group(1))
    assert lib.vh_abi_version() == version


def test_workspace_queries(lib):
    assert lib.vh_srnl_workspace_bytes(10, 7, 16) == 10 * 7 * 16 * 16 * 4
    assert lib.vh_srnl_workspace_bytes(0, 7, 16) == 0
    # 100 pixels, B=2: the 32 KiB synchronisation header, then the partial sums of the
    # two-pass statistics, which split each image into 13 slabs of 8 pixels (the one-pass
    # kernel needs one piece per image here)
    assert lib.vh_grn_workspace_bytes(2, 8, 10, 10) == 32768 + 2 * 13 * 8 * 4
    # 56x56x96, B=128: the scalar statistics' 49 slabs of 64 pixels exceed the one-pass
    # kernel's 19 pieces of 21 x 8 rows
    assert lib.vh_grn_workspace_bytes(128, 96, 56, 56) == 32768 + 128 * 49 * 96 * 4


def _consts():
    return hip.make_consts(0.025, 0.0, 2.197224577, 0.999, True, 0.999999)


def _spatial(lib, head_dim=16, dtype=hip.VH_DTYPE_BF16, workspace=4096, x=1, chunks=(4, 4, 4, 4),
             consts=None):
    p = ctypes.c_void_p(0x1000)
    arr, keep = hip.int64_array(chunks)
    return lib.vh_srnl_spatial_forward(
        ctypes.c_void_p(x) if x else None, p, dtype, p, p, p, p, p, p, 0, p, p,
        2, 4, 4, 2 * head_dim if head_dim else 32, head_dim, arr,
        consts if consts is not None else _consts(), p, workspace, None)


def test_srnl_rejects_bad_head_dim(lib):
    assert _spatial(lib, head_dim=12) == hip.VH_ERR_HEAD_DIM
    assert b"head_dim" in lib.vh_last_error()


def test_srnl_rejects_bad_dtype(lib):
    assert _spatial(lib, dtype=7) == hip.VH_ERR_DTYPE


def test_srnl_rejects_small_workspace(lib):
    assert _spatial(lib, workspace=16) == hip.VH_ERR_WORKSPACE
    assert b"workspace" in lib.vh_last_error()


def test_srnl_rejects_null_input(lib):
    assert _spatial(lib, x=0) == hip.VH_ERR_ARG


def test_srnl_rejects_bad_chunks_and_constants(lib):
    assert _spatial(lib, chunks=(4, 0, 4, 4)) == hip.VH_ERR_ARG
    bad = hip.make_consts(0.025, 1.5, 2.197224577, 0.999, True, 0.999999)
    assert _spatial(lib, consts=bad) == hip.VH_ERR_ARG
    assert b"MIN_RETENTION" in lib.vh_last_error()


def test_grn_rejects_missing_workspace(lib):
    p = ctypes.c_void_p(0x1000)
    rc = lib.vh_grn_forward(p, hip.VH_DTYPE_BF16, p, p, p, hip.VH_DTYPE_F32, p, p, 2, 8, 4, 4, 1e-6, None, 0,
                            None)
    assert rc == hip.VH_ERR_WORKSPACE


def test_layernorm_rejects_empty(lib):
    p = ctypes.c_void_p(0x1000)
    rc = lib.vh_layernorm2d_forward(p, hip.VH_DTYPE_F32, p, p, p, hip.VH_DTYPE_F32, None, None, 0, 8, 4, 4, 1e-6,
                                    1, None)
    assert rc == hip.VH_ERR_SHAPE


def test_layernorm_and_grn_reject_bad_output_dtype(lib):
    p = ctypes.c_void_p(0x1000)
    rc = lib.vh_layernorm2d_forward(p, hip.VH_DTYPE_F32, p, p, p, 9, None, None, 2, 8, 4, 4, 1e-6, 1, None)
    assert rc == hip.VH_ERR_DTYPE
    rc = lib.vh_grn_forward(p, hip.VH_DTYPE_BF16, p, p, p, 9, p, p, 2, 8, 4, 4, 1e-6, p, 1 << 20, None)
    assert rc == hip.VH_ERR_DTYPE


def test_dwconv_rejects_bad_arguments(lib):
    p = ctypes.c_void_p(0x1000)

    def call(ksize=3, epilogue=0, aux=None, channels=16, x=p):
        return lib.vh_dwconv2d_nhwc_forward(x, hip.VH_DTYPE_BF16, p, p, ksize, epilogue, aux, p,
                                            2, 4, 4, channels, None)

    assert call(ksize=4) == hip.VH_ERR_ARG
    assert call(epilogue=9) == hip.VH_ERR_ARG
    assert call(epilogue=2) == hip.VH_ERR_ARG          # gate tensor missing
    assert call(channels=12) == hip.VH_ERR_SHAPE       # C % 8 != 0
    assert call(x=None) == hip.VH_ERR_ARG
    assert call(x=ctypes.c_void_p(0x1008)) == hip.VH_ERR_ARG   # misaligned
    assert b"aligned" in lib.vh_last_error()


def test_pointwise_conv_rejects_bad_arguments(lib):
    p = ctypes.c_void_p(0x1000)

    def call(dtype=hip.VH_DTYPE_BF16, epilogue=0, residual=None, scale=None, beta=None, per_image=0,
             m=64, n=64, k=64, x=p):
        return lib.vh_pointwise_conv_nhwc_forward(x, dtype, p, p, epilogue, residual, scale, beta, per_image,
                                                  p, m, n, k, None)

    assert call(dtype=hip.VH_DTYPE_F32) == hip.VH_ERR_DTYPE
    assert call(k=48) == hip.VH_ERR_SHAPE                # K % 32 != 0
    assert call(n=48) == hip.VH_ERR_SHAPE                # N % 32 != 0
    assert call(n=48) == hip.VH_ERR_SHAPE
    assert call(m=0) == hip.VH_ERR_SHAPE
    assert call(epilogue=4) == hip.VH_ERR_ARG
    assert call(epilogue=2) == hip.VH_ERR_ARG            # residual missing
    assert call(scale=p) == hip.VH_ERR_ARG               # beta missing
    assert call(scale=p, beta=p, per_image=48) == hip.VH_ERR_SHAPE   # M not a multiple of it
    assert call(x=None) == hip.VH_ERR_ARG
    assert call(x=ctypes.c_void_p(0x1008)) == hip.VH_ERR_ARG
    assert b"aligned" in lib.vh_last_error()


def test_pointwise_chain_and_add_layernorm_reject_bad_arguments(lib):
    """The chained proj_in + local_gate and the proj_out + add + norm2 entries validate their
    shapes, pointers and alignment before launching anything."""
    p = ctypes.c_void_p(0x1000)

    def chain(m=64, n=128, k=256, x=p, w2=p):
        return lib.vh_pointwise_chain_nhwc_forward(x, p, p, w2, p, p, p, m, n, k, None)

    assert chain(n=256) == hip.VH_ERR_SHAPE              # N = 32, 64 or 128 only
    assert chain(k=96) == hip.VH_ERR_SHAPE               # K % 64 for N = 64, 128
    assert chain(n=32, k=128) == hip.VH_ERR_SHAPE        # N = 32 takes K = 32 or 64
    assert chain(m=0) == hip.VH_ERR_SHAPE
    assert chain(w2=None) == hip.VH_ERR_ARG
    assert chain(x=ctypes.c_void_p(0x1008)) == hip.VH_ERR_ARG

    def addln(m=64, n=256, k=128, eps=1e-6, res=p, x=p):
        return lib.vh_pointwise_add_layernorm_nhwc_forward(x, p, p, res, p, p, eps, p, p, m, n, k, None)

    assert addln(n=512) == hip.VH_ERR_SHAPE
    assert addln(n=64, k=128) == hip.VH_ERR_SHAPE
    assert addln(k=256) == hip.VH_ERR_SHAPE
    assert addln(m=0) == hip.VH_ERR_SHAPE
    assert addln(eps=0.0) == hip.VH_ERR_ARG
    assert addln(res=None) == hip.VH_ERR_ARG
    assert addln(x=ctypes.c_void_p(0x1008)) == hip.VH_ERR_ARG


def test_readout_lepe_rejects_bad_arguments(lib):
    p = ctypes.c_void_p(0x1000)
    arr, keep = hip.int64_array((4, 4, 4, 4))

    def call(taps=p, h=4, w=4):
        return lib.vh_srnl_spatial_readout_lepe(p, p, hip.VH_DTYPE_BF16, p, 0, p, taps, None, p, 2, h, w, 32, 16,
                                                arr, p, 1 << 20, None)

    assert call(taps=None) == hip.VH_ERR_ARG
    assert call(h=0) == hip.VH_ERR_SHAPE


def test_grn_scale_rejects_bad_arguments(lib):
    p = ctypes.c_void_p(0x1000)

    def call(channels=64, ws=1 << 20, x=p):
        return lib.vh_grn_scale_forward(x, hip.VH_DTYPE_BF16, p, p, p, p, 2, channels, 4, 4, 1e-6, p, ws, None)

    assert call(x=None) == hip.VH_ERR_ARG
    assert call(channels=12) == hip.VH_ERR_SHAPE
    assert call(ws=16) == hip.VH_ERR_WORKSPACE


def test_bias_act_rejects_bad_arguments(lib):
    p = ctypes.c_void_p(0x1000)

    def call(act=0, total=64, channels=16, x=p, dtype=hip.VH_DTYPE_BF16):
        return lib.vh_bias_act_nhwc_forward(x, dtype, p, act, p, total, channels, None)

    assert call(act=2) == hip.VH_ERR_ARG
    assert call(channels=12) == hip.VH_ERR_SHAPE
    assert call(total=40) == hip.VH_ERR_SHAPE           # not a whole number of pixels
    assert call(dtype=9) == hip.VH_ERR_DTYPE
    assert call(x=None) == hip.VH_ERR_ARG


def test_conv3x3_rejects_bad_arguments(lib):
    p = ctypes.c_void_p(0x1000)

    def call(dtype=hip.VH_DTYPE_BF16, act=0, cin=32, cout=64, stride=1, b=2, x=p, h=8):
        return lib.vh_conv3x3_nhwc_forward(x, dtype, p, p, act, p, b, h, 8, cin, cout, stride, None)

    assert call(stride=3) == hip.VH_ERR_ARG
    assert call(act=2) == hip.VH_ERR_ARG
    assert call(cin=48) == hip.VH_ERR_SHAPE              # neither 3 nor a multiple of 32
    assert call(cout=80) == hip.VH_ERR_SHAPE             # not a multiple of 32
    assert call(dtype=hip.VH_DTYPE_F32) == hip.VH_ERR_DTYPE   # fp32 only for the 3-channel image
    assert call(cin=3, dtype=hip.VH_DTYPE_F16) == hip.VH_ERR_DTYPE
    assert call(b=0) == hip.VH_ERR_SHAPE
    assert call(h=1 << 20, b=1 << 12) == hip.VH_ERR_SHAPE    # more than 2^31 output pixels
    assert call(x=None) == hip.VH_ERR_ARG
    assert call(x=ctypes.c_void_p(0x1008)) == hip.VH_ERR_ARG  # misaligned bf16 map
    assert b"aligned" in lib.vh_last_error()


def test_dwconv_grn_workspace_query(lib):
    # Blocks of G x r threads (G = C / 8 channel groups, r <= 256 / G pixel segments, the
    # largest r dividing an image's rows x segments) tile whole images.
    assert lib.vh_dwconv2d_gelu_grn_workspace_bytes(2, 56, 56, 256, 3) == 2 * 49 * 256 * 4
    assert lib.vh_dwconv2d_gelu_grn_workspace_bytes(128, 14, 14, 1024, 3) == 128 * 14 * 1024 * 4
    # Base stage 2: 96 groups x 2 segments (192 threads), 64 rows x 8 segments -> 256 per image
    assert lib.vh_dwconv2d_gelu_grn_workspace_bytes(8, 64, 64, 768, 3) == 8 * 256 * 768 * 4
    # Base stage 1: 48 groups x 4 segments (5 do not divide 128 rows x 16 segments)
    assert lib.vh_dwconv2d_gelu_grn_workspace_bytes(8, 128, 128, 384, 3) == 8 * 512 * 384 * 4
    # 14 rows x 2 segments: 32 groups x 7 segments, 4 blocks per image
    assert lib.vh_dwconv2d_gelu_grn_workspace_bytes(1, 14, 14, 256, 3) == 4 * 256 * 4
    assert lib.vh_dwconv2d_gelu_grn_workspace_bytes(1, 7, 7, 2560, 3) == 0      # 320 groups > 256
    assert lib.vh_dwconv2d_gelu_grn_workspace_bytes(1, 8, 8, 100, 3) == 0       # C % 8
    p = ctypes.c_void_p(0x1000)
    rc = lib.vh_dwconv2d_gelu_grn_forward(p, hip.VH_DTYPE_BF16, p, p, 3, p, ctypes.c_float(1e-6), p, p, p, p,
                                          1, 7, 7, 2560, p, 1 << 20, None)
    assert rc == hip.VH_ERR_SHAPE


def test_dwconv_add_layernorm_validates(lib):
    """The fused CPE + LayerNorm takes kernel size 3 and C = 8 * 2^k <= 256 only."""
    p = ctypes.c_void_p(0x1000)

    def call(C=256, ksize=3, x=p, eps=1e-6, dtype=hip.VH_DTYPE_BF16):
        return lib.vh_dwconv2d_add_layernorm2d_forward(x, dtype, p, p, ksize, p, p, ctypes.c_float(eps), p, p,
                                                       2, 14, 14, C, None)

    assert call(C=96) == hip.VH_ERR_SHAPE      # C/8 = 12 is not a power of two
    assert call(C=512) == hip.VH_ERR_SHAPE     # 64 groups: more than one 32-lane row group
    assert call(ksize=5) == hip.VH_ERR_ARG
    assert call(x=None) == hip.VH_ERR_ARG
    assert call(eps=0.0) == hip.VH_ERR_ARG
    assert call(dtype=7) == hip.VH_ERR_DTYPE
    assert call(x=ctypes.c_void_p(0x1008)) == hip.VH_ERR_ARG   # misaligned
    assert b"aligned" in lib.vh_last_error()


def test_check_raises_with_message(lib):
    assert _spatial(lib, head_dim=12) == hip.VH_ERR_HEAD_DIM
    with pytest.raises(RuntimeError, match="head_dim"):
        hip.check(hip.VH_ERR_HEAD_DIM, "vh_srnl_spatial_forward")
    with pytest.raises(TypeError):
        hip.check(hip.VH_ERR_DTYPE, "x")


def test_missing_library_fails_loudly(tmp_path):
    with pytest.raises(hip.NativeLibraryMissing):
        hip.load_library(tmp_path / "absent.so")


def _backward(lib, directions=4, consts=None):
    p = ctypes.c_void_p(0x1000)
    arr, keep = hip.int64_array([4] * 4)
    return lib.vh_srnl_backward(p, p, hip.VH_DTYPE_F32, 1, p, p, p, p, p, p, 0, p, p, p, p, p, p, p,
                                2, directions, 2, 8, 16, arr, consts if consts is not None else _consts(),
                                p, 1 << 30, None)


def test_srnl_backward_validates_directions_and_constants(lib):
    """The backward checks what the forward checks: 1, 2 or 4 directions and the ranges of
    the stability constants (a zero injection margin would give NaN gradients)."""
    assert _backward(lib, directions=3) == hip.VH_ERR_SHAPE
    assert b"directions" in lib.vh_last_error()
    for bad, name in ((hip.make_consts(0.025, 1.5, 2.197224577, 0.999, True, 0.999999), b"MIN_RETENTION"),
                      (hip.make_consts(0.025, 0.0, 2.197224577, 0.0, True, 0.999999), b"INJECTION_MARGIN"),
                      (hip.make_consts(-1.0, 0.0, 2.197224577, 0.999, True, 0.999999), b"STEP_SCALE"),
                      (hip.make_consts(0.025, 0.0, 2.197224577, 0.999, True, 1.5), b"SPECTRAL_MARGIN")):
        assert _backward(lib, consts=bad) == hip.VH_ERR_ARG
        assert name in lib.vh_last_error()
    bad_margin = hip.make_consts(0.025, 0.0, 2.197224577, 0.999, True, 0.0)
    assert _spatial(lib, consts=bad_margin) == hip.VH_ERR_ARG


def test_dispatch_overrides_are_validated(lib):
    """Kernel choices are forced only through vh_set_dispatch_override, which rejects unknown
    names and malformed values; nothing is read from the environment."""
    assert lib.vh_set_dispatch_override(b"no_such_knob", b"1") == hip.VH_ERR_ARG
    assert b"unknown" in lib.vh_last_error()
    for name, bad in ((b"scan_wide", b"3"), (b"scan_pack", b"3x4"), (b"scan_pack", b"4x2"), (b"scan_ut", b"yes"),
                      (b"grn_spin_limit", b"0"), (b"grn_spin_limit", b"2000000"), (b"pw_cfg", b"q1"),
                      (b"dw_launch_bytes", b"-5"), (b"scan_tb", b"12345678901234567890123456789012345")):
        assert lib.vh_set_dispatch_override(name, bad) == hip.VH_ERR_ARG, (name, bad)
    for name, good in ((b"scan_wide", b"2"), (b"scan_pack", b"2x4"), (b"grn_spin_limit", b"64"),
                       (b"pw_cfg", b"t128x128k32o2"), (b"dw_launch_bytes", b"4097")):
        assert lib.vh_set_dispatch_override(name, good) == hip.VH_OK, (name, good)
        assert lib.vh_set_dispatch_override(name, None) == hip.VH_OK
    lib.vh_clear_dispatch_overrides()


def test_no_environment_reads_in_the_library():
    """The shipped sources choose kernels from their arguments (and the dispatch overrides);
    the only environment variables read anywhere are the reference's numerics constants."""
    sources = list((ROOT / "visionhope_amd" / "csrc").glob("*.hip")) + list((ROOT / "visionhope_amd" / "csrc").glob("*.h"))
    for path in sources:
        assert "getenv" not in path.read_text(), path.name
    for path in (ROOT / "visionhope_amd").rglob("*.py"):
        text = path.read_text()
        if "os.environ" in text:
            assert path.name in ("chunk.py", "build.py"), path


def test_grn_fallback_query_validates(lib):
    count = ctypes.c_int64(-1)
    assert lib.vh_grn_workspace_fallbacks(None, 1 << 20, None, ctypes.byref(count)) == hip.VH_ERR_ARG
    assert lib.vh_grn_workspace_fallbacks(ctypes.c_void_p(0x1000), 100, None, ctypes.byref(count)) == hip.VH_ERR_WORKSPACE
