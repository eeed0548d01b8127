"""vh_srnl_spatial_forward_noalloc: the fused spatial operator with its chunk-state buffer in
the library's fixed device array instead of a caller workspace.

Through the C ABI, each call must give exactly the bits of vh_srnl_spatial_forward (same
kernels on the same inputs) with a torch-allocated workspace.  Two calls in a row, the
second smaller: the array keeps the first call's contents, which must not leak into the
second.  Calls beyond the array's 96 MiB are rejected on the host before any GPU work.
"""

import ctypes
import math

import pytest
import torch

from tests.helpers import memories, randn
from visionhope_amd.utils import hip

SCRATCH_BYTES = 96 << 20


def _consts():
    return hip.make_consts(0.025, 0.0, 2.197224577, 0.999, True, 0.999999)


def _case(batch, height, width, heads, head_dim, dtype, seed, device):
    channels = heads * head_dim
    mems = tuple(torch.from_numpy(m).to(device)
                 for m in memories(4, heads, head_dim, kind="perturbed", seed=seed))
    x = randn(batch, height, width, channels, seed=seed + 1).to(dtype).to(device)
    q = randn(batch, height, width, channels, seed=seed + 2).to(dtype).to(device)
    skip = randn(channels, seed=seed + 3, scale=0.1).to(device)
    wts = (1 + randn(4, channels, seed=seed + 4, scale=0.1)).to(device)
    return mems, x, q, skip, wts


def _run(lib, mems, x, q, skip, wts, head_dim, *, noalloc):
    batch, height, width, channels = x.shape
    out = torch.empty(batch, height, width, channels, device=x.device, dtype=torch.float32)
    chunks, keep = hip.int64_array([width, width, height, height])
    common = [hip.ptr(x), hip.ptr(q), hip.dtype_code(x.dtype), *[hip.ptr(m) for m in mems], hip.ptr(skip), 0,
              hip.ptr(wts), hip.ptr(out), batch, height, width, channels, head_dim, chunks, _consts()]
    if noalloc:
        rc = lib.vh_srnl_spatial_forward_noalloc(*common, hip.stream_of(x))
    else:
        max_chunks = max(math.ceil(height * width / c) for c in (width, height))
        ws = hip.workspace(lib.vh_srnl_workspace_bytes(batch * 4 * (channels // head_dim), max_chunks, head_dim),
                           x.device)
        rc = lib.vh_srnl_spatial_forward(*common, hip.ptr(ws), ws.numel() * 4, hip.stream_of(x))
    hip.check(rc, "spatial forward")
    return out


@pytest.mark.gpu
def test_noalloc_matches_workspace_entry_twice(device):
    lib = hip.load_library()
    cases = [(4, 28, 28, 4, 16, torch.bfloat16, 10),     # Tiny stage-2 operator shape, 4 images
             (2, 14, 9, 2, 16, torch.float32, 20),       # smaller, rectangular, fp32
             (1, 12, 12, 3, 32, torch.bfloat16, 30)]     # smaller still, head_dim 32
    for batch, height, width, heads, head_dim, dtype, seed in cases:
        print(f"noalloc case B={batch} {height}x{width} heads={heads} d={head_dim} {dtype}", flush=True)
        mems, x, q, skip, wts = _case(batch, height, width, heads, head_dim, dtype, seed, device)
        got = _run(lib, mems, x, q, skip, wts, head_dim, noalloc=True)
        want = _run(lib, mems, x, q, skip, wts, head_dim, noalloc=False)
        torch.cuda.synchronize()
        assert torch.isfinite(got).all()
        assert torch.equal(got, want), f"noalloc differs: max {(got - want).abs().max().item():.3e}"


@pytest.mark.gpu
def test_noalloc_inside_graph_capture(device):
    """The call allocates nothing, so it can be captured; every replay matches the eager
    workspace entry (replays interleaved with eager work)."""
    lib = hip.load_library()
    mems, x, q, skip, wts = _case(2, 14, 14, 2, 16, torch.bfloat16, 40, device)
    want = _run(lib, mems, x, q, skip, wts, 16, noalloc=False)
    _run(lib, mems, x, q, skip, wts, 16, noalloc=True)          # first call on the device: address lookup
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            out = _run(lib, mems, x, q, skip, wts, 16, noalloc=True)
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want)
        _run(lib, mems, x, q, skip, wts, 16, noalloc=False)      # eager work between replays


def test_noalloc_rejects_calls_beyond_its_scratch():
    """Validation happens on the host before the device is touched (runs without a GPU)."""
    lib = hip.load_library()
    p = ctypes.c_void_p(0x1000)
    # Base 512^2 stage 1 at B = 512: 512*4*3 lines x 128 chunks x 1 KB = 805 MB > 96 MiB
    chunks, keep = hip.int64_array([128] * 4)
    rc = lib.vh_srnl_spatial_forward_noalloc(p, p, hip.VH_DTYPE_BF16, p, p, p, p, p, p, 0, p, p,
                                             512, 128, 128, 48, 16, chunks, _consts(), None)
    assert rc == hip.VH_ERR_WORKSPACE
    assert b"vh_srnl_spatial_forward" in lib.vh_last_error()
    assert lib.vh_srnl_workspace_bytes(512 * 4 * 3, 128, 16) > SCRATCH_BYTES
    rc = lib.vh_srnl_spatial_forward_noalloc(p, p, hip.VH_DTYPE_BF16, p, p, p, p, p, p, 0, p, p,
                                             2, 8, 8, 48, 12, chunks, _consts(), None)
    assert rc == hip.VH_ERR_HEAD_DIM


_FOOTPRINT_PROBE = r"""
import ctypes, json, sys
sys.path.insert(0, sys.argv[1])
import torch
from visionhope_amd.utils import hip
dev = torch.device("cuda:0")
gen = torch.Generator().manual_seed(3)
mems = [torch.randn(4, 2, 16, 16, generator=gen).mul(0.01).to(dev) for _ in range(3)]
mems += [torch.zeros(4, 2, 16, device=dev) for _ in range(2)]
x = torch.randn(1, 8, 8, 32, generator=gen).bfloat16().to(dev)
q = torch.randn(1, 8, 8, 32, generator=gen).bfloat16().to(dev)
skip, w = torch.zeros(32, device=dev), torch.ones(4, 32, device=dev)
out, out2, ws = torch.empty(1, 8, 8, 32, device=dev), torch.empty(1, 8, 8, 32, device=dev), torch.empty(1 << 20, device=dev)
lib = hip.load_library()
chunks, keep = hip.int64_array([8] * 4)
consts = hip.make_consts(0.025, 0.0, 2.197224577, 0.999, True, 0.999999)
args = [hip.ptr(x), hip.ptr(q), 1, *[hip.ptr(m) for m in mems], hip.ptr(skip), 0, hip.ptr(w)]
torch.cuda.synchronize()
f0 = torch.cuda.mem_get_info()[0]
hip.check(lib.vh_srnl_spatial_forward(*args, hip.ptr(out), 1, 8, 8, 32, 16, chunks, ctypes.byref(consts),
                                      hip.ptr(ws), ws.numel() * 4, hip.stream_of(x)), "forward")
torch.cuda.synchronize()
f1 = torch.cuda.mem_get_info()[0]
hip.check(lib.vh_srnl_spatial_forward_noalloc(*args, hip.ptr(out2), 1, 8, 8, 32, 16, chunks, ctypes.byref(consts),
                                              hip.stream_of(x)), "noalloc")
torch.cuda.synchronize()
f2 = torch.cuda.mem_get_info()[0]
print(json.dumps({"ordinary": f0 - f1, "noalloc": f1 - f2, "equal": bool(torch.equal(out, out2))}))
"""


@pytest.mark.gpu
def test_scratch_array_is_held_only_by_processes_that_call_the_entry():
    """The array lives in its own code object, which the HIP runtime loads at the first use
    of that object's kernels or symbols: in a fresh process, an ordinary SRNL call adds a
    few MiB of device memory (its own code object), and only the first no-alloc call adds
    the array's 96 MiB."""
    import json
    import subprocess
    import sys
    from pathlib import Path

    root = Path(__file__).resolve().parents[1]
    proc = subprocess.run([sys.executable, "-c", _FOOTPRINT_PROBE, str(root)], capture_output=True, text=True,
                          timeout=180)
    assert proc.returncode == 0, proc.stderr[-2000:]
    result = json.loads(proc.stdout.strip().splitlines()[-1])
    print(f"[footprint] {result}", flush=True)
    assert result["equal"]
    assert result["ordinary"] < 32 << 20, result
    assert result["noalloc"] >= SCRATCH_BYTES, result
