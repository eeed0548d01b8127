"""Benchmark: VisionHOPE-Tiny classification forward, 224x224, B=128, bf16 autocast, on one
MI355X, plus live roofline figures for the SRNL operator and the memory-bound tail.

    python bench.py [--gpus 1] [--steps K] [--warmup W]

Prints ONE JSON line.  ``value`` is images/s of the full forward (HIP graph replay,
inputs resident in HBM).  ``roofline`` covers the SRNL spatial operator launches
(scan + readout, ``vh_srnl_spatial_forward``) summed over one forward, timed with
HIP events on the stream they run on, with their counter-measured HBM traffic;
``kernels`` breaks it down per stage and adds the fused elementwise workload (B=128 at
56x56x96 and 28x28x192).  ``cpu_baseline`` times the same model on the host cores with
the CPU oracle standing in for SRNL (the reference has no CPU SRNL path).
"""

from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

METRIC = "images/s VisionHOPE-Tiny 224² B=128 bf16; SRNL-scan ms + % of roofline"
HBM_PEAK_GBS = 8000.0
FP32_PEAK_TFLOPS = 157.3
BF16_PEAK_TFLOPS = 2500.0   # dense bf16 matrix peak: the instruction the SRNL scan and readout issue
SEED = 1234
TINY_STAGES = [  # (grid, mixer channels, depth), head_dim 16 (models/factory.py, hierarchical.py)
    (56, 32, 3), (28, 64, 4), (14, 128, 18), (7, 256, 4)]
# HBM bytes per vh_srnl_spatial_forward launch (scan + readout) at B=128, bf16, from
# rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE of `bench.py --stages-only`, calibrated against a
# 512 MiB copy (profiles/srnl_stages_b128_traffic.md).  Valid for the kernels measured there.
SRNL_TRAFFIC_BYTES_B128 = {56: 271.0e6, 28: 187.8e6, 14: 152.9e6, 7: 135.6e6}


def srnl_flops(batch, height, width, channels, head_dim, chunks):
    """Reference analytic count (analysis/operation_count.py:36-44), FLOP = 2 MAC."""
    heads = channels // head_dim
    length = height * width
    token_cost = 6 * head_dim ** 2 + 20 * head_dim
    boundary_cost = 3 * head_dim ** 3 + 2 * head_dim ** 2
    macs = 0
    for chunk in chunks:
        boundaries = math.ceil(length / chunk)
        macs += batch * heads * (boundaries * chunk * token_cost + boundaries * boundary_cost)
    return 2 * macs


def event_time_ms(fn, stream, iters, warmup=2):
    import torch
    for _ in range(warmup):
        fn()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record(stream)
    for _ in range(iters):
        fn()
    end.record(stream)
    end.synchronize()
    return start.elapsed_time(end) / iters


def graph_time_ms(fn, iters, reps=3):
    """Milliseconds per call of ``fn`` with ``iters`` back-to-back calls captured in one HIP
    graph, replayed ``reps`` times: the GPU time of its launches without the Python
    wrapper's host time between them (how a serving loop runs these ops)."""
    import torch
    fn()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(iters):
            fn()
    ms = event_time_ms(graph.replay, torch.cuda.current_stream(), reps, warmup=1)
    del graph
    return ms / iters


def _perturbed_memories(heads, head_dim, device, gen):
    """Repo default init for the matrix memories, N(0, 0.1^2) gate vectors so gates vary."""
    import torch
    mats = []
    for _ in range(3):
        m = torch.empty(4, heads, head_dim, head_dim, device=device)
        torch.nn.init.trunc_normal_(m, std=0.01, generator=gen)
        mats.append(m)
    vecs = [torch.randn(4, heads, head_dim, device=device, generator=gen) * 0.1 for _ in range(2)]
    return (*mats, *vecs)


def measure_srnl_stages(device, batch):
    """Average duration of one vh_srnl_spatial_forward launch pair per Tiny stage."""
    import torch
    from visionhope_amd.models.srnl_core.fused import srnl_spatial_inference

    stream = torch.cuda.current_stream(device)
    gen = torch.Generator(device=device).manual_seed(SEED)
    rows, total_flops, total_ms, total_bytes, total_compulsory = [], 0.0, 0.0, 0.0, 0.0
    for grid, channels, depth in TINY_STAGES:
        head_dim = 16
        heads = channels // head_dim
        mems = _perturbed_memories(heads, head_dim, device, gen)
        x = torch.randn(batch, grid, grid, channels, device=device, generator=gen).bfloat16()
        q = torch.randn(batch, grid, grid, channels, device=device, generator=gen).bfloat16()
        skip = torch.zeros(channels, device=device)
        wts = torch.ones(4, channels, device=device)
        chunks = (grid, grid, grid, grid)
        ms = event_time_ms(lambda: srnl_spatial_inference(mems, x, q, skip, wts, chunks), stream, 20)
        flops = srnl_flops(batch, grid, grid, channels, head_dim, chunks)
        # compulsory bytes: x and q in bf16, the FP32 output (the chunk states are not)
        compulsory = batch * grid * grid * channels * (2 + 2 + 4)
        row = {"stage": f"{grid}x{grid} C={channels} d={head_dim}", "blocks": depth,
               "ms_per_launch": round(ms, 4), "tflops": round(flops / ms / 1e9, 3),
               "compulsory_bytes_per_launch": compulsory}
        if batch == 128:
            row["hbm_bytes_per_launch"] = SRNL_TRAFFIC_BYTES_B128[grid]
            row["traffic_over_compulsory"] = round(SRNL_TRAFFIC_BYTES_B128[grid] / compulsory, 3)
            total_bytes += SRNL_TRAFFIC_BYTES_B128[grid] * depth
        rows.append(row)
        total_flops += flops * depth
        total_ms += ms * depth
        total_compulsory += compulsory * depth
    return rows, total_flops, total_ms, (total_bytes if batch == 128 else None), total_compulsory


def measure_tail(device):
    """Fusion, GRN and LN at B=128, 56x56x96 and 28x28x192, bf16: GB/s of compulsory traffic,
    each op timed as graph replays (GPU time of its launches)."""
    import torch
    from visionhope_amd.utils.direction_fusion import visionhope_postprocess_scale
    from visionhope_amd.utils.grn_cuda import visionhope_grn
    from visionhope_amd.utils.layer_norm_cuda import visionhope_layernorm2d

    stream = torch.cuda.current_stream(device)
    gen = torch.Generator(device=device).manual_seed(SEED)
    out = {}
    for batch, grid, channels in ((128, 56, 96), (128, 28, 192)):
        heads, head_dim = channels // 16, 16
        n = batch * grid * grid * channels
        x = torch.randn(batch, grid, grid, channels, device=device, generator=gen).bfloat16()
        xc = x.permute(0, 3, 1, 2)
        gamma = torch.randn(channels, device=device, generator=gen) * 0.1
        beta = torch.randn(channels, device=device, generator=gen) * 0.1
        ys = torch.randn(batch, 4, heads, grid * grid, head_dim, device=device, generator=gen).bfloat16()
        xs = torch.randn(batch, 4, heads, grid * grid, head_dim, device=device, generator=gen).bfloat16()
        skip = torch.randn(heads, head_dim, device=device, generator=gen) * 0.1
        scale = 1 + torch.randn(4, channels, device=device, generator=gen) * 0.1
        tag = f"{grid}x{grid}x{channels}"
        ops = (("fusion", lambda: visionhope_postprocess_scale(ys, xs, skip, scale, grid, grid, True), 20),
               ("grn", lambda: visionhope_grn(xc, gamma, beta, 1e-6), 6),
               ("layernorm", lambda: visionhope_layernorm2d(xc, gamma, beta, 1e-6), 6))
        for _, fn, _ in ops:   # untimed pass: the first graphs of a process run measurably slower
            graph_time_ms(fn, 20)
        for name, fn, bytes_per in ops:
            ms = graph_time_ms(fn, 20)
            gbs = bytes_per * n / ms / 1e6
            out[f"{name}_{tag}"] = {"ms": round(ms, 4), "GB/s": round(gbs, 1),
                                    "frac_hbm": round(gbs / HBM_PEAK_GBS, 3)}
        del x, ys, xs
    return out


def measure_tail_backward(device):
    """Backward of fusion, GRN and LN (autograd, the native backward entries) at B=128,
    56x56x96, bf16 activations: GB/s of compulsory traffic per element (fusion: fp32
    dout + four y and x reads + four dy and dx writes = 36 B; GRN and LN: fp32 dout, the
    bf16 input and the bf16 input gradient = 8 B) against the HBM peak."""
    import torch
    from visionhope_amd.utils.direction_fusion import visionhope_postprocess_scale
    from visionhope_amd.utils.grn_cuda import visionhope_grn
    from visionhope_amd.utils.layer_norm_cuda import visionhope_layernorm2d

    stream = torch.cuda.current_stream(device)
    gen = torch.Generator(device=device).manual_seed(SEED)
    batch, grid, channels = 128, 56, 96
    heads, head_dim = channels // 16, 16
    n = batch * grid * grid * channels
    x = torch.randn(batch, grid, grid, channels, device=device, generator=gen).bfloat16()
    xc = x.permute(0, 3, 1, 2).requires_grad_()
    gamma = (torch.randn(channels, device=device, generator=gen) * 0.1).requires_grad_()
    beta = (torch.randn(channels, device=device, generator=gen) * 0.1).requires_grad_()
    ys = torch.randn(batch, 4, heads, grid * grid, head_dim, device=device, generator=gen).bfloat16().requires_grad_()
    xs = torch.randn(batch, 4, heads, grid * grid, head_dim, device=device, generator=gen).bfloat16().requires_grad_()
    skip = (torch.randn(heads, head_dim, device=device, generator=gen) * 0.1).requires_grad_()
    scale = (1 + torch.randn(4, channels, device=device, generator=gen) * 0.1).requires_grad_()
    dout = torch.randn(batch, grid, grid, channels, device=device, generator=gen).permute(0, 3, 1, 2)
    out = {}
    for name, fwd, inputs, bytes_per in (
            ("fusion", lambda: visionhope_postprocess_scale(ys, xs, skip, scale, grid, grid, True),
             (ys, xs, skip, scale), 36),
            ("grn", lambda: visionhope_grn(xc, gamma, beta, 1e-6), (xc, gamma, beta), 8),
            ("layernorm", lambda: visionhope_layernorm2d(xc, gamma, beta, 1e-6), (xc, gamma, beta), 8)):
        y = fwd()
        # eager autograd (the backward is not captured in a graph: autograd runs it on its
        # own device thread), so short kernels include the host time between launches
        ms = event_time_ms(lambda: torch.autograd.grad(y, inputs, dout, retain_graph=True), stream, 5)
        gbs = bytes_per * n / ms / 1e6
        out[f"{name}_backward_{grid}x{grid}x{channels}"] = {"ms": round(ms, 4), "GB/s": round(gbs, 1),
                                                            "frac_hbm": round(gbs / HBM_PEAK_GBS, 3),
                                                            "timing": "eager autograd"}
        del y
    return out


def measure_srnl_backward(device):
    """vh_srnl_backward on config 1 (standalone SRNL, fp32, d = 32) and on the lines of one
    Tiny stage-3 operator (B = 128, bf16, d = 16): event-timed ms, and TFLOP/s of three
    times the reference's forward FLOP count (the backward recomputes the forward and
    runs the reverse recurrence, about twice its MACs) against the FP32 peak."""
    import torch
    from visionhope_amd.models.srnl_core.chunk import srnl_packed_backward

    stream = torch.cuda.current_stream(device)
    gen = torch.Generator(device=device).manual_seed(SEED)
    out = {}
    for tag, batch, dirs, heads, grid, d, dtype in (("config1_2x196x64_d32_fp32", 2, 1, 2, 14, 32, torch.float32),
                                                    ("tiny_stage3_128x14x14x128_d16_bf16", 128, 4, 8, 14, 16,
                                                     torch.bfloat16)):
        n = grid * grid
        mems = _perturbed_memories(heads, d, device, gen)
        mems = tuple(m[:dirs].contiguous() for m in mems)
        x = torch.randn(batch, dirs, heads, n, d, device=device, generator=gen).to(dtype)
        q = torch.randn(batch, dirs, n, heads * d, device=device, generator=gen).to(dtype)
        dy = torch.randn(batch, dirs, heads, n, d, device=device, generator=gen)
        chunks = [grid] * dirs
        ms = event_time_ms(lambda: srnl_packed_backward(mems, x, q, chunks, dy, q_raw=True), stream, 3, warmup=1)
        flops = 3 * srnl_flops(batch, grid, grid, heads * d, d, chunks)
        out[f"srnl_backward_{tag}"] = {"ms": round(ms, 3), "forward_equiv_gflop": round(flops / 1e9, 3),
                                       "tflops": round(flops / ms / 1e9, 3),
                                       "frac_fp32_peak": round(flops / ms / 1e9 / FP32_PEAK_TFLOPS, 4)}
    return out


def build_tiny(device, channels_last=True):
    import torch
    from visionhope_amd.inference.prepare import prepare_for_inference
    from visionhope_amd.models import create_model

    torch.manual_seed(SEED)
    model = create_model("visionhope_tiny", drop_path_rate=0.0).to(device)
    if channels_last:
        model = model.to(memory_format=torch.channels_last)
    prepare_for_inference(model)
    return model


def measure_base512(device, batch=8, reps=5):
    """Config 4: VisionHOPE-Base at 512x512, B=8, bf16 autocast, prepared, the four stage
    feature maps (no task head; 128^2 / 64^2 / 32^2 / 16^2 token grids, chunks of 128 at
    stage 1), one forward captured in a HIP graph: ms per forward and images/s."""
    import torch
    from visionhope_amd.inference.prepare import prepare_for_inference
    from visionhope_amd.models import create_model

    with torch.inference_mode(False):   # parameters are ordinary tensors even inside the bench's inference mode
        torch.manual_seed(SEED)
        model = create_model("visionhope_base", drop_path_rate=0.0).to(device).to(memory_format=torch.channels_last)
        model.eval()
        prepare_for_inference(model)
    gen = torch.Generator().manual_seed(SEED + 4)
    images = torch.randn(batch, 3, 512, 512, generator=gen).to(device).contiguous(memory_format=torch.channels_last)

    def forward():
        with torch.inference_mode(), torch.autocast("cuda", dtype=torch.bfloat16):
            return model.forward_intermediates(images)

    feats = forward()
    torch.cuda.synchronize()
    if not all(torch.isfinite(f).all() for f in feats):
        raise FloatingPointError("Base 512 forward produced NaN/Inf")
    graph = torch.cuda.CUDAGraph()
    with torch.inference_mode(), torch.cuda.graph(graph):
        forward()
    ms = event_time_ms(graph.replay, torch.cuda.current_stream(device), reps, warmup=2)
    del graph, model
    return {"base512_b8_features": {"ms_per_forward": round(ms, 3), "images_per_s": round(batch * 1000.0 / ms, 1),
                                    "feature_shapes": [list(f.shape) for f in feats]}}


CONFIG3 = dict(batch=32, grid=56, channels=96, head_dim=32)


def _config3_operator(device):
    """Config 3: the four-direction operator (96 channels, 3 heads of 32, chunks 56), repo
    default init plus N(0, 0.1^2) gate vectors and skip, 1 + N(0, 0.1^2) direction scales,
    fast inference; its bf16 channels-last input [32, 96, 56, 56] (what proj_in feeds it
    under autocast)."""
    import torch
    from visionhope_amd.models import VisionHOPEOperator

    c = CONFIG3
    with torch.inference_mode(False):
        torch.manual_seed(SEED)
        op = VisionHOPEOperator(c["channels"], head_dim=c["head_dim"], direction_merge="scale").to(device).eval()
        gen = torch.Generator(device=device).manual_seed(SEED + 3)
        with torch.no_grad():
            for p in (op.srnl.M_eta_0, op.srnl.M_alpha_0, op.d_skip):
                p.copy_(torch.randn(p.shape, device=device, generator=gen) * 0.1)
            op.direction_scale.add_(torch.randn(op.direction_scale.shape, device=device, generator=gen) * 0.1)
        op.fast_inference = True
    gen = torch.Generator().manual_seed(SEED + 33)
    x = torch.randn(c["batch"], c["grid"], c["grid"], c["channels"], generator=gen).bfloat16().to(device)
    return op, x.permute(0, 3, 1, 2)


def measure_operator_config3(device, reps=10):
    """Config 3 timed two ways: the whole operator forward (W_q projection, scans, readout
    and fusion; one forward per HIP graph replay) and its SRNL launch pair alone (scan +
    readout, event-timed on its stream).  The bound is max(FLOP / FP32 matrix peak, bytes /
    HBM peak): the recurrence computes in FP32, and the compulsory bytes are x and q in bf16
    and the FP32 output."""
    import torch
    from visionhope_amd.models.srnl_core.fused import srnl_spatial_inference

    c = CONFIG3
    op, x = _config3_operator(device)

    def forward():
        with torch.autocast("cuda", dtype=torch.bfloat16):
            return op(x)

    forward()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        forward()
    ms_op = event_time_ms(graph.replay, torch.cuda.current_stream(device), reps, warmup=2)
    del graph
    x_nhwc = x.permute(0, 2, 3, 1)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        q_nhwc = op.W_q(x_nhwc)
    mems = tuple(m.detach() for m in op.srnl.initial_memories)
    wts = op.direction_weights().detach().float()
    chunks = (c["grid"],) * 4
    ms = event_time_ms(lambda: srnl_spatial_inference(mems, x_nhwc, q_nhwc, op.d_skip, wts, chunks),
                       torch.cuda.current_stream(device), reps)
    flops = srnl_flops(c["batch"], c["grid"], c["grid"], c["channels"], c["head_dim"], chunks)
    nbytes = c["batch"] * c["grid"] * c["grid"] * c["channels"] * (2 + 2 + 4)
    bound_ms = max(flops / FP32_PEAK_TFLOPS / 1e9, nbytes / HBM_PEAK_GBS / 1e6)
    return {"operator_config3_b32_56x56x96_d32_bf16": {
        "ms_operator_forward": round(ms_op, 4), "ms_srnl_scan_readout": round(ms, 4),
        "algorithmic_gflop": round(flops / 1e9, 3), "algorithmic_mb": round(nbytes / 1e6, 1),
        "tflops": round(flops / ms / 1e9, 3), "frac_fp32_peak": round(flops / ms / 1e9 / FP32_PEAK_TFLOPS, 4),
        "roofline_bound_ms": round(bound_ms, 4), "frac_of_roofline": round(bound_ms / ms, 4),
        "bound": "fp32 matrix (FLOP) vs HBM (bytes), the larger"}}


def profile_config3(device):
    """Three config-3 operator forwards (eager, bf16 autocast) for kernel traces."""
    import torch

    op, x = _config3_operator(device)
    with torch.inference_mode(), torch.autocast("cuda", dtype=torch.bfloat16):
        for i in range(3):
            op(x)
            torch.cuda.synchronize()
            print(f"config 3 operator forward {i}", flush=True)
    return 0


def profile_base512(device, batch=8):
    """Three Base 512 B=8 feature forwards (prepared, bf16 autocast, eager) for kernel traces."""
    import torch
    from visionhope_amd.inference.prepare import prepare_for_inference
    from visionhope_amd.models import create_model

    torch.manual_seed(SEED)
    model = create_model("visionhope_base", drop_path_rate=0.0).to(device).to(memory_format=torch.channels_last)
    model.eval()
    prepare_for_inference(model)
    gen = torch.Generator().manual_seed(SEED + 4)
    images = torch.randn(batch, 3, 512, 512, generator=gen).to(device).contiguous(memory_format=torch.channels_last)
    with torch.inference_mode(), torch.autocast("cuda", dtype=torch.bfloat16):
        for i in range(3):
            model.forward_intermediates(images)
            torch.cuda.synchronize()
            print(f"Base 512 B={batch} forward {i}", flush=True)
    return 0


def cpu_baseline(sample_batch=8, reps=3):
    """Tiny forward on the host: PyTorch CPU for convs/linears/norms and the CPU oracle
    (oracle/liboracle_srnl.so, OpenMP) for the four-direction SRNL operator."""
    import torch
    from oracle import oracle
    from visionhope_amd.models import operator as op_mod

    threads = torch.get_num_threads()

    def oracle_forward(self, x, *, channels_last=None):
        x_nhwc = x.float().permute(0, 2, 3, 1).contiguous()
        with torch.no_grad():
            q = self.W_q(x_nhwc)
        mems = tuple(m.detach().numpy() for m in self.srnl.initial_memories)
        out = oracle.operator_forward(x_nhwc.numpy(), q.numpy(), mems, self.d_skip.detach().numpy(),
                                      self.direction_weights().detach().numpy(), self.head_dim)
        return torch.from_numpy(out).permute(0, 3, 1, 2)

    model = build_tiny(torch.device("cpu"), channels_last=False)
    original = op_mod.VisionHOPEOperator.forward
    op_mod.VisionHOPEOperator.forward = oracle_forward
    try:
        # On CPU tensors the blocks take the ordinary branch, which calls operator.forward.
        gen = torch.Generator().manual_seed(SEED)
        images = torch.randn(sample_batch, 3, 224, 224, generator=gen)
        times = []
        with torch.no_grad():
            model(images)
            for _ in range(reps):
                t0 = time.perf_counter()
                model(images)
                times.append(time.perf_counter() - t0)
    finally:
        op_mod.VisionHOPEOperator.forward = original
    sec = statistics.median(times)
    return {"value": round(sample_batch / sec, 3), "unit": "images/s", "cores": threads,
            "kind": "port",
            "sample": f"VisionHOPE-Tiny 224x224 forward, B={sample_batch}, fp32, median of {reps}; "
                      f"PyTorch CPU ({threads} threads) + C oracle SRNL (OMP_NUM_THREADS="
                      f"{os.environ.get('OMP_NUM_THREADS', 'unset')}), "
                      f"os.cpu_count()={os.cpu_count()}, affinity={len(os.sched_getaffinity(0))}"}


def fast_path_audit(model, forward):
    """The reference's fast-path audit (``inference/audit.py``, ``analysis/benchmark.py:48-71``)
    on one untimed forward: queries projected once per operator call, one SRNL scan and one
    readout launch per call.  Returns the evidence, or the error if the audit fails."""
    from visionhope_amd.inference.audit import audit_fast_path

    try:
        _, evidence = audit_fast_path(model, forward)
        return evidence
    except Exception as exc:   # reported in the JSON line; the timing still runs
        return {"error": f"{type(exc).__name__}: {exc}"}


def validate_graph_changed_input(graph, graph_out, forward, images):
    """The reference's graph check (``analysis/benchmark.py:74-87``): new images are copied
    into the captured input buffer, the graph is replayed, and its logits are compared with
    an independent eager forward of the same images (bf16: atol 1e-3, rtol 1e-2)."""
    import torch

    if graph is None:
        return {"changed_input": False, "reason": "eager timing"}
    gen = torch.Generator().manual_seed(SEED + 99)
    fresh = torch.randn(images.shape, generator=gen).to(images.device)
    images.copy_(fresh.contiguous(memory_format=torch.channels_last))
    graph.replay()
    torch.cuda.synchronize()
    replayed = graph_out.float().clone()
    expected = forward().float()
    torch.cuda.synchronize()
    torch.testing.assert_close(replayed, expected, atol=1e-3, rtol=1e-2)
    return {"changed_input": True, "max_abs": float((replayed - expected).abs().max()),
            "bitwise_equal": bool(torch.equal(replayed, expected)), "atol": 1e-3, "rtol": 1e-2}


COPY_CALIBRATION_BYTES = 512 << 20


def profile_stages(device, batch):
    """Per-stage SRNL launches (3 each) then a 512 MiB FP32 scale-by-one copy, whose
    dispatch reads and writes exactly COPY_CALIBRATION_BYTES, for counter runs."""
    import torch
    from visionhope_amd.models.srnl_core.fused import srnl_spatial_inference

    torch.cuda.set_device(device)
    gen = torch.Generator(device=device).manual_seed(SEED)
    for grid, channels, _ in TINY_STAGES:
        heads = channels // 16
        mems = _perturbed_memories(heads, 16, device, gen)
        x = torch.randn(batch, grid, grid, channels, device=device, generator=gen).bfloat16()
        q = torch.randn(batch, grid, grid, channels, device=device, generator=gen).bfloat16()
        skip = torch.zeros(channels, device=device)
        wts = torch.ones(4, channels, device=device)
        for _ in range(3):
            srnl_spatial_inference(mems, x, q, skip, wts, (grid,) * 4)
        torch.cuda.synchronize()
        print(f"stage {grid}x{grid} C={channels}: 3 launches", flush=True)
        del x, q
    src = torch.ones(COPY_CALIBRATION_BYTES // 4, device=device)
    dst = torch.empty_like(src)
    torch.mul(src, 1.0, out=dst)
    torch.cuda.synchronize()
    print(f"calibration copy: {COPY_CALIBRATION_BYTES} bytes read and written", flush=True)
    return 0


def main(argv=None):
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=20)
    parser.add_argument("--warmup", type=int, default=5)
    parser.add_argument("--batch", type=int, default=128)
    parser.add_argument("--no-graph", action="store_true", help="time eager forwards instead of a HIP graph")
    parser.add_argument("--skip-cpu", action="store_true", help="omit the CPU baseline leg")
    parser.add_argument("--cudnn-benchmark", action="store_true",
                        help="let MIOpen search convolution solvers (analysis/benchmark.py:234)")
    parser.add_argument("--stages-only", action="store_true",
                        help="profiling workload for rocprofv3 --pmc: the per-stage SRNL launches and "
                             "one FP32 copy of COPY_CALIBRATION_BYTES (HBM counter calibration); "
                             "no model forward, no JSON line")
    parser.add_argument("--tail-only", action="store_true",
                        help="profiling workload for rocprofv3: the config-2 fusion, GRN and LayerNorm "
                             "launches of the `kernels` entry and the calibration copy; no JSON line")
    parser.add_argument("--config3-only", action="store_true",
                        help="profiling workload for rocprofv3: three config-3 operator forwards; no JSON line")
    parser.add_argument("--base512-only", action="store_true",
                        help="profiling workload for rocprofv3: three Base 512 B=8 feature forwards; no JSON line")
    parser.add_argument("--backward-only", action="store_true",
                        help="profiling workload for rocprofv3: the SRNL backward and the fusion, GRN and "
                             "LayerNorm backward launches of the `kernels` entry; no JSON line")
    args = parser.parse_args(argv)
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported "
              "(every GPU box in this build has a single MI355X).", file=sys.stderr)
        return 2

    import torch

    if args.stages_only:
        return profile_stages(torch.device("cuda:0"), args.batch)
    if args.config3_only:
        return profile_config3(torch.device("cuda:0"))
    if args.base512_only:
        return profile_base512(torch.device("cuda:0"))
    if args.backward_only:
        device = torch.device("cuda:0")
        rows = measure_srnl_backward(device)
        rows.update(measure_tail_backward(device))
        for name, row in rows.items():
            print(name, row, flush=True)
        return 0
    if args.tail_only:
        with torch.inference_mode():
            for name, row in measure_tail(torch.device("cuda:0")).items():
                print(name, row, flush=True)
            src = torch.ones(COPY_CALIBRATION_BYTES // 4, device="cuda:0")
            torch.mul(src, 1.0, out=torch.empty_like(src))
            torch.cuda.synchronize()
        print(f"calibration copy: {COPY_CALIBRATION_BYTES} bytes read and written", flush=True)
        return 0

    device = torch.device("cuda:0")
    torch.cuda.set_device(device)
    torch.backends.cuda.matmul.allow_tf32 = True
    torch.backends.cudnn.allow_tf32 = True
    torch.backends.cudnn.benchmark = args.cudnn_benchmark
    model = build_tiny(device)
    gen = torch.Generator().manual_seed(SEED)
    images = torch.randn(args.batch, 3, 224, 224, generator=gen).to(device)
    images = images.contiguous(memory_format=torch.channels_last)

    def forward():
        with torch.autocast("cuda", dtype=torch.bfloat16):
            return model(images)

    with torch.inference_mode():
        for _ in range(3):
            out = forward()
        torch.cuda.synchronize()
        if not torch.isfinite(out).all():
            raise FloatingPointError("Tiny forward produced NaN/Inf")
        execution = "eager"
        graph = None
        if not args.no_graph:
            try:
                graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(graph):
                    graph_out = forward()
                graph.replay()
                torch.cuda.synchronize()
                if not torch.allclose(graph_out.float(), out.float(), atol=1e-2, rtol=1e-2):
                    raise RuntimeError("graph replay disagrees with eager forward")
                execution = "hip_graph"
            except Exception as exc:  # capture unsupported by a library call: time eager
                print(f"HIP graph capture unavailable ({exc}); timing eager forwards", file=sys.stderr)
                graph = None
        audit = fast_path_audit(model, forward)
        step = graph.replay if graph is not None else forward
        for _ in range(args.warmup):
            step()
        torch.cuda.synchronize()
        stream = torch.cuda.current_stream(device)
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        start.record(stream)
        for _ in range(args.steps):
            step()
        end.record(stream)
        end.synchronize()
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        ms = start.elapsed_time(end) / args.steps
        validation = validate_graph_changed_input(graph, graph_out if graph is not None else None, forward, images)
        del graph

        stage_rows, srnl_flops_total, srnl_ms_total, srnl_bytes, srnl_compulsory = measure_srnl_stages(
            device, args.batch)
        tail = measure_tail(device)
        tail.update(measure_operator_config3(device))
        tail.update(measure_base512(device))
        tail.update(measure_srnl_backward(device))
        with torch.inference_mode(False), torch.enable_grad():   # autograd tensors, outside inference mode
            tail.update(measure_tail_backward(device))

    images_per_s = args.batch * 1000.0 / ms
    achieved = srnl_flops_total / srnl_ms_total / 1e9  # TFLOP/s
    result = {
        "metric": METRIC,
        "value": round(images_per_s, 2),
        "unit": "images/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "visionhope_tiny_classification_forward", "resolution": 224,
                   "global_batch": args.batch, "execution": execution, "autocast": "bf16",
                   "cudnn_benchmark": args.cudnn_benchmark,
                   "weights": "random-init (repo default init)", "seed": SEED,
                   "wall_s_timed_region": round(wall, 3)},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 3), "peak": BF16_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / BF16_PEAK_TFLOPS, 5), "traffic": srnl_bytes,
                     "kernel": "vh_srnl_spatial_forward (srnl_scan16_ut_kernel + srnl_readout_tile_kernel)",
                     "scope": "sum over the 29 SRNL launches of one forward (3/4/18/4 blocks at "
                              "56/28/14/7); achieved = reference FLOP count / event-timed duration; "
                              "peak = dense bf16 MFMA, the only matrix instruction the two kernels issue; "
                              "traffic = rocprofv3 FETCH_SIZE+WRITE_SIZE bytes, calibrated",
                     "srnl_ms_per_forward": round(srnl_ms_total, 3),
                     "algorithmic_gflop_per_forward": round(srnl_flops_total / 1e9, 2),
                     "compulsory_bytes_per_forward": srnl_compulsory,
                     "traffic_over_compulsory": (round(srnl_bytes / srnl_compulsory, 3) if srnl_bytes else None),
                     "fp32_equivalent": {"peak": FP32_PEAK_TFLOPS, "frac": round(achieved / FP32_PEAK_TFLOPS, 5),
                                         "issue_factor": 3,
                                         "note": "the recurrence computes in FP32: every FP32 product is "
                                                 "issued as three bf16 MFMAs (hi*hi + hi*lo + lo*hi), so "
                                                 "this is the rate against the FP32 matrix peak the same "
                                                 "arithmetic would have on FP32 MFMA"}},
        "kernels": {"srnl_stages": stage_rows, **tail},
        "graph_validation": validation,
        "audit": audit,
    }
    if not args.skip_cpu:
        result["cpu_baseline"] = cpu_baseline()
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
