"""Audits of the prepared inference forward (reference ``inference/audit.py:11-99`` and
``analysis/benchmark.py:48-71``): every VisionHOPE operator projects its queries exactly
once per call, and every operator call runs exactly one fused SRNL scan and one readout.

``ModelAudit`` keeps the reference's hook structure: a forward pre-hook on each
operator's owning block records the input shape and counts calls, a forward pre-hook on
``W_q`` checks that the projection covers B*H*W tokens once, and standalone SRNL modules
are counted.  The fused block path computes W_q with the native 1x1 kernel instead of
calling the module, and runs W_q's registered forward pre-hooks with the tensor it
projects (``models/block.py``), so the hooks see the same projection either way.

``count_srnl_launches`` counts the library's scan and readout kernels in a
``torch.profiler`` trace of one forward and compares both with the audited calls.
"""

from __future__ import annotations

import torch

from ..models.block import VisionHOPEBlock
from ..models.operator import VisionHOPEOperator
from ..models.srnl import SRNL
from ..utils.grn import GlobalResponseNorm

# Kernel families of libvisionhope_hip.so: one scan and one readout per SRNL call.
SCAN_KERNELS = ("srnl_scan16_ut_kernel", "srnl_scan16_utw_kernel", "srnl_scan32_utw_kernel", "srnl_scan16_kernel",
                "srnl_scanw_kernel", "srnl_scan_kernel")
READOUT_KERNELS = ("srnl_readout_tile_kernel", "srnl_fuse_readout_kernel", "srnl_packed_readout_kernel")


class ModelAudit:
    def __init__(self, model):
        self.handles = []
        self.query = {}
        self.grn = {}
        self.srnl = {}
        self.shapes = {}
        self.operator_calls = {}
        self.expected_queries = set()
        self.expected_srnl = set()
        modules = list(model.named_modules())
        owners = {id(module.operator): (name, module) for name, module in modules
                  if isinstance(module, VisionHOPEBlock)}
        nested_srnl = {id(module.srnl) for _, module in modules if isinstance(module, VisionHOPEOperator)}
        self.block_count = len(owners)
        for name, module in modules:
            if isinstance(module, VisionHOPEOperator):
                owner_name, owner = owners.get(id(module), (name, module))
                self.expected_queries.add(owner_name)
                self.handles.append(owner.register_forward_pre_hook(self._input_hook(owner_name), with_kwargs=True))
                self.handles.append(module.W_q.register_forward_pre_hook(self._query_hook(owner_name)))
            if isinstance(module, SRNL) and id(module) not in nested_srnl:
                self.expected_srnl.add(name)
                self.handles.append(module.register_forward_pre_hook(self._srnl_hook(name), with_kwargs=True))
            if isinstance(module, GlobalResponseNorm):
                self.handles.append(module.register_forward_hook(self._grn_hook(name)))

    def _input_hook(self, name):
        def hook(module, inputs, kwargs):
            x = inputs[0] if inputs else kwargs["x"]
            self.shapes[name] = list(x.shape)
            self.operator_calls[name] = self.operator_calls.get(name, 0) + 1
        return hook

    def _query_hook(self, name):
        def hook(module, inputs):
            shape = self.shapes[name]
            projected = inputs[0].numel() // inputs[0].shape[-1]
            spatial = shape[0] * shape[-2] * shape[-1]
            if projected != spatial:
                raise RuntimeError(f"Query-once audit failed for {name}: {projected} != {spatial}")
            previous = self.query.get(name, {"call_count": 0, "projected_tokens": 0, "spatial_tokens": 0})
            self.query[name] = {"input_shape": shape, "query_input": list(inputs[0].shape),
                                "call_count": previous["call_count"] + 1,
                                "projected_tokens": previous["projected_tokens"] + projected,
                                "spatial_tokens": previous["spatial_tokens"] + spatial}
        return hook

    def _srnl_hook(self, name):
        def hook(module, inputs, kwargs):
            x = inputs[0] if inputs else kwargs["x"]
            previous = self.srnl.get(name, {"call_count": 0})
            self.srnl[name] = {"input_shape": list(x.shape), "call_count": previous["call_count"] + 1}
        return hook

    def _grn_hook(self, name):
        # GRN modules called as modules must return FP32 (the reference's precision check);
        # the fused block path applies GRN inside fc2 and never calls the module.
        def hook(module, inputs, output):
            if output.dtype != torch.float32:
                raise RuntimeError(f"GRN output must be FP32: {name} returned {output.dtype}")
            self.grn[name] = {"input_dtype": str(inputs[0].dtype), "output_dtype": str(output.dtype),
                              "shape": list(inputs[0].shape)}
        return hook

    def close(self):
        for handle in self.handles:
            handle.remove()
        self.handles.clear()

    def finish(self):
        self.close()
        if not self.expected_queries and not self.expected_srnl:
            raise RuntimeError("No VisionHOPE operator or SRNL instance was found")
        if set(self.query) != self.expected_queries:
            raise RuntimeError("Not every VisionHOPE query projection was observed during evaluation")
        if set(self.srnl) != self.expected_srnl:
            raise RuntimeError("Not every standalone SRNL instance was observed during evaluation")
        if any(record["call_count"] != self.operator_calls[name]
               or record["projected_tokens"] != record["spatial_tokens"]
               for name, record in self.query.items()):
            raise RuntimeError("A VisionHOPE operator did not project its input exactly once per call")
        return {"query_audit": self.query, "grn_audit": self.grn, "srnl_audit": self.srnl}


def _kernel_family(name, families):
    return any(family in name for family in families)


def audit_fast_path(model, forward):
    """Runs ``forward()`` once under ``ModelAudit`` and ``torch.profiler`` and checks that
    the scan and readout launches both equal the audited SRNL calls (operator calls plus
    standalone SRNL calls).  Returns the evidence; raises on any mismatch."""
    audit = ModelAudit(model)
    activities = [torch.profiler.ProfilerActivity.CPU, torch.profiler.ProfilerActivity.CUDA]
    try:
        with torch.profiler.profile(activities=activities) as profile:
            output = forward()
            torch.cuda.synchronize()
        evidence = audit.finish()
    finally:
        audit.close()
    names = [event.name for event in profile.events()
             if getattr(event, "device_type", None) == torch.autograd.DeviceType.CUDA]
    if not names:
        raise RuntimeError("The profiler recorded no GPU kernels; the launch audit cannot run")
    scans = sum(_kernel_family(n, SCAN_KERNELS) for n in names)
    readouts = sum(_kernel_family(n, READOUT_KERNELS) for n in names)
    expected = sum(record["call_count"] for key in ("query_audit", "srnl_audit")
                   for record in evidence[key].values())
    if scans != expected or readouts != expected:
        raise RuntimeError(f"Expected {expected} SRNL scans and readouts, observed {scans} and {readouts}")
    # separate 5x5 depthwise launches (the position encoding when the readout does not
    # compute it)
    lepe_passes = sum(1 for n in names if "dwconv_nhwc_kernel<5" in n or "dwconv_tile_kernel<5" in n)
    return output, {"fused_blocks": audit.block_count, "fused_operators": len(evidence["query_audit"]),
                    "fused_srnl_calls": expected, "query_once": True if evidence["query_audit"] else None,
                    "scan_kernels": scans, "readout_kernels": readouts, "gpu_kernels": len(names),
                    "separate_lepe_kernels": lepe_passes, "grn_modules_fp32": len(evidence["grn_audit"])}
