"""Build libvisionhope_hip.so (gfx950) in-tree with hipcc.

Usage: ``python -m visionhope_amd.csrc.build`` or ``build()`` from Python.
The library lands in ``visionhope_amd/_lib/`` (git-ignored, shipped with the
tree).  Objects are compiled in parallel; every call recompiles.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

CSRC = Path(__file__).resolve().parent
PKG = CSRC.parent
LIB_DIR = PKG / "_lib"
LIB_NAME = "libvisionhope_hip.so"
SOURCES = ("vh_common.hip", "srnl.hip", "elementwise.hip", "dwconv.hip", "pointwise.hip", "conv3x3.hip", "srnl_backward.hip",
           "tail_backward.hip", "srnl_noalloc.hip", "srnl_wide.hip", "srnl_ut.hip", "srnl_utw.hip",
           "srnl_utw32.hip")
ARCH = os.environ.get("VISIONHOPE_OFFLOAD_ARCH", "gfx950")

# Packed-fp32 VALU ops are disabled for all device code (hipcc's host pass
# warns that it does not know the feature; that is expected).
HIPCC_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
]


def _hipcc():
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found; ROCm is required to build libvisionhope_hip.so")
    return path


def _torch_lib_dir():
    try:
        import torch  # noqa: F401  (only to locate its bundled HIP runtime)
        return str(Path(torch.__file__).resolve().parent / "lib")
    except Exception:
        return None


def build(verbose: bool = False) -> Path:
    """Compile every HIP source for gfx950 and link the shared library."""
    hipcc = _hipcc()
    obj_dir = LIB_DIR / "obj"
    obj_dir.mkdir(parents=True, exist_ok=True)

    def compile_one(name):
        src = CSRC / name
        obj = obj_dir / (src.stem + ".o")
        cmd = [hipcc, *HIPCC_FLAGS, "-c", str(src), "-o", str(obj)]
        proc = subprocess.run(cmd, capture_output=True, text=True)
        if proc.returncode != 0:
            raise RuntimeError(f"hipcc failed for {name}:\n{proc.stdout}\n{proc.stderr}")
        noise = "is not a recognized feature for this target"
        msgs = [ln for ln in (proc.stdout + proc.stderr).splitlines() if noise not in ln and ln.strip()]
        if verbose and msgs:
            print("\n".join(msgs), file=sys.stderr)
        return obj

    with ThreadPoolExecutor(max_workers=min(len(SOURCES), 4)) as pool:
        objs = list(pool.map(compile_one, SOURCES))

    out = LIB_DIR / LIB_NAME
    tmp = LIB_DIR / (LIB_NAME + ".tmp")
    link = [hipcc, "-shared", "-fPIC", f"--offload-arch={ARCH}", *map(str, objs), "-o", str(tmp)]
    torch_lib = _torch_lib_dir()
    if torch_lib:
        # Resolve the HIP runtime that torch bundles, so one runtime serves both.
        link += [f"-Wl,-rpath,{torch_lib}"]
    proc = subprocess.run(link, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    print(build(verbose=True))
