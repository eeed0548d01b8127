"""Write the SRNL golden fixtures from the fp64 CPU oracle.

The reference ships no golden vectors and cannot run here (CUDA-only SRNL), so these
fixtures are produced by the build's own fp64 oracle (oracle/srnl_oracle.c), which the
CPU tests pin independently.  They freeze the expected outputs so that the GPU kernels
and any later change of the oracle are checked against the same numbers.

    python tests/golden/make_fixtures.py
"""

import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import oracle  # noqa: E402
from tests.helpers import memories  # noqa: E402

OUT = Path(__file__).resolve().parent


def config1():
    """Standalone SRNL: B=2, 14x14 tokens (L=196), C=64 in 2 heads of 32, chunk 14."""
    rng = np.random.default_rng(1234)
    x = rng.normal(size=(2, 196, 64)).astype(np.float32)
    out = {}
    for kind in ("default", "perturbed"):
        mems = memories(1, 2, 32, kind=kind, seed=1234)
        packed = x.reshape(2, 1, 196, 2, 32).transpose(0, 1, 3, 2, 4)
        y = oracle.sequence_forward(packed, x.reshape(2, 1, 196, 64), mems, [14], dtype=np.float64)
        out[kind] = (mems, y[:, 0].transpose(0, 2, 1, 3).reshape(2, 196, 64).astype(np.float32))
    np.savez_compressed(OUT / "srnl_config1.npz", x=x,
                        **{f"{k}_{n}": v for k, (mems, y) in out.items()
                           for n, v in list(zip(("M_m", "M_v", "M_k", "M_eta", "M_alpha"), mems))
                           + [("y", y)]})


def operator7x7():
    """Four-direction operator, B=2, 7x9 image, C=32 in 2 heads of 16, strong parameters."""
    rng = np.random.default_rng(77)
    x = rng.normal(size=(2, 7, 9, 32)).astype(np.float32)
    q = rng.normal(size=(2, 7, 9, 32)).astype(np.float32)
    mems = memories(4, 2, 16, kind="strong", seed=77)
    skip = (rng.normal(size=(4, 32)) * 0.1).astype(np.float32)
    w = (1 + rng.normal(size=(4, 32)) * 0.1).astype(np.float32)
    out = oracle.operator_forward(x, q, mems, skip, w, 16, dtype=np.float64).astype(np.float32)
    np.savez_compressed(OUT / "operator_7x9.npz", x=x, q=q, M_m=mems[0], M_v=mems[1], M_k=mems[2],
                        M_eta=mems[3], M_alpha=mems[4], d_skip=skip, weights=w, out=out)


if __name__ == "__main__":
    config1()
    operator7x7()
    for p in sorted(OUT.glob("*.npz")):
        print(p.name, p.stat().st_size)
