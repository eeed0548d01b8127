"""Autograd plumbing shared by the native wrappers.

The SRNL packed paths (raw and normalised queries, chunks of at most 64) have native
backward kernels (``vh_srnl_backward``).  The other Functions are forward-only and raise
a clear error if a gradient is requested instead of silently producing wrong gradients.
"""


def backward_unavailable(name):
    raise NotImplementedError(
        f"{name}: this path is forward-only in the MI355X build; its backward kernels "
        "(reference lines.cu:252-760, direction_fusion.cu:123-691, grn_cuda.cu:126-359, "
        "layer_norm_cuda.py:59-192) are not ported yet")
