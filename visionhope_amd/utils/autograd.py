"""Forward-only autograd plumbing shared by the native wrappers.

The MI355X build ports the forward (inference) hot path.  Backward kernels are
not part of it, so each Function raises a clear error if a gradient is
requested instead of silently producing wrong gradients.
"""


def backward_unavailable(name):
    raise NotImplementedError(
        f"{name}: the MI355X build implements the forward pass only; backward kernels "
        "(reference chunk.cu:511-1057, lines.cu:252-760, direction_fusion.cu:123-691, "
        "grn_cuda.cu:126-359) are not ported yet")
