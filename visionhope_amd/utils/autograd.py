"""Autograd plumbing shared by the native wrappers.

The SRNL packed paths (raw and normalised queries, rectangular row/column scans, long
lines, chunks of at most 256), direction fusion, GRN, LayerNorm2d, the query
normalisation and the residual add have native backward kernels.  Chunks above 256 are
forward-only and raise a clear error if a gradient is requested instead of silently
producing wrong gradients.
"""


def backward_unavailable(name):
    raise NotImplementedError(
        f"{name}: this path is forward-only in the MI355X build; its backward kernels "
        "for chunks above 256 tokens are not built")
