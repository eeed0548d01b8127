"""FP32-state SRNL recurrence on MI355X (mirrors ``models/srnl_core/__init__.py``).

The public trainable module is :class:`visionhope_amd.models.SRNL`.  These
functions expose the packed recurrence used by that module and its
directional operator.
"""

from .chunk import MAX_CHUNK, SUPPORTED_HEAD_DIMS, srnl_normalized_query, srnl_raw_query
from .lines import srnl_long_chunk, srnl_variable_lines

__all__ = [
    "MAX_CHUNK", "SUPPORTED_HEAD_DIMS", "srnl_normalized_query", "srnl_raw_query",
    "srnl_long_chunk", "srnl_variable_lines",
]
