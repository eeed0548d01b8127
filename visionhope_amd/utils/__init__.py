"""Shared numerical utilities for VisionHOPE inference on MI355X."""

from .grn import GlobalResponseNorm, global_response_norm, grn_reference

__all__ = ["GlobalResponseNorm", "global_response_norm", "grn_reference"]
