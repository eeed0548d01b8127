"""VisionHOPE models and reusable components on MI355X (mirrors ``models/__init__.py``)."""

from .srnl import SRNL
from .operator import VisionHOPEOperator
from .block import VisionHOPEBlock
from .hierarchical import HierarchicalVisionHOPE
from .factory import MODEL_CONFIGS, create_model

__all__ = ["SRNL", "VisionHOPEOperator", "VisionHOPEBlock", "HierarchicalVisionHOPE",
           "MODEL_CONFIGS", "create_model"]
