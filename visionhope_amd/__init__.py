"""VisionHOPE SRNL operator hot path, native to AMD MI355X (gfx950).

Mirrors the reference package layout (``visionhope.models``, ``visionhope.utils``,
``visionhope.inference.prepare``); the arithmetic runs in ``_lib/libvisionhope_hip.so``
(C ABI: ``include/visionhope_hip.h``).
"""

__version__ = "0.1.0"
