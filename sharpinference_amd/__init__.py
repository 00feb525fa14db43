"""MI355X (gfx950) backend for SharpInference's quantized matrix-vector hot path.

The compute lives in ``libsharpinference_hip.so`` (hand-written HIP for
gfx950, C ABI in ``include/sharpinference_hip.h``); ``native`` binds it.
"""
from . import native  # noqa: F401

__all__ = ["native"]
