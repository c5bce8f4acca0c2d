"""flashqwen_amd — MI355X (gfx950) per-step attention path of the FlashQwen engine.

Pack -> fused QK-norm/RoPE/paged append -> split-K decode + varlen FA-2 prefill, as
hand-written HIP behind the C ABI in include/fqa.h (libfqa.so).
"""
from ._lib import LIB_PATH, FqaError, load  # noqa: F401

__all__ = ["LIB_PATH", "FqaError", "load"]
