"""flashqwen_amd — MI355X (gfx950) per-step attention path of the FlashQwen engine.

Pack -> fused QK-norm/RoPE/paged append -> split-K decode + varlen FA-2 prefill, as
hand-written HIP behind the C ABI in include/fqa.h (libfqa.so); around it the layer
projections (fqa_gemm, and the QKV projection fused with the append) and token sampling.

Python entry points (torch tensors as device memory, all calls through the C ABI):
  step.AttnStep      the per-step context: pack, append, decode, prefill
  gemm.gemm          y = x . W^T (LaunchGemm)
  sample.sample      greedy / temperature / top-p sampling (LaunchSampleBatch)
"""
from ._lib import LIB_PATH, FqaError, load  # noqa: F401

__all__ = ["LIB_PATH", "FqaError", "load"]
