"""Token sampling on the GPU through the C ABI (fqa_sample; LaunchSampleBatch,
engine/src/kernels.cu:184-327): greedy rows (inv_temp <= 0) and temperature + top-p rows
with the caller's uniform draws, torch tensors as device memory."""
from __future__ import annotations

import torch

from ._lib import check, load


def _ptr(t: torch.Tensor):
    return t.data_ptr()


def sample(logits: torch.Tensor, inv_temp: torch.Tensor, top_p: torch.Tensor,
           u: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """logits [B, N] fp32 (rows may be strided), inv_temp / top_p / u [B] fp32 -> [B] int32
    tokens, on the current stream."""
    if logits.dtype != torch.float32 or logits.dim() != 2 or logits.stride(1) != 1:
        raise ValueError("logits must be a 2-D fp32 tensor with unit column stride")
    B, N = logits.shape
    for name, t in (("inv_temp", inv_temp), ("top_p", top_p), ("u", u)):
        if t.dtype != torch.float32 or t.shape != (B,) or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous fp32 tensor of shape ({B},)")
    if out is None:
        out = torch.empty(B, dtype=torch.int32, device=logits.device)
    stream = torch.cuda.current_stream(logits.device).cuda_stream
    check(load().fqa_sample(_ptr(logits), B, N, logits.stride(0), _ptr(inv_temp), _ptr(top_p),
                            _ptr(u), _ptr(out), stream), "fqa_sample")
    return out
