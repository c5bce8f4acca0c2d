"""The layer projections y = x . W^T on the GPU through the C ABI (fqa_gemm; LaunchGemm,
engine/src/kernels.cu:9-16), torch tensors as device memory."""
from __future__ import annotations

import torch

from ._lib import check, load

_ws: dict[torch.device, torch.Tensor] = {}


def workspace_bytes(M: int, N: int, K: int) -> int:
    return int(load().fqa_gemm_workspace_bytes(M, N, K))


def _workspace(dev: torch.device, nbytes: int) -> torch.Tensor | None:
    if nbytes == 0:
        return None
    ws = _ws.get(dev)
    if ws is None or ws.numel() < nbytes:
        ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
        _ws[dev] = ws
    return ws


def gemm(x: torch.Tensor, w: torch.Tensor, out: torch.Tensor | None = None,
         out_f32: bool = False, workspace: torch.Tensor | None = None) -> torch.Tensor:
    """x [M, K] bf16, w [N, K] bf16 (row strides allowed) -> y [M, N] bf16 (fp32 with
    out_f32), on the current stream."""
    if x.dtype != torch.bfloat16 or w.dtype != torch.bfloat16 or x.dim() != 2 or w.dim() != 2:
        raise ValueError("x and w must be 2-D bf16 tensors")
    if x.stride(1) != 1 or w.stride(1) != 1:
        raise ValueError("x and w need unit column stride")
    M, K = x.shape
    N, K2 = w.shape
    if K != K2:
        raise ValueError(f"inner sizes differ: {K} vs {K2}")
    dt = torch.float32 if out_f32 else torch.bfloat16
    if out is None:
        out = torch.empty(M, N, dtype=dt, device=x.device)
    elif out.dtype != dt or out.shape != (M, N) or out.stride(1) != 1:
        raise ValueError("out has the wrong dtype, shape or column stride")
    need = workspace_bytes(M, N, K)
    if workspace is None:
        workspace = _workspace(x.device, need)
    ws_ptr = workspace.data_ptr() if workspace is not None else None
    ws_len = workspace.numel() * workspace.element_size() if workspace is not None else 0
    stream = torch.cuda.current_stream(x.device).cuda_stream
    check(load().fqa_gemm(x.data_ptr(), x.stride(0), w.data_ptr(), w.stride(0), out.data_ptr(),
                          out.stride(0), M, N, K, int(out_f32), ws_ptr, ws_len, stream),
          "fqa_gemm")
    return out


def gemm_argmax(x: torch.Tensor, w: torch.Tensor, out: torch.Tensor | None = None,
                workspace: torch.Tensor | None = None) -> torch.Tensor:
    """Greedy tokens of x . W^T (lm_head + argmax, smallest index on ties) without writing
    the logits: x [M, K] bf16, w [N, K] bf16 -> [M] int32, on the current stream."""
    if x.dtype != torch.bfloat16 or w.dtype != torch.bfloat16 or x.dim() != 2 or w.dim() != 2:
        raise ValueError("x and w must be 2-D bf16 tensors")
    if x.stride(1) != 1 or w.stride(1) != 1 or x.shape[1] != w.shape[1]:
        raise ValueError("x and w need unit column stride and equal inner sizes")
    M, K = x.shape
    N = w.shape[0]
    if out is None:
        out = torch.empty(M, dtype=torch.int32, device=x.device)
    lib = load()
    need = int(lib.fqa_gemm_argmax_workspace_bytes(M, N, K))
    if workspace is None:
        workspace = _workspace(x.device, max(need, 16))
    ws_len = workspace.numel() * workspace.element_size()
    stream = torch.cuda.current_stream(x.device).cuda_stream
    check(lib.fqa_gemm_argmax(x.data_ptr(), x.stride(0), w.data_ptr(), w.stride(0), M, N, K,
                              out.data_ptr(), workspace.data_ptr(), ws_len, stream),
          "fqa_gemm_argmax")
    return out
