"""fqa_qkv_proj_append (the QKV projection fused with the norm/RoPE/append of a6-a7,
model_runtime.cu:261-268) against the unfused path on the GPU: fqa_gemm into a bf16 qkv
buffer, then fqa_qknorm_rope_append.  The two must agree bit for bit on q (and k with
write_k) in qkv and on every pool byte, for split-K row counts (the append then reads
the fp32 partials) and for an unsplit one.  Rows cover full pages (the transposed V
store), partly filled pages, a position outside the RoPE table and a slot outside the
pool."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest


def _case(gpu, M, K, write_k, seed, rows=None):
    import torch

    from flashqwen_amd import _lib
    from flashqwen_amd.gemm import gemm, workspace_bytes
    from flashqwen_amd.step import alloc_pool, make_dims, rope_tables

    print(f"[qkv_fused] M={M} K={K} write_k={write_k} rows={rows}", flush=True)
    lib = _lib.load()
    rng = np.random.default_rng(seed)
    P, max_pos = 64 + M // 8, 4096
    x = (torch.from_numpy(rng.standard_normal((M, K)).astype(np.float32))).to(torch.bfloat16).to(gpu)
    w = (torch.from_numpy(rng.standard_normal((6144, K)).astype(np.float32)) * 0.03).to(
        torch.bfloat16).to(gpu)
    qn = torch.from_numpy(rng.uniform(0.5, 1.5, 128).astype(np.float32)).to(gpu)
    kn = torch.from_numpy(rng.uniform(0.5, 1.5, 128).astype(np.float32)).to(gpu)
    cos, sin = rope_tables(max_pos)
    cos, sin = torch.from_numpy(cos).to(gpu), torch.from_numpy(sin).to(gpu)
    # rows 0..31: two full pages (slots 32..63); the rest: distinct random slots
    pos = rng.integers(0, max_pos, M).astype(np.int32)
    pos[:32] = np.arange(100, 132)
    slots = np.empty(M, np.int32)
    slots[:32] = np.arange(32, 64)
    rest = rng.permutation(np.arange(64, P * 16))[: M - 32]
    slots[32:] = rest
    if M >= 300:
        # full pages inside a 256-row tile (rows 96..111) and across its end (rows 248..263):
        # whole-page V^T stores in the fused epilogue only where the page is in one tile
        for r0, page in ((96, P - 3), (248, P - 2)):
            pos[r0:r0 + 16] = np.arange(512, 528)
            slots[r0:r0 + 16] = np.arange(page * 16, page * 16 + 16)
        slots[32:] = np.where(np.isin(slots[32:], np.arange((P - 3) * 16, (P - 1) * 16)) &
                              ~np.isin(np.arange(32, M), np.r_[96:112, 248:264]),
                              -1, slots[32:])
    if rows is not None:
        # a full page across the row count (rows rows-10 .. rows+5): its rows below the count
        # are appended as a partly filled page, the rest not at all
        r0, page = rows - 10, P - 4
        pos[r0:r0 + 16] = np.arange(700, 716)
        slots[r0:r0 + 16] = np.arange(page * 16, page * 16 + 16)
        other = np.ones(M, bool)
        other[r0:r0 + 16] = False
        slots[other & (slots // 16 == page)] = -1
    pos[M // 2] = max_pos + 5          # no table row
    slots[M // 3] = P * 16 + 40        # page outside the pool
    pos_t = torch.from_numpy(pos).to(gpu)
    slot_t = torch.from_numpy(slots).to(gpu)
    meta = torch.zeros(16, dtype=torch.int32, device=gpu)
    T = M if rows is None else rows
    meta[_lib.META_ROWS] = T
    dims = make_dims()

    qkv_a = torch.full((M, 6144), 3.0, dtype=torch.bfloat16, device=gpu)
    pool_a = alloc_pool(P)[0].zero_()
    gemm(x, w, out=qkv_a)
    _lib.check(lib.fqa_qknorm_rope_append(
        C.byref(dims), qkv_a.data_ptr(), qn.data_ptr(), kn.data_ptr(), cos.data_ptr(),
        sin.data_ptr(), max_pos, pos_t.data_ptr(), slot_t.data_ptr(), meta.data_ptr(), M,
        pool_a.data_ptr(), P, int(write_k), None), "append")

    qkv_b = torch.full((M, 6144), 3.0, dtype=torch.bfloat16, device=gpu)
    pool_b = alloc_pool(P)[0].zero_()
    nb = workspace_bytes(M, 6144, K)
    ws = torch.empty(max(nb, 16), dtype=torch.uint8, device=gpu)
    _lib.check(lib.fqa_qkv_proj_append(
        C.byref(dims), x.data_ptr(), K, w.data_ptr(), K, M, K, qkv_b.data_ptr(), qn.data_ptr(),
        kn.data_ptr(), cos.data_ptr(), sin.data_ptr(), max_pos, pos_t.data_ptr(),
        slot_t.data_ptr(), meta.data_ptr(), pool_b.data_ptr(), P, int(write_k),
        ws.data_ptr() if nb else None, nb, None), "fqa_qkv_proj_append")
    torch.cuda.synchronize()
    ncols = 5120 if write_k else 4096
    a16 = qkv_a.view(torch.int16)[:T, :ncols].cpu().numpy()
    b16 = qkv_b.view(torch.int16)[:T, :ncols].cpu().numpy()
    assert np.array_equal(a16, b16), int((a16 != b16).sum())
    # rows at or past the row count: the fused path leaves qkv untouched (the unfused
    # projection writes every row it is given)
    rest = qkv_b[T:].float().cpu().numpy()
    assert np.all(rest == 3.0), int((rest != 3.0).sum())
    pa = pool_a.view(torch.int16).cpu().numpy()
    pb = pool_b.view(torch.int16).cpu().numpy()
    assert np.array_equal(pa, pb), int((pa != pb).sum())
    assert np.any(pa != 0)
    return nb


@pytest.mark.gpu
@pytest.mark.parametrize("M,K,write_k", [(40, 1024, 0), (256, 1024, 1), (256, 4096, 0),
                                         (1000, 1024, 1), (1300, 512, 0), (2100, 1024, 1),
                                         (8192, 4096, 0)])
def test_qkv_fused_equals_unfused(gpu, M, K, write_k):
    """Split row counts: the append kernel reads the projection's partials.  Unsplit ones
    (1000 rows on 256 x 128 tiles, 1300 and more on 256 x 256 tiles): the projection's
    epilogue does the norm, RoPE and append itself."""
    nb = _case(gpu, M, K, write_k, seed=M + K)
    if M <= 256:
        assert nb > 0  # the split path (partials read by the append kernel) was exercised
    else:
        assert nb == 0


@pytest.mark.gpu
@pytest.mark.parametrize("M,rows", [(1300, 1290), (1000, 990)])
def test_qkv_fused_rows_below_m(gpu, M, rows):
    """Unsplit tiles (256 x 256 at 1300 rows, 256 x 128 at 1000) with the pack's row
    count below M inside the last tile: rows at or past it are neither normalised nor
    appended, and a page that the count cuts is appended as a partly filled one; the
    pool equals the unfused path's byte for byte."""
    nb = _case(gpu, M, 1024, 0, seed=M + 7, rows=rows)
    assert nb == 0
