"""Host-side mirror of the reference's per-step attention interface, over libfqa.so.

The reference engine drives the path from C++ (engine/src/model_runtime.cu):

    StepContext::PrepareInputs(in, rng, stream)               once per step  (:295-302)
    per layer l:
      LaunchHeadNormRope(qkv, q_norm, k_norm, cos, sin, pos, ...)            (:263-265)
      KvStore::StoreKV(l, qkv, bt, bt_stride, req, pos, M, stream)           (:267-268)
      LaunchAttnDecodeCute(qkv, ..., pm, pl, pa, stream)                     (:269-273)
      LaunchAttnPrefillCute(qkv, ..., stream)                                (:274-278)

`AttnStep` keeps that shape: `prepare_inputs` (or `schedule_and_prepare`, which also runs
the token-budget selection on the GPU) once per step, then `run_layer` per layer, which
issues fqa_qknorm_rope_append (the first two calls fused), fqa_decode and fqa_prefill.
PyTorch is used only to own device memory and to name the stream; all work is in the HIP
library.  Buffers are sized once at construction to the worst case, as StepContext does
(model_runtime.cu:160-174), so no step allocates.
"""
from __future__ import annotations

import ctypes as C
import math

import numpy as np
import torch

from . import _lib
from ._lib import FqaBatch, FqaDims, FqaPackCfg, FqaPackOut, check
from .synth import HEAD_DIM, N_KV, N_Q, PAGE, QKV_STRIDE, RMS_EPS, ROPE_THETA


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def make_dims(qkv_stride: int = QKV_STRIDE) -> FqaDims:
    return FqaDims(N_Q, N_KV, HEAD_DIM, PAGE, qkv_stride, RMS_EPS, 1.0 / math.sqrt(HEAD_DIM))


def rope_tables(max_pos: int, theta: float = ROPE_THETA) -> tuple[np.ndarray, np.ndarray]:
    """cos/sin [max_pos][64] float tables built by the library (RopeTables::Build)."""
    lib = _lib.load()
    cos = np.empty((max_pos, HEAD_DIM // 2), np.float32)
    sin = np.empty_like(cos)
    check(lib.fqa_rope_tables(max_pos, HEAD_DIM, theta, cos.ctypes.data, sin.ctypes.data),
          "fqa_rope_tables")
    return cos, sin


def pool_bytes(pages: int) -> int:
    return int(_lib.load().fqa_pool_bytes(C.byref(make_dims()), pages))


def alloc_pool(pages: int, layers: int = 1, device="cuda") -> torch.Tensor:
    """[layers, pages, kv_heads, 2, 16, 128] bf16 pool; one contiguous 8 KiB run per
    (layer, page, kv head): K [16][128] then V^T [128][16]."""
    return torch.empty((layers, pages, N_KV, 2, PAGE, HEAD_DIM), dtype=torch.bfloat16,
                       device=device)


class AttnStep:
    """Per-step context + per-layer launches of the attention path (one GPU, one stream)."""

    def __init__(self, *, max_rows: int, max_reqs: int, max_ctx: int, pool_pages: int,
                 device="cuda", dec_grid_waves: int | None = None, dec_min_pages: int = 8,
                 pre_tile_q: int = _lib.FQA_PRE_TILE_Q, max_bt_pages: int | None = None,
                 dec_share: bool = False, dec_prefix_pages: int = 0, dec_pre_cap: int = 4096):
        """dec_share: run_layer will be given a side stream, so a step with both decode
        and prefill rows plans its decode for the CUs the prefill leaves (fqa.h).
        dec_prefix_pages > 0: decode sequences sharing a prefix of at least that many pages
        attend it once per group (fqa.h, dec_prefix_pages), with up to dec_pre_cap prefix
        items per step (past that the step plans without groups)."""
        self.lib = _lib.load()
        if max_reqs > _lib.FQA_MAX_REQS:
            raise ValueError(f"max_reqs {max_reqs} > {_lib.FQA_MAX_REQS}")
        self.device = torch.device(device)
        self.dims = make_dims()
        self.max_rows, self.max_reqs, self.max_ctx = max_rows, max_reqs, max_ctx
        self.pool_pages = pool_pages
        self.max_blocks = -(-max_ctx // PAGE)
        self.pre_tile_q = pre_tile_q
        if dec_grid_waves is None:  # fill the device: one decode wave per SIMD
            dec_grid_waves = int(self.lib.fqa_dec_default_waves(self.device.index or 0)) or 1024
        self.dec_grid_waves = dec_grid_waves
        self.dec_wave_cap = int(self.lib.fqa_dec_wave_bound(max_reqs, dec_grid_waves))
        self.pre_cap = int(self.lib.fqa_pre_item_bound(max_reqs, max_rows, pre_tile_q))
        self.dec_share = bool(dec_share)
        self.dec_prefix_pages = int(dec_prefix_pages)
        self.dec_pre_cap = int(dec_pre_cap) if dec_prefix_pages > 0 else 0
        self.cfg = FqaPackCfg(max_rows, self.max_blocks, pool_pages, dec_grid_waves,
                              dec_min_pages, self.dec_wave_cap, pre_tile_q, self.pre_cap,
                              int(dec_share), self.dec_prefix_pages, self.dec_pre_cap)
        i32 = dict(dtype=torch.int32, device=self.device)
        R = max_reqs
        self.cu_seqlens = torch.zeros(R + 1, **i32)
        self.qlen = torch.zeros(R, **i32)
        self.positions = torch.zeros(max(max_rows, 1), **i32)
        self.row_req = torch.zeros(max(max_rows, 1), **i32)
        self.slot_mapping = torch.zeros(max(max_rows, 1), **i32)
        self.block_tables = torch.full((R, self.max_blocks), -1, **i32)
        self.decode_rids = torch.zeros(R, **i32)
        self.prefill_rids = torch.zeros(R, **i32)
        self.dec_seqs = torch.zeros((max(R, 1), 4), **i32)
        self.dec_waves = torch.zeros((max(self.dec_wave_cap, 1), 8), **i32)
        self.pre_items = torch.zeros((max(self.pre_cap, 1), 4), **i32)
        self.meta = torch.zeros(_lib.META_LEN, **i32)
        self.dec_prefix = torch.zeros((max(R, 1), 8), **i32)
        self.dec_pre_items = torch.zeros((max(self.dec_pre_cap, 1), 12), **i32)
        ws = int(self.lib.fqa_decode_prefix_workspace_bytes(C.byref(self.dims), self.dec_wave_cap,
                                                            self.dec_pre_cap))
        self.workspace = torch.empty(max(ws, 16), dtype=torch.uint8, device=self.device)
        cos, sin = rope_tables(max_ctx)
        self.cos = torch.from_numpy(cos).to(self.device)
        self.sin = torch.from_numpy(sin).to(self.device)
        self.out_struct = FqaPackOut(*[
            _ptr(t) for t in (self.cu_seqlens, self.qlen, self.positions, self.row_req,
                              self.slot_mapping, self.block_tables, self.decode_rids,
                              self.prefill_rids, self.dec_seqs, self.dec_waves,
                              self.pre_items, self.meta, self.dec_prefix,
                              self.dec_pre_items)])
        # device-side selection buffers (schedule_and_prepare)
        self.max_bt_pages = max_bt_pages if max_bt_pages is not None else R * self.max_blocks
        self.sel_req = torch.zeros(R, **i32)
        self.sel_n = torch.zeros(R, **i32)
        self.n_sel = torch.zeros(1, **i32)
        self.b_computed = torch.zeros(R, **i32)
        self.b_n_new = torch.zeros(R, **i32)
        self.b_bt_off = torch.zeros(R + 1, **i32)
        self.b_bt_pages = torch.zeros(max(self.max_bt_pages, 1), **i32)
        self.n_reqs_bound = 0
        self.rows_bound = 0

    @property
    def stream(self) -> int:
        return torch.cuda.current_stream(self.device).cuda_stream

    # ---- StepContext::PrepareInputs -------------------------------------------------------
    def prepare_inputs(self, computed: torch.Tensor, n_new: torch.Tensor, bt_off: torch.Tensor,
                       bt_pages: torch.Tensor, n_reqs: int | None = None,
                       rows_bound: int | None = None, n_reqs_dev: torch.Tensor | None = None):
        """GPU pack of a ragged batch given as device int32 arrays."""
        R = int(computed.shape[0]) if n_reqs is None else n_reqs
        if R > self.max_reqs:
            raise ValueError("too many requests for this AttnStep")
        batch = FqaBatch(_ptr(computed), _ptr(n_new), _ptr(bt_off), _ptr(bt_pages),
                         _ptr(n_reqs_dev), R)
        check(self.lib.fqa_pack(C.byref(batch), C.byref(self.cfg), C.byref(self.out_struct),
                                self.stream), "fqa_pack")
        self.n_reqs_bound = R
        self.rows_bound = self.max_rows if rows_bound is None else rows_bound

    def schedule_and_prepare(self, num_tokens: torch.Tensor, computed: torch.Tensor,
                             bt_off: torch.Tensor, bt_pages: torch.Tensor, token_budget: int,
                             prefill_chunk: int, rows_bound: int | None = None,
                             fused: bool = True):
        """Scheduler::BuildBatch selection + gather + pack, all on the GPU: two launches
        (fqa_schedule_gather, fqa_pack), or with fused=False three (fqa_schedule,
        fqa_gather_batch, fqa_pack)."""
        n_run = int(num_tokens.shape[0])
        if fused:
            check(self.lib.fqa_schedule_gather(
                _ptr(num_tokens), _ptr(computed), n_run, token_budget, prefill_chunk,
                _ptr(bt_off), _ptr(bt_pages), _ptr(self.sel_req), _ptr(self.sel_n),
                _ptr(self.n_sel), _ptr(self.b_computed), _ptr(self.b_n_new), _ptr(self.b_bt_off),
                _ptr(self.b_bt_pages), self.max_bt_pages, self.stream), "fqa_schedule_gather")
        else:
            check(self.lib.fqa_schedule(_ptr(num_tokens), _ptr(computed), n_run, token_budget,
                                        prefill_chunk, _ptr(self.sel_req), _ptr(self.sel_n),
                                        _ptr(self.n_sel), self.stream), "fqa_schedule")
            check(self.lib.fqa_gather_batch(_ptr(self.sel_req), _ptr(self.sel_n),
                                            _ptr(self.n_sel), n_run, _ptr(computed),
                                            _ptr(bt_off), _ptr(bt_pages), _ptr(self.b_computed),
                                            _ptr(self.b_n_new), _ptr(self.b_bt_off),
                                            _ptr(self.b_bt_pages), self.max_bt_pages,
                                            self.stream), "fqa_gather_batch")
        self.prepare_inputs(self.b_computed, self.b_n_new, self.b_bt_off, self.b_bt_pages,
                            n_reqs=n_run, rows_bound=rows_bound, n_reqs_dev=self.n_sel)

    # ---- per layer ------------------------------------------------------------------------
    def head_norm_rope_store_kv(self, qkv, pool_layer, q_norm_w, k_norm_w, write_k=False):
        """LaunchHeadNormRope + KvStore::StoreKV, fused."""
        check(self.lib.fqa_qknorm_rope_append(
            C.byref(self.dims), _ptr(qkv), _ptr(q_norm_w), _ptr(k_norm_w), _ptr(self.cos),
            _ptr(self.sin), self.max_ctx, _ptr(self.positions), _ptr(self.slot_mapping),
            _ptr(self.meta), self.rows_bound, _ptr(pool_layer), self.pool_pages, int(write_k),
            self.stream), "fqa_qknorm_rope_append")

    def attn_decode(self, qkv, pool_layer, out):
        """LaunchAttnDecodeCute: split-K decode + combine (with dec_prefix_pages, the
        groups' shared prefixes first)."""
        if self.dec_prefix_pages > 0:
            check(self.lib.fqa_decode_prefix(
                C.byref(self.dims), _ptr(qkv), _ptr(pool_layer), self.pool_pages,
                _ptr(self.block_tables), self.max_blocks, _ptr(self.dec_waves),
                _ptr(self.dec_seqs), _ptr(self.dec_prefix), _ptr(self.dec_pre_items),
                _ptr(self.meta), self.dec_wave_cap, self.dec_pre_cap, self.n_reqs_bound,
                _ptr(self.workspace), _ptr(out), self.stream), "fqa_decode_prefix")
            return
        check(self.lib.fqa_decode(
            C.byref(self.dims), _ptr(qkv), _ptr(pool_layer), self.pool_pages,
            _ptr(self.block_tables), self.max_blocks, _ptr(self.dec_waves),
            _ptr(self.dec_seqs), _ptr(self.meta), self.dec_wave_cap, self.n_reqs_bound,
            _ptr(self.workspace), _ptr(out), self.stream), "fqa_decode")

    def decode_read_floor(self, pool_layer):
        """Read the decode plan's pages with fqa_decode's loads and no arithmetic (the HBM
        floor of this plan); the sink is the decode workspace."""
        check(self.lib.fqa_decode_read_floor_prefix(
            _ptr(pool_layer), self.pool_pages, _ptr(self.block_tables), self.max_blocks,
            _ptr(self.dec_waves), _ptr(self.dec_seqs),
            _ptr(self.dec_prefix) if self.dec_prefix_pages > 0 else None, _ptr(self.meta),
            self.dec_wave_cap, _ptr(self.workspace), self.stream), "fqa_decode_read_floor")

    def attn_prefill(self, qkv, pool_layer, out):
        """LaunchAttnPrefillCute: varlen causal FA-2."""
        check(self.lib.fqa_prefill(
            C.byref(self.dims), _ptr(qkv), _ptr(pool_layer), self.pool_pages,
            _ptr(self.block_tables), self.max_blocks, _ptr(self.cu_seqlens),
            _ptr(self.positions), _ptr(self.pre_items), _ptr(self.meta), self.pre_tile_q,
            self.pre_cap, _ptr(out), self.stream), "fqa_prefill")

    def run_layer(self, qkv, pool_layer, q_norm_w, k_norm_w, out, write_k=False,
                  decode=True, prefill=True, side_stream=None):
        """The attention block of one layer (model_runtime.cu:263-278).  With side_stream
        (and both kinds of rows), the decode runs on it concurrently with the prefill,
        queued first so that its workgroups take their CUs before the prefill's fill the
        rest (with dec_share the decode plan leaves the prefill its share): the two write
        disjoint output rows and only read the pool, and the decode is HBM-bound while the
        prefill is MFMA-bound."""
        self.head_norm_rope_store_kv(qkv, pool_layer, q_norm_w, k_norm_w, write_k)
        if decode and prefill and side_stream is not None:
            cur = torch.cuda.current_stream(self.device)
            side_stream.wait_stream(cur)
            with torch.cuda.stream(side_stream):  # self.stream follows the current stream
                self.attn_decode(qkv, pool_layer, out)
            self.attn_prefill(qkv, pool_layer, out)
            cur.wait_stream(side_stream)
            return
        if decode:
            self.attn_decode(qkv, pool_layer, out)
        if prefill:
            self.attn_prefill(qkv, pool_layer, out)

    def meta_host(self) -> np.ndarray:
        return self.meta.cpu().numpy()
