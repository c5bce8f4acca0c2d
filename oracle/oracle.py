"""ctypes wrapper of the CPU oracle (oracle/build/libfqa_oracle.so).

TEST INFRASTRUCTURE: imported only by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg.  All arrays are host numpy arrays in the formats of include/fqa.h.
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "build" / "libfqa_oracle.so"
_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def load() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        _lib = C.CDLL(str(LIB_PATH))
        _lib.fqo_f32_to_bf16.restype = C.c_uint16
        _lib.fqo_f32_to_bf16.argtypes = [C.c_float]
        _lib.fqo_bf16_to_f32.restype = C.c_float
        _lib.fqo_bf16_to_f32.argtypes = [C.c_uint16]
        _lib.fqo_pool_offset.restype = C.c_int64
        _lib.fqo_pool_offset.argtypes = [C.c_int, C.c_int, C.c_int64, C.c_int, C.c_int, C.c_int,
                                         C.c_int]
        _lib.fqo_num_threads.restype = C.c_int
    return _lib


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return C.c_void_p(a.ctypes.data)


def i32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.int32))


def num_threads() -> int:
    return int(load().fqo_num_threads())


def rope_tables(max_pos: int, head_dim: int = 128, theta: float = 1e6):
    cos = np.empty((max_pos, head_dim // 2), np.float32)
    sin = np.empty_like(cos)
    load().fqo_rope_tables(max_pos, head_dim, C.c_float(theta), _p(cos), _p(sin))
    return cos, sin


def schedule(num_tokens, computed, token_budget: int, prefill_chunk: int):
    num_tokens, computed = i32(num_tokens), i32(computed)
    n = num_tokens.shape[0]
    req = np.zeros(max(n, 1), np.int32)
    nn = np.zeros(max(n, 1), np.int32)
    R = load().fqo_schedule(n, _p(num_tokens), _p(computed), token_budget, prefill_chunk,
                            _p(req), _p(nn))
    return req[:R].copy(), nn[:R].copy()


def pack(computed, n_new, bt_off, bt_pages, *, max_rows, max_blocks, pool_pages,
         dec_grid_waves, dec_min_pages, dec_wave_cap, pre_tile_q, pre_item_cap,
         dec_share=0, dec_prefix_pages=0, dec_pre_cap=0) -> dict:
    computed, n_new, bt_off = i32(computed), i32(n_new), i32(bt_off)
    bt_pages = i32(bt_pages) if len(bt_pages) else np.zeros(1, np.int32)
    R = computed.shape[0]
    out = dict(
        cu_seqlens=np.zeros(R + 1, np.int32), qlen=np.zeros(max(R, 1), np.int32),
        positions=np.zeros(max(max_rows, 1), np.int32),
        row_req=np.zeros(max(max_rows, 1), np.int32),
        slot_mapping=np.zeros(max(max_rows, 1), np.int32),
        block_tables=np.zeros(max(R * max_blocks, 1), np.int32),
        decode_rids=np.zeros(max(R, 1), np.int32), prefill_rids=np.zeros(max(R, 1), np.int32),
        dec_seqs=np.zeros((max(R, 1), 4), np.int32),
        dec_waves=np.zeros((max(dec_wave_cap, 1), 8), np.int32),
        pre_items=np.zeros((max(pre_item_cap, 1), 4), np.int32),
        dec_prefix=np.zeros((max(R, 1), 8), np.int32),
        dec_pre_items=np.zeros((max(dec_pre_cap, 1), 12), np.int32),
        meta=np.zeros(16, np.int32))
    status = load().fqo_pack(
        R, _p(computed), _p(n_new), _p(bt_off), _p(bt_pages), max_rows, max_blocks,
        C.c_int64(pool_pages), dec_grid_waves, dec_min_pages, dec_wave_cap, pre_tile_q,
        pre_item_cap, int(dec_share), int(dec_prefix_pages), int(dec_pre_cap),
        *[_p(out[k]) for k in (
            "cu_seqlens", "qlen", "positions", "row_req", "slot_mapping", "block_tables",
            "decode_rids", "prefill_rids", "dec_seqs", "dec_waves", "pre_items", "dec_prefix",
            "dec_pre_items", "meta")])
    out["status"] = status
    return out


def qknorm_rope_append(qkv, wq, wk, cos, sin, positions, slot_mapping, rows, pool, pool_pages,
                       write_k=False, eps=1e-6, n_q=32, n_kv=8, head_dim=128):
    """In place on qkv (uint16 [rows, stride]) and pool (uint16, flat layout)."""
    stride = qkv.shape[1]
    wq = np.ascontiguousarray(wq, np.float32)
    wk = np.ascontiguousarray(wk, np.float32)
    load().fqo_qknorm_rope_append(n_q, n_kv, head_dim, stride, C.c_float(eps), _p(qkv), _p(wq),
                                  _p(wk), _p(cos), _p(sin), cos.shape[0], _p(i32(positions)),
                                  _p(i32(slot_mapping)), rows, _p(pool), C.c_int64(pool_pages),
                                  int(write_k))


def decode(qkv, pool, pool_pages, block_tables, max_blocks, cu_seqlens, positions, decode_rids,
           n_decode, out, scale=1.0 / np.sqrt(128.0), n_q=32, n_kv=8, head_dim=128):
    load().fqo_decode(n_q, n_kv, head_dim, qkv.shape[1], C.c_float(scale), _p(qkv), _p(pool),
                      C.c_int64(pool_pages), _p(i32(block_tables)), max_blocks,
                      _p(i32(cu_seqlens)), _p(i32(positions)), _p(i32(decode_rids)), n_decode,
                      _p(out))


def prefill(qkv, pool, pool_pages, block_tables, max_blocks, cu_seqlens, positions,
            prefill_rids, n_prefill, out, scale=1.0 / np.sqrt(128.0), n_q=32, n_kv=8,
            head_dim=128):
    load().fqo_prefill(n_q, n_kv, head_dim, qkv.shape[1], C.c_float(scale), _p(qkv), _p(pool),
                       C.c_int64(pool_pages), _p(i32(block_tables)), max_blocks,
                       _p(i32(cu_seqlens)), _p(i32(positions)), _p(i32(prefill_rids)),
                       n_prefill, _p(out))


def prefill_absv(qkv, pool, pool_pages, block_tables, max_blocks, cu_seqlens, positions,
                 prefill_rids, n_prefill, out, scale=1.0 / np.sqrt(128.0), n_q=32, n_kv=8,
                 head_dim=128):
    """prefill() into `out`, and per output element sum_k p_k |V_kd| / sum_k p_k (float32
    [rows, n_q * head_dim]; 0 on rows that are not prefill rows): the scale of what rounding
    P to bf16 can move an output by (each weight moves by at most 2^-9 relative)."""
    absv = np.zeros(out.shape, np.float32)
    load().fqo_prefill_absv(n_q, n_kv, head_dim, qkv.shape[1], C.c_float(scale), _p(qkv),
                            _p(pool), C.c_int64(pool_pages), _p(i32(block_tables)), max_blocks,
                            _p(i32(cu_seqlens)), _p(i32(positions)), _p(i32(prefill_rids)),
                            n_prefill, _p(out), _p(absv))
    return absv


def pool_offset(page, kvh, plane, tok, d, n_kv=8, head_dim=128) -> int:
    return int(load().fqo_pool_offset(n_kv, head_dim, page, kvh, plane, tok, d))


def sample(logits, inv_temp, top_p, u):
    """LaunchSampleBatch restated in fp64 (oracle/fqa_oracle.c, fqo_sample): returns the
    picked token per row, the smallest kept weight and the kept mass (both fp64)."""
    logits = np.ascontiguousarray(logits, np.float32)
    B, N = logits.shape
    f32 = lambda x: np.ascontiguousarray(x, np.float32)  # noqa: E731
    it, tp, uu = f32(inv_temp), f32(top_p), f32(u)
    out = np.zeros(max(B, 1), np.int32)
    thr = np.zeros(max(B, 1), np.float64)
    mass = np.zeros(max(B, 1), np.float64)
    lib = load()
    lib.fqo_sample.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_int64, C.c_void_p, C.c_void_p,
                               C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p]
    lib.fqo_sample(_p(logits), B, N, N, _p(it), _p(tp), _p(uu), _p(out), _p(thr), _p(mass))
    return out[:B].copy(), thr[:B].copy(), mass[:B].copy()
