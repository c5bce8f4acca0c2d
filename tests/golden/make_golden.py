"""Writes tests/golden/step_small.npz: one small mixed step (a decode, a fresh prompt and a
chunk on a cached prefix, 18 rows over a 12-page pool) run through the CPU oracle chain
(pack -> norm/RoPE/append -> decode + prefill).  The inputs are a fixed function of the
element index (splitmix64, see `inputs`), so the test regenerates them instead of storing
them; the fixture holds the expected outputs: the pack arrays, the attention output and,
per row and kv head, the K row and V column the step appended.
Run: python -m tests.golden.make_golden"""
from __future__ import annotations

from pathlib import Path

import numpy as np

OUT = Path(__file__).resolve().parent / "step_small.npz"
POOL_PAGES, MAX_CTX = 12, 256
COMPUTED = [39, 0, 16]
N_NEW = [1, 12, 5]
TABLES = [[7, 2, 9], [4, 11], [0, 5]]


def _mix(x: np.ndarray) -> np.ndarray:
    x = (x + np.uint64(0x9E3779B97F4A7C15)).astype(np.uint64)
    x = (x ^ (x >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
    x = (x ^ (x >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return x ^ (x >> np.uint64(31))


def _bf16(tag: int, n: int, a: float) -> np.ndarray:
    """n bf16 bit patterns, uniform in [-a, a), keyed by (tag, index); RNE rounding."""
    with np.errstate(over="ignore"):
        h = _mix((np.uint64(tag) << np.uint64(40)) ^ np.arange(n, dtype=np.uint64))
    f = ((h >> np.uint64(40)).astype(np.float64) / 16777216.0 * 2.0 - 1.0) * a
    u = f.astype(np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def inputs():
    from flashqwen_amd import synth
    from tests import stepcase as sc

    cfg = synth._assemble("golden-small", COMPUTED, N_NEW, [np.array(t) for t in TABLES],
                          POOL_PAGES, MAX_CTX)
    qkv = _bf16(1, cfg.rows * synth.QKV_STRIDE, 2.0).reshape(cfg.rows, synth.QKV_STRIDE)
    pool = _bf16(2, sc.pool_elems(POOL_PAGES), 1.5)
    wq = synth.bf16_to_f32(_bf16(3, synth.HEAD_DIM, 1.0)) + 1.0
    wk = synth.bf16_to_f32(_bf16(4, synth.HEAD_DIM, 1.0)) + 1.0
    kw = sc.pack_kwargs(cfg, dec_grid_waves=16, dec_min_pages=1)
    return cfg, qkv, pool, wq.astype(np.float32), wk.astype(np.float32), kw


def appended(pool: np.ndarray, slots: np.ndarray) -> np.ndarray:
    """[rows][kv heads][256]: the K row (128) then the V column (128) of each row's slot."""
    from flashqwen_amd import synth

    runs = pool.reshape(POOL_PAGES, synth.N_KV, 2 * synth.PAGE * synth.HEAD_DIM)
    out = np.empty((len(slots), synth.N_KV, 2 * synth.HEAD_DIM), np.uint16)
    for i, s in enumerate(slots):
        page, tok = int(s) // synth.PAGE, int(s) % synth.PAGE
        k = runs[page, :, tok * synth.HEAD_DIM:(tok + 1) * synth.HEAD_DIM]
        v = runs[page, :, synth.PAGE * synth.HEAD_DIM + tok::synth.PAGE]
        out[i] = np.concatenate([k, v], axis=1)
    return out


def expected():
    from tests import stepcase as sc

    cfg, qkv, pool, wq, wk, kw = inputs()
    ref = sc.oracle_chain(cfg, qkv, pool, wq, wk, kw)
    pk = ref["pack"]
    T = ref["T"]
    return dict(meta=pk["meta"], positions=pk["positions"][:T],
                slot_mapping=pk["slot_mapping"][:T], cu_seqlens=pk["cu_seqlens"],
                block_tables=pk["block_tables"], out=ref["out"],
                kv=appended(ref["pool"], pk["slot_mapping"][:T]))


if __name__ == "__main__":
    e = expected()
    np.savez_compressed(OUT, **e)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes): rows {len(e['out'])}")
