"""Seeded synthetic scheduler state for the five benchmark configurations.

Each config is the state the reference's token-budget scheduler (engine/src/scheduler.cc:
116-143) hands to one forward step: requests with a cached prefix (`computed`), the rows
they add this step (`n_new`), and block tables of 16-token page ids placed by a seeded
permutation of the pool.  Values (q/k/v, pooled K/V, norm weights) are drawn by the
callers from N(0, 1) and rounded to bf16.

Config 4 is given as *running* state (num_tokens, computed) so the token-budget selection
itself runs on the GPU (fqa_schedule); every other config is a ready batch.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

PAGE = 16
N_Q, N_KV, HEAD_DIM = 32, 8, 128
QKV_STRIDE = (N_Q + 2 * N_KV) * HEAD_DIM
ROPE_THETA = 1.0e6
RMS_EPS = 1e-6
KV_BYTES_PER_TOKEN = 2 * N_KV * HEAD_DIM * 2  # 4096 B per token per layer
PAGE_BYTES = PAGE * KV_BYTES_PER_TOKEN  # 64 KiB per page per layer


def cdiv(a: int, b: int) -> int:
    return -(-a // b)


@dataclass
class StepConfig:
    name: str
    computed: np.ndarray  # int32 [R]
    n_new: np.ndarray  # int32 [R]
    bt_off: np.ndarray  # int32 [R+1]
    bt_pages: np.ndarray  # int32 [sum pages]
    pool_pages: int
    max_ctx: int
    layers: int = 1
    # running state for configs whose batch is selected on the GPU
    num_tokens: np.ndarray | None = None
    token_budget: int = 0
    prefill_chunk: int = 0
    notes: dict = field(default_factory=dict)

    @property
    def n_reqs(self) -> int:
        return int(self.computed.shape[0])

    @property
    def max_blocks(self) -> int:
        return cdiv(self.max_ctx, PAGE)

    @property
    def rows(self) -> int:
        return int(self.n_new.sum())

    def tables(self) -> list[np.ndarray]:
        return [self.bt_pages[self.bt_off[r]: self.bt_off[r + 1]] for r in range(self.n_reqs)]


def _assemble(name, computed, n_new, tables, pool_pages, max_ctx, **kw) -> StepConfig:
    off = np.zeros(len(tables) + 1, np.int32)
    off[1:] = np.cumsum([len(t) for t in tables])
    pages = np.concatenate(tables).astype(np.int32) if tables else np.zeros(0, np.int32)
    return StepConfig(name, np.asarray(computed, np.int32), np.asarray(n_new, np.int32), off,
                      pages, pool_pages, max_ctx, **kw)


def _place(rng: np.random.Generator, pool_pages: int, counts: list[int]) -> list[np.ndarray]:
    perm = rng.permutation(pool_pages).astype(np.int32)
    assert sum(counts) <= pool_pages, "pool too small"
    out, o = [], 0
    for c in counts:
        out.append(perm[o: o + c])
        o += c
    return out


def config1(seed: int = 1) -> StepConfig:
    """Decode-only batch of 4 at contexts {17, 100, 255, 512} in a 256-page pool."""
    rng = np.random.default_rng(seed)
    L = [17, 100, 255, 512]
    tables = _place(rng, 256, [cdiv(x, PAGE) for x in L])
    return _assemble("config1", [x - 1 for x in L], [1] * 4, tables, 256, 4096)


def config2(seed: int = 2) -> StepConfig:
    """Pure decode: 64 sequences, contexts U[512, 4096], pool sized for 200k tokens."""
    rng = np.random.default_rng(seed)
    L = rng.integers(512, 4096, size=64, endpoint=True)
    pool = 200_000 // PAGE
    tables = _place(rng, pool, [cdiv(int(x), PAGE) for x in L])
    return _assemble("config2", L - 1, np.ones(64, np.int32), tables, pool, 4096)


def config3(seed: int = 3) -> StepConfig:
    """Pure ragged prefill: 16 prompts, log-normal lengths (median 400, sigma 1.0) clipped to
    [32, 4096], admitted in order while the total fits an 8192-token budget; the first prompt
    that does not fit is truncated to the remaining budget and admission stops."""
    rng = np.random.default_rng(seed)
    raw = np.clip(np.round(rng.lognormal(np.log(400.0), 1.0, size=16)), 32, 4096).astype(int)
    lens, budget = [], 8192
    for x in raw:
        if budget <= 0:
            break
        n = min(int(x), budget)
        lens.append(n)
        budget -= n
    pool = 200_000 // PAGE
    tables = _place(rng, pool, [cdiv(x, PAGE) for x in lens])
    return _assemble("config3", [0] * len(lens), lens, tables, pool, 4096,
                     notes={"prompt_lens": lens})


def config4(seed: int = 4, decode_sigma: float = 1.0) -> StepConfig:
    """Mixed 8192-token budget step from running state: 2 chunked-prefill continuations
    (3000 cached, 4096 still to go, chunk 2048), 3 fresh prompts of 512/700/900 tokens and
    256 decodes with contexts log-normal (median 1500, sigma `decode_sigma`) clipped to
    [64, 8192].  computed/bt_* are the running state; n_new is zero because the batch (n per
    request, batch order) is chosen on the GPU by fqa_schedule."""
    rng = np.random.default_rng(seed)
    dec_L = np.clip(np.round(rng.lognormal(np.log(1500.0), decode_sigma, size=256)), 64,
                    8192).astype(int)
    run_tokens = [3000 + 4096, 3000 + 4096, 512, 700, 900] + [int(x) for x in dec_L]
    run_comp = [3000, 3000, 0, 0, 0] + [int(x) - 1 for x in dec_L]
    order = rng.permutation(len(run_tokens))
    num_tokens = np.array([run_tokens[i] for i in order], np.int32)
    computed = np.array([run_comp[i] for i in order], np.int32)
    chunk, budget = 2048, 8192
    # tables grown to cover everything this step can schedule (allocator Grow, host side)
    cover = [min(int(t), int(c) + chunk) if t - c > 1 else int(t)
             for t, c in zip(num_tokens, computed)]
    need = [cdiv(x, PAGE) for x in cover]
    pool = int(sum(need) * 1.25) + 64
    tables = _place(rng, pool, need)
    cfg = _assemble("config4", computed, np.zeros(len(computed), np.int32), tables, pool, 8192,
                    num_tokens=num_tokens, token_budget=budget, prefill_chunk=chunk,
                    notes={"decode_sigma": decode_sigma})
    return cfg


def config5(seed: int = 5, layers: int = 36, pool_pages: int | None = None) -> StepConfig:
    """One decode step over all 36 layers: 32 sequences at 32768 tokens, plus 96 sequences in
    4 groups of 24 that share a 2048-token (128-page) prefix through their block tables and
    then diverge by U[64, 512] tokens.  Pool ~200 GB over 36 layers (84.8k pages/layer)."""
    rng = np.random.default_rng(seed)
    long_L = [32768] * 32
    div = rng.integers(64, 512, size=96, endpoint=True)
    if pool_pages is None:
        pool_pages = int(200e9 // (layers * PAGE_BYTES))
    perm = rng.permutation(pool_pages).astype(np.int32)
    o = 0

    def take(n):
        nonlocal o
        t = perm[o: o + n]
        o += n
        assert o <= pool_pages, "pool too small"
        return t

    tables, ctx = [], []
    for L in long_L:
        tables.append(take(cdiv(L, PAGE)))
        ctx.append(L)
    prefixes = [take(2048 // PAGE) for _ in range(4)]
    for i, d in enumerate(div):
        L = 2048 + int(d)
        own = take(cdiv(L, PAGE) - 2048 // PAGE)
        tables.append(np.concatenate([prefixes[i // 24], own]))
        ctx.append(L)
    ctx = np.array(ctx)
    return _assemble("config5", ctx - 1, np.ones(len(ctx), np.int32), tables, pool_pages, 32768,
                     layers=layers, notes={"unique_pages": o})


CONFIGS = {1: config1, 2: config2, 3: config3, 4: config4, 5: config5}


def rand_bf16(rng: np.random.Generator, shape) -> np.ndarray:
    """N(0,1) samples rounded to bf16 (RNE); returned as uint16 bit patterns."""
    x = rng.standard_normal(shape, dtype=np.float32)
    u = x.view(np.uint32)
    # finite float32 bit patterns stay below 2^32 - 2^16, so the sum cannot wrap
    u = (u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)
    return u.astype(np.uint16)


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    return (b.astype(np.uint32) << 16).view(np.float32)


def norm_weights(seed: int = 7) -> tuple[np.ndarray, np.ndarray]:
    """q_norm / k_norm weights ~ N(0,1) bf16, widened to float as the reference uploads them
    (UploadTensors<float>, model_runtime.cu:33-37)."""
    rng = np.random.default_rng(seed)
    return bf16_to_f32(rand_bf16(rng, HEAD_DIM)), bf16_to_f32(rand_bf16(rng, HEAD_DIM))


def decode_bytes(cfg: StepConfig) -> tuple[int, int]:
    """Algorithmic HBM bytes of the decode kernel for one layer: every decode sequence's K/V
    (L tokens x 4096 B, shared prefix pages counted per reader) + 16 KiB of Q read and O
    written per sequence.  Returns (logical, unique-KV) bytes."""
    dec = cfg.n_new == 1
    L = cfg.computed[dec].astype(np.int64) + 1
    logical = int(L.sum()) * KV_BYTES_PER_TOKEN + int(dec.sum()) * 2 * N_Q * HEAD_DIM * 2
    pages = set()
    for r in np.nonzero(dec)[0]:
        pages.update(cfg.bt_pages[cfg.bt_off[r]: cfg.bt_off[r + 1]].tolist())
    return logical, len(pages) * PAGE_BYTES


def prefill_flops(computed: np.ndarray, n_new: np.ndarray) -> int:
    """Causal unmasked FLOPs of the prefill: 4 * D * Hq * sum(n*c + n(n+1)/2)."""
    pre = n_new != 1
    n = n_new[pre].astype(np.int64)
    c = computed[pre].astype(np.int64)
    return int(4 * HEAD_DIM * N_Q * (n * c + n * (n + 1) // 2).sum())
