"""Shared helpers of the test suite: build one step's inputs, run the CPU oracle chain and
the HIP chain on them, and compare.  Tolerances are those of the attention path's
contract: pack/plan arrays bit-exact; norm/RoPE outputs within 1 bf16 ulp (fp32
summation order differs); attention outputs max-abs <= 2e-2 and mean-abs <= 2e-3, and decode rows (P kept at fp32
precision, as in the reference) within 1 bf16 ulp or 2^-16 of the oracle."""
from __future__ import annotations

import numpy as np

from flashqwen_amd import synth
from flashqwen_amd.synth import HEAD_DIM, N_KV, N_Q, PAGE, QKV_STRIDE

ATT_MAX_ABS = 2e-2
ATT_MEAN_ABS = 2e-3


def pack_kwargs(cfg: synth.StepConfig, max_rows=None, dec_grid_waves=1024, dec_min_pages=8,
                pre_tile_q=64, max_reqs=None, dec_share=0, dec_prefix_pages=0, dec_pre_cap=0):
    from oracle import oracle as orc  # noqa: F401  (tests only)

    R = cfg.n_reqs if max_reqs is None else max_reqs
    max_rows = max(cfg.rows, 1) if max_rows is None else max_rows
    pre_cap = max_rows // pre_tile_q + R
    return dict(max_rows=max_rows, max_blocks=cfg.max_blocks, pool_pages=cfg.pool_pages,
                dec_grid_waves=dec_grid_waves, dec_min_pages=dec_min_pages,
                dec_wave_cap=dec_grid_waves, pre_tile_q=pre_tile_q, pre_item_cap=pre_cap,
                dec_share=int(dec_share), dec_prefix_pages=int(dec_prefix_pages),
                dec_pre_cap=int(dec_pre_cap) if dec_prefix_pages else 0)


def pool_elems(pages: int) -> int:
    return pages * N_KV * 2 * PAGE * HEAD_DIM


def ulp_diff_bf16(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """Distance in bf16 ulps between two bf16 bit-pattern arrays (ordered-int trick)."""
    def key(x):
        x = x.astype(np.int32)
        return np.where(x & 0x8000, 0x8000 - (x & 0x7FFF), 0x8000 + x)
    return np.abs(key(a) - key(b))


def assert_rope_close(got: np.ndarray, ref: np.ndarray, what: str = "") -> None:
    """bf16 outputs of fp32 norm/RoPE math: within one bf16 ulp (2^-7 relative) plus an
    absolute 1e-5 for results that cancel (y1*cos - y2*sin ~ 0), where fp32 rounding of
    O(1) operands is many ulps of a tiny result."""
    g = synth.bf16_to_f32(got).astype(np.float64)
    r = synth.bf16_to_f32(ref).astype(np.float64)
    bad = np.abs(g - r) > 2.0 ** -7 * np.abs(r) + 1e-5
    assert not bad.any(), f"{what}: {int(bad.sum())} of {bad.size} outside 1 ulp + 1e-5"


def assert_decode_rows_close(got_bits: np.ndarray, ref_bits: np.ndarray, label: str) -> None:
    """Decode rows: the kernel differs from the oracle only in fp32 summation order (and
    P's hi+lo split, ~16 significand bits), so each output is within one bf16 step of the
    oracle's, or within 2^-16 where the output is a near-cancelling sum (a few keys)
    whose size is set by the fp32 rounding of its terms (3.3e-6 seen at 2048 short
    sequences).  P rounded to bf16 instead would leave errors of 1e-4..1e-3."""
    g = synth.bf16_to_f32(got_bits).astype(np.float64)
    r = synth.bf16_to_f32(ref_bits).astype(np.float64)
    # bf16 values as integers that are monotone in the value (sign-magnitude -> two's
    # complement order), so a difference of 1 is one representable step
    def ordered(b):
        b = b.astype(np.int32)
        return np.where(b & 0x8000, -(b & 0x7FFF), b)
    steps = np.abs(ordered(got_bits) - ordered(ref_bits))
    bad = (steps > 1) & (np.abs(g - r) > 2.0 ** -16)
    assert not bad.any(), (label, int(bad.sum()), float(np.abs(g - r)[bad].max()),
                           int(steps.max()))


def assert_prefill_rows_close(got_bits: np.ndarray, ref_bits: np.ndarray, absv: np.ndarray,
                              label: str) -> tuple[float, int]:
    """Prefill rows, element by element.  The kernel and the oracle both round P to bf16
    in the numerator (the reference does, attn_cute.cu:128); they differ in the max each
    weight is taken against (the kernel's is lazy), and the kernel also sums the rounded
    weights into l.  bf16 rounds a weight by at most 2^-8 relative, so
    |kernel - exact| <= 2^-8 (A + |O|) and |oracle - exact| <= 2^-8 A (checked against
    fp64 in tests/test_oracle.py), with A = sum_k p_k |V_kd| / sum_k p_k (`absv`, from the
    oracle), plus each final rounding.  Allowed: 2^-7 A + 2^-8 |O| + 2 bf16 steps of the
    oracle's output.  Returns the worst |difference| / allowance and the worst difference
    in bf16 steps among outputs of magnitude >= 2^-6."""
    g = synth.bf16_to_f32(got_bits).astype(np.float64)
    r = synth.bf16_to_f32(ref_bits).astype(np.float64)
    a = np.abs(r)
    ulp = np.where(a > 0, np.exp2(np.floor(np.log2(np.maximum(a, 1e-30))) - 7), 0.0)
    allow = 2.0 ** -7 * absv.astype(np.float64) + 2.0 ** -8 * a + 2 * ulp + 1e-6
    diff = np.abs(g - r)
    ratio = diff / allow
    def ordered(b):
        b = b.astype(np.int32)
        return np.where(b & 0x8000, -(b & 0x7FFF), b)
    # bf16 steps where the output is not near 0 (across 0 the step count means nothing)
    big = a >= 2.0 ** -6
    steps = np.abs(ordered(got_bits) - ordered(ref_bits))[big]
    worst = float(ratio.max(initial=0.0))
    bad = ratio > 1.0
    assert not bad.any(), (label, int(bad.sum()), worst, float(diff[bad].max()))
    return worst, int(steps.max(initial=0))


def att_errors(got_bits: np.ndarray, ref_bits: np.ndarray) -> tuple[float, float]:
    g = synth.bf16_to_f32(got_bits).astype(np.float64)
    r = synth.bf16_to_f32(ref_bits).astype(np.float64)
    d = np.abs(g - r)
    return float(d.max(initial=0.0)), float(d.mean()) if d.size else 0.0


def oracle_chain(cfg: synth.StepConfig, qkv: np.ndarray, pool: np.ndarray, wq, wk, kw: dict,
                 computed=None, n_new=None, bt_off=None, bt_pages=None):
    """The reference step restated on the CPU: pack -> norm/rope/append -> decode, prefill.
    qkv and pool are copied; returns dict with pack, qkv, pool, out."""
    from oracle import oracle as orc

    computed = cfg.computed if computed is None else computed
    n_new = cfg.n_new if n_new is None else n_new
    bt_off = cfg.bt_off if bt_off is None else bt_off
    bt_pages = cfg.bt_pages if bt_pages is None else bt_pages
    pk = orc.pack(computed, n_new, bt_off, bt_pages, **kw)
    T = int(pk["meta"][0])
    cos, sin = orc.rope_tables(cfg.max_ctx)
    q = qkv.copy()
    p = pool.copy()
    orc.qknorm_rope_append(q, wq, wk, cos, sin, pk["positions"], pk["slot_mapping"], T, p,
                           cfg.pool_pages)
    out = np.zeros((max(T, 1), N_Q * HEAD_DIM), np.uint16)
    R = len(computed)
    bt = pk["block_tables"]
    orc.decode(q, p, cfg.pool_pages, bt, kw["max_blocks"], pk["cu_seqlens"], pk["positions"],
               pk["decode_rids"], int(pk["meta"][1]), out)
    orc.prefill(q, p, cfg.pool_pages, bt, kw["max_blocks"], pk["cu_seqlens"], pk["positions"],
                pk["prefill_rids"], int(pk["meta"][2]), out)
    return dict(pack=pk, qkv=q, pool=p, out=out[:T], R=R, T=T)


def written_mask(pk: dict, T: int) -> tuple[np.ndarray, np.ndarray]:
    slots = pk["slot_mapping"][:T].astype(np.int64)
    return slots // PAGE, slots % PAGE
