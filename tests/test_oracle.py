"""Pins the CPU oracle (oracle/fqa_oracle.c) before anything is checked against it.

The reference ships no tests or golden vectors for this path (its only tests are Go
text-tier tests), so each oracle function is pinned by library routines and closed forms
chosen so that a plausible mistake (dropped term, wrong sign or index, transposed
operand, off-by-one mask) fails:

  bf16 rounding        torch's float32 -> bfloat16 cast (RNE)
  RoPE tables          float64 cos/sin of the float32 angle; p = 0 gives cos 1, sin 0
  RMSNorm + RoPE       torch fp64 rms_norm + rotate-half; p = 0 identity; constant input;
                       pair-norm preservation; relative-position invariance of q.k
  append               exact placement of k and raw v at the slot; nothing else written
  attention            torch fp64 scaled_dot_product_attention (GQA, causal offset);
                       single key -> V; identical keys -> mean(V); first causal row ->
                       V[0]; page-permutation invariance (bit-exact)
  pack / plans         an independent Python restatement (tests/pyref.py) on random
                       batches, hand-built known answers, every status code
  selection            the reference's greedy loop restated in Python; config 4's known
                       batch (261 requests, 6464 rows)
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from flashqwen_amd import synth
from flashqwen_amd.synth import HEAD_DIM, N_KV, N_Q, PAGE, QKV_STRIDE
from oracle import oracle as orc
from tests import pyref
from tests import stepcase as sc

F32 = np.float32


def bf(x: np.ndarray) -> np.ndarray:
    """float -> bf16 bits via torch (RNE) — the library routine the oracle must match."""
    t = torch.from_numpy(np.ascontiguousarray(x, dtype=F32)).to(torch.bfloat16)
    return t.view(torch.int16).numpy().view(np.uint16)


def f32(b: np.ndarray) -> np.ndarray:
    return synth.bf16_to_f32(b)


# ---------------------------------------------------------------------------------------
def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(20000).astype(F32) * 10 ** rng.uniform(-40, 38, 20000).astype(F32),
                        np.array([0.0, -0.0, np.inf, -np.inf, 1e-45, 3.0e38, 1.00390625, 1.01171875], F32)])
    x = x[np.isfinite(x) | np.isinf(x)]
    lib = orc.load()
    got = np.array([lib.fqo_f32_to_bf16(float(v)) for v in x], np.uint16)
    assert np.array_equal(got, bf(x))
    # ties go to even
    assert lib.fqo_f32_to_bf16(1.00390625) == 0x3F80
    assert lib.fqo_f32_to_bf16(1.01171875) == 0x3F82


def test_rope_tables():
    cos, sin = orc.rope_tables(4096)
    assert np.all(cos[0] == 1.0) and np.all(sin[0] == 0.0)
    # fp64 truth of angle p * theta^(-2i/128): the tables compute the angle in float32,
    # so they may differ by the float32 rounding of the angle (a few ulps of p * inv)
    i = np.arange(64)
    ang = np.arange(4096, dtype=np.float64)[:, None] * np.power(1e6, -2.0 * i / 128)[None, :]
    tol = 4 * 2.0 ** -24 * np.maximum(ang, 1.0) + 2e-7
    assert np.all(np.abs(cos - np.cos(ang)) <= tol)
    assert np.all(np.abs(sin - np.sin(ang)) <= tol)
    # a dropped factor 2 or a wrong sign in the exponent would be far outside tol
    wrong = np.arange(4096.0)[:, None] * np.power(1e6, -1.0 * i / 128)[None, :]
    assert np.abs(cos - np.cos(wrong)).max() > 0.1


# ---------------------------------------------------------------------------------------
def _norm_case(rows=12, seed=0, positions=None):
    rng = np.random.default_rng(seed)
    qkv = synth.rand_bf16(rng, (rows, QKV_STRIDE))
    wq, wk = synth.norm_weights(seed + 1)
    pos = np.arange(rows, dtype=np.int32) * 37 if positions is None else np.asarray(positions, np.int32)
    pool_pages = 64
    slots = (rng.permutation(pool_pages * PAGE)[:rows]).astype(np.int32)
    pool = np.zeros(sc.pool_elems(pool_pages), np.uint16)
    return qkv, wq, wk, pos, slots, pool, pool_pages


def _torch_norm_rope(x_bits, w, pos, cos, sin):
    x = torch.from_numpy(f32(x_bits).astype(np.float64))
    wt = torch.from_numpy(w.astype(np.float64))
    y = torch.nn.functional.rms_norm(x, (HEAD_DIM,), wt, eps=1e-6)
    c = torch.from_numpy(cos[pos].astype(np.float64))
    s = torch.from_numpy(sin[pos].astype(np.float64))
    y1, y2 = y[..., :64], y[..., 64:]
    return torch.cat([y1 * c - y2 * s, y2 * c + y1 * s], -1).numpy()


def test_qknorm_rope_against_torch_fp64():
    qkv, wq, wk, pos, slots, pool, pp = _norm_case()
    cos, sin = orc.rope_tables(4096)
    q = qkv.copy()
    orc.qknorm_rope_append(q, wq, wk, cos, sin, pos, slots, len(pos), pool, pp)
    for head in range(N_Q + N_KV):
        w = wq if head < N_Q else wk
        src = qkv[:, head * HEAD_DIM:(head + 1) * HEAD_DIM]
        ref = _torch_norm_rope(src, w, pos[:, None].repeat(1, 0)[:, 0], cos, sin)
        if head < N_Q:
            got = f32(q[:, head * HEAD_DIM:(head + 1) * HEAD_DIM]).astype(np.float64)
        else:
            kvh = head - N_Q
            pg, tk = slots // PAGE, slots % PAGE
            got = np.stack([f32(pool[[orc.pool_offset(int(pg[t]), kvh, 0, int(tk[t]), d)
                                      for d in range(HEAD_DIM)]]) for t in range(len(pos))])
        # one bf16 rounding of the fp32 result + fp32 vs fp64 evaluation
        assert np.all(np.abs(got - ref) <= 2.0 ** -8 * np.abs(ref) + 2e-5), head


def test_qknorm_rope_closed_forms():
    cos, sin = orc.rope_tables(4096)
    qkv, wq, wk, pos, slots, pool, pp = _norm_case(rows=4, positions=[0, 0, 0, 0])
    # constant input: rms_norm(c * 1) = sign(c) (eps negligible), times w; pos 0 = identity
    qkv[0, :] = bf(np.full(QKV_STRIDE, 2.5, F32))
    qkv[1, :] = bf(np.full(QKV_STRIDE, -0.75, F32))
    q = qkv.copy()
    orc.qknorm_rope_append(q, wq, wk, cos, sin, pos, slots, 4, pool, pp)
    assert np.array_equal(q[0, :HEAD_DIM], bf(wq))
    assert np.array_equal(q[1, :HEAD_DIM], bf(-wq))
    # pos 0 is the identity: output = bf16(x / rms * w)
    x = f32(qkv[2, :HEAD_DIM]).astype(np.float64)
    y = x / np.sqrt(np.mean(x * x) + 1e-6) * wq
    assert np.all(np.abs(f32(q[2, :HEAD_DIM]) - y) <= 2.0 ** -8 * np.abs(y) + 1e-6)

    # rotation: pair norms preserved, and q.k depends only on the position difference
    qkv, wq, wk, _, slots, pool, pp = _norm_case(rows=4, seed=3)
    qkv[2] = qkv[0]
    qkv[3] = qkv[1]
    pos = np.array([5, 3, 1005, 1003], np.int32)
    q = qkv.copy()
    orc.qknorm_rope_append(q, wq, wk, cos, sin, pos, slots, 4, pool, pp)
    ref0 = orc.rope_tables(1)  # noqa: F841  (tables for p=0 are identity, checked above)
    q0 = qkv.copy()
    orc.qknorm_rope_append(q0, wq, wk, cos, sin, np.zeros(4, np.int32), slots, 4,
                           np.zeros_like(pool), pp)
    a, b = f32(q[:, :HEAD_DIM]).astype(np.float64), f32(q0[:, :HEAD_DIM]).astype(np.float64)
    pn = lambda v: v[:, :64] ** 2 + v[:, 64:] ** 2  # noqa: E731
    assert np.allclose(pn(a), pn(b), rtol=2e-2, atol=1e-3)
    d1 = np.dot(a[0], a[1])
    d2 = np.dot(a[2], a[3])
    assert abs(d1 - d2) <= 2e-2 * (abs(d1) + 1.0)
    assert abs(d1 - np.dot(b[0], b[1])) > 1e-3  # rotation is not a no-op


def test_append_placement_and_bounds():
    cos, sin = orc.rope_tables(64)
    qkv, wq, wk, pos, slots, pool, pp = _norm_case(rows=5, positions=[1, 2, 3, 63, 64])
    slots[2] = pp * PAGE + 3  # page out of range: nothing written for this row
    slots[1] = -16 + 11  # page id -1, token 11: negative slot, nothing written (C division
    # truncates -5 / 16 to page 0; a slot test, not a page test, must reject it)
    q = qkv.copy()
    orc.qknorm_rope_append(q, wq, wk, cos, sin, pos, slots, 5, pool, pp, write_k=True)
    # row 4 has no table row (pos 64 >= 64): untouched
    assert np.array_equal(q[4], qkv[4])
    written = set()
    for t in (0, 3):
        pg, tk = int(slots[t] // PAGE), int(slots[t] % PAGE)
        for kvh in range(N_KV):
            for d in range(HEAD_DIM):
                ko = orc.pool_offset(pg, kvh, 0, tk, d)
                vo = orc.pool_offset(pg, kvh, 1, tk, d)
                assert pool[ko] == q[t, (N_Q + kvh) * HEAD_DIM + d]  # normed k (write_k)
                assert pool[vo] == qkv[t, (N_Q + N_KV + kvh) * HEAD_DIM + d]  # raw v
                written.update((ko, vo))
    mask = np.ones(pool.size, bool)
    mask[list(written)] = False
    assert not pool[mask].any()


# ---------------------------------------------------------------------------------------
def _attn_case(seed, lens, computed, pool_pages=128, perm_seed=None):
    """Random q/pool for requests with given new rows (lens) and cached prefixes."""
    rng = np.random.default_rng(seed)
    tables = []
    perm = np.random.default_rng(perm_seed if perm_seed is not None else seed).permutation(pool_pages)
    o = 0
    for n, c in zip(lens, computed):
        k = synth.cdiv(n + c, PAGE)
        tables.append(perm[o:o + k].astype(np.int32))
        o += k
    cfg = synth._assemble("t", computed, lens, tables, pool_pages, 4096)
    T = cfg.rows
    qkv = synth.rand_bf16(rng, (T, QKV_STRIDE))
    pool = synth.rand_bf16(np.random.default_rng(seed + 1000), sc.pool_elems(pool_pages))
    kw = sc.pack_kwargs(cfg)
    pk = orc.pack(cfg.computed, cfg.n_new, cfg.bt_off, cfg.bt_pages, **kw)
    return cfg, qkv, pool, pk, kw


def _run_attn(cfg, qkv, pool, pk, kw):
    T = cfg.rows
    out = np.zeros((T, N_Q * HEAD_DIM), np.uint16)
    orc.decode(qkv, pool, cfg.pool_pages, pk["block_tables"], kw["max_blocks"], pk["cu_seqlens"],
               pk["positions"], pk["decode_rids"], int(pk["meta"][1]), out)
    orc.prefill(qkv, pool, cfg.pool_pages, pk["block_tables"], kw["max_blocks"],
                pk["cu_seqlens"], pk["positions"], pk["prefill_rids"], int(pk["meta"][2]), out)
    return out


def _logical_kv(cfg, pool, r, nkeys):
    """[nkeys, 8, 128] K and V of request r read through its block table."""
    K = np.zeros((nkeys, N_KV, HEAD_DIM))
    V = np.zeros_like(K)
    t = cfg.tables()[r]
    d = np.arange(HEAD_DIM)
    for kp in range(nkeys):
        pg, tk = int(t[kp // PAGE]), kp % PAGE
        for kvh in range(N_KV):
            base = ((pg * N_KV + kvh) * 2) * PAGE * HEAD_DIM
            K[kp, kvh] = f32(pool[base + tk * HEAD_DIM + d])
            V[kp, kvh] = f32(pool[base + PAGE * HEAD_DIM + d * PAGE + tk])
    return K, V


@pytest.mark.parametrize("lens,computed", [([1, 1, 1], [0, 40, 300]), ([37, 1, 20], [0, 90, 50])])
def test_attention_against_torch_sdpa(lens, computed):
    cfg, qkv, pool, pk, kw = _attn_case(7, lens, computed)
    out = _run_attn(cfg, qkv, pool, pk, kw)
    for r, (n, c) in enumerate(zip(lens, computed)):
        K, V = _logical_kv(cfg, pool, r, n + c)
        q0 = pk["cu_seqlens"][r]
        Q = f32(qkv[q0:q0 + n, :N_Q * HEAD_DIM]).reshape(n, N_Q, HEAD_DIM).astype(np.float64)
        Qt = torch.from_numpy(Q).transpose(0, 1)  # [H, n, D]
        Kt = torch.from_numpy(K).transpose(0, 1).repeat_interleave(4, 0)  # GQA: h -> h//4
        Vt = torch.from_numpy(V).transpose(0, 1).repeat_interleave(4, 0)
        mask = torch.arange(n + c)[None, :] <= (c + torch.arange(n))[:, None]
        ref = torch.nn.functional.scaled_dot_product_attention(Qt, Kt, Vt, attn_mask=mask)
        ref = ref.transpose(0, 1).reshape(n, -1).numpy()
        got = f32(out[q0:q0 + n]).astype(np.float64)
        assert np.abs(got - ref).max() <= 2e-2
        assert np.abs(got - ref).mean() <= 2e-3


def test_prefill_rounding_allowance_against_fp64():
    """The per-element allowance the GPU tests give prefill rows rests on two facts checked
    here against torch fp64: prefill_absv's A equals sum_k p_k |V_kd| / sum_k p_k, and the
    oracle's output (P rounded to bf16 in the numerator, as attn_cute.cu:128) is within
    2^-8 A of the exact attention (bf16 rounds a weight by at most 2^-8 relative) plus
    its final rounding (half a bf16 step, of the larger binade at a boundary)."""
    lens, computed = [37, 20, 64], [0, 50, 200]
    cfg, qkv, pool, pk, kw = _attn_case(11, lens, computed)
    out = np.zeros((cfg.rows, N_Q * HEAD_DIM), np.uint16)
    absv = orc.prefill_absv(qkv, pool, cfg.pool_pages, pk["block_tables"], kw["max_blocks"],
                            pk["cu_seqlens"], pk["positions"], pk["prefill_rids"],
                            int(pk["meta"][2]), out)
    assert np.array_equal(out, _run_attn(cfg, qkv, pool, pk, kw))  # same outputs as prefill()
    worst = 0.0
    for r, (n, c) in enumerate(zip(lens, computed)):
        K, V = _logical_kv(cfg, pool, r, n + c)
        q0 = pk["cu_seqlens"][r]
        Q = f32(qkv[q0:q0 + n, :N_Q * HEAD_DIM]).reshape(n, N_Q, HEAD_DIM).astype(np.float64)
        Kh = np.repeat(K.transpose(1, 0, 2), 4, 0)  # [H, keys, D], GQA h -> h // 4
        Vh = np.repeat(V.transpose(1, 0, 2), 4, 0)
        s = np.einsum("nhd,hkd->hnk", Q, Kh) / np.sqrt(HEAD_DIM)
        mask = np.arange(n + c)[None, :] <= (c + np.arange(n))[:, None]
        s = np.where(mask[None], s, -np.inf)
        p = np.exp(s - s.max(-1, keepdims=True))
        exact = np.einsum("hnk,hkd->nhd", p, Vh) / p.sum(-1).T[..., None]
        a_ref = np.einsum("hnk,hkd->nhd", p, np.abs(Vh)) / p.sum(-1).T[..., None]
        a_got = absv[q0:q0 + n].reshape(n, N_Q, HEAD_DIM)
        assert np.allclose(a_got, a_ref, rtol=1e-4, atol=1e-6)
        got = f32(out[q0:q0 + n]).reshape(n, N_Q, HEAD_DIM).astype(np.float64)
        ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(exact), 1e-30))) - 7)
        allow = 2.0 ** -8 * a_ref + ulp + 1e-6
        ratio = np.abs(got - exact) / allow
        assert ratio.max() <= 1.0, ratio.max()
        worst = max(worst, float(ratio.max()))
    assert worst > 0.3  # the allowance is not slack by orders of magnitude


def test_attention_closed_forms():
    # single key: decode at context 1 returns V[0] exactly; first row of a fresh prompt too
    cfg, qkv, pool, pk, kw = _attn_case(3, [1, 9], [0, 0])
    out = _run_attn(cfg, qkv, pool, pk, kw)
    for r in range(2):
        K, V = _logical_kv(cfg, pool, r, 1)
        row = pk["cu_seqlens"][r]
        want = bf(np.repeat(V[0], 4, axis=0).reshape(-1).astype(F32))
        assert np.array_equal(out[row], want)
    # identical keys: softmax is uniform, output = mean of V
    cfg, qkv, pool, pk, kw = _attn_case(4, [1], [40])
    t = cfg.tables()[0]
    k_src = pool[((int(t[0]) * N_KV) * 2) * PAGE * HEAD_DIM:][:HEAD_DIM].copy()
    for kp in range(41):
        pg, tk = int(t[kp // PAGE]), kp % PAGE
        for kvh in range(N_KV):
            base = ((pg * N_KV + kvh) * 2) * PAGE * HEAD_DIM
            pool[base + tk * HEAD_DIM: base + (tk + 1) * HEAD_DIM] = k_src
    out = _run_attn(cfg, qkv, pool, pk, kw)
    K, V = _logical_kv(cfg, pool, 0, 41)
    want = np.repeat(V.mean(0), 4, axis=0).reshape(-1)
    assert np.abs(f32(out[0]) - want).max() <= 2.0 ** -7 * np.abs(want).max() + 1e-6


def test_attention_page_permutation_invariance():
    lens, comp = [1, 23, 1], [77, 10, 5]
    a = _attn_case(9, lens, comp, perm_seed=1)
    b = _attn_case(9, lens, comp, perm_seed=2)
    # same logical K/V in both pools: copy a's pages into b's placement
    cfg_a, qkv, pool_a, pk_a, kw = a
    cfg_b, _, pool_b, pk_b, _ = b
    run = 2 * N_KV * PAGE * HEAD_DIM
    for ta, tb in zip(cfg_a.tables(), cfg_b.tables()):
        for pa, pb in zip(ta, tb):
            pool_b[int(pb) * run:(int(pb) + 1) * run] = pool_a[int(pa) * run:(int(pa) + 1) * run]
    oa = _run_attn(cfg_a, qkv, pool_a, pk_a, kw)
    ob = _run_attn(cfg_b, qkv, pool_b, pk_b, kw)
    assert np.array_equal(oa, ob)


# ---------------------------------------------------------------------------------------
def _kw(R, max_rows=4096, **over):
    kw = dict(max_rows=max_rows, max_blocks=256, pool_pages=4096, dec_grid_waves=64,
              dec_min_pages=2, dec_wave_cap=64, pre_tile_q=32, pre_item_cap=max_rows // 32 + R)
    kw.update(over)
    return kw


def _compare_pack(comp, nnew, tabs, kw):
    cfg = synth._assemble("p", comp, nnew, tabs, kw["pool_pages"], 4096)
    got = orc.pack(cfg.computed, cfg.n_new, cfg.bt_off, cfg.bt_pages, **kw)
    ref = pyref.pack(list(comp), list(nnew), [list(t) for t in tabs], **kw)
    assert list(got["meta"]) == ref["meta"]
    if ref["meta"][7] not in (0, 4):
        return got, ref
    R, T = len(comp), ref["meta"][0]
    assert list(got["cu_seqlens"][:R + 1]) == ref["cu_seqlens"]
    for k in ("positions", "row_req", "slot_mapping"):
        assert list(got[k][:T]) == ref[k], k
    for k in ("decode_rids", "prefill_rids", "qlen"):
        assert list(got[k][:R]) == list(ref[k]), k
    assert list(got["block_tables"][:R * kw["max_blocks"]]) == ref["block_tables"]
    nd, G, npi = ref["meta"][1], ref["meta"][4], ref["meta"][5]
    assert got["dec_seqs"][:nd].tolist() == ref["dec_seqs"]
    assert got["dec_waves"][:G].tolist() == ref["dec_waves"]
    assert got["pre_items"][:npi].tolist() == ref["pre_items"]
    assert got["dec_prefix"][:nd, :4].tolist() == ref["dec_prefix"]
    assert got["dec_pre_items"][:ref["meta"][10]].tolist() == ref["dec_pre_items"]
    return got, ref


@pytest.mark.parametrize("seed", range(8))
def test_pack_against_python_restatement(seed):
    from tests.test_gpu_pack import rand_batch

    rng = np.random.default_rng(seed)
    R = int(rng.choice([0, 1, 5, 40, 200]))
    comp, nnew, tabs = rand_batch(rng, R, share=True)
    kw = _kw(R, max_rows=max(1, int(np.sum(nnew)) if R else 1),
             dec_grid_waves=int(rng.choice([1, 3, 64, 2048])),
             dec_min_pages=int(rng.choice([0, 1, 8])), pre_tile_q=int(rng.choice([32, 64, 128])))
    kw["dec_wave_cap"] = kw["dec_grid_waves"]
    kw["pre_item_cap"] = kw["max_rows"] // kw["pre_tile_q"] + R
    _compare_pack(comp, nnew, tabs, kw)
    _compare_pack(comp, nnew, tabs, dict(kw, dec_share=1))
    _compare_pack(comp, nnew, tabs, dict(kw, dec_prefix_pages=1, dec_pre_cap=64 * R + 8))


@pytest.mark.parametrize("seed", range(10))
def test_pack_prefix_groups_against_python_restatement(seed):
    """Shared-prefix groups over tables that share leading runs of any length (1..all of
    their pages, from 3 run sets), with and without dec_share, at minimum prefix lengths
    1, 2 and 8 pages, and with a prefix-item capacity too small for the plan (the plan
    then has no groups)."""
    from tests.test_gpu_pack import rand_batch

    rng = np.random.default_rng(100 + seed)
    R = int(rng.choice([2, 9, 40, 150]))
    comp, nnew, tabs = rand_batch(rng, R, share="deep")
    kw = _kw(R, max_rows=max(1, int(np.sum(nnew))), dec_grid_waves=int(rng.choice([3, 64, 1024])),
             dec_min_pages=int(rng.choice([1, 8])), pre_tile_q=64)
    kw["dec_wave_cap"] = kw["dec_grid_waves"]
    kw["pre_item_cap"] = kw["max_rows"] // 64 + R
    seen = 0
    for minp in (1, 2, 8):
        got, ref = _compare_pack(comp, nnew, tabs, dict(kw, dec_prefix_pages=minp,
                                                        dec_pre_cap=64 * R + 8))
        seen += ref["meta"][11]
        _compare_pack(comp, nnew, tabs, dict(kw, dec_prefix_pages=minp, dec_pre_cap=64 * R + 8,
                                             dec_share=1))
    if ref["meta"][10] > 0:
        small = dict(kw, dec_prefix_pages=8, dec_pre_cap=ref["meta"][10] - 1)
        got, ref2 = _compare_pack(comp, nnew, tabs, small)
        assert ref2["meta"][10] == ref2["meta"][11] == 0
    assert R < 40 or seen > 0


def test_pack_prefix_known_answer():
    """Shared-prefix groups by hand.  Decodes: r0 (41 keys, pages 5 6 7), r1 (48 keys,
    5 6 9), r2 (21 keys, 8 1), r4 (71 keys, 5 6 7 2 3); r3 is a prefill starting at page 5
    too (prefills neither join nor cause groups).  The group of first page 5 is led by r0
    (decode index 0); common runs with it: r0 3 pages, capped at 40 // 16 = 2; r1 2; r4 3.
    So P = 2: pages 0 and 1 of the three are attended once (8 items, one per kv head, one
    chunk, one octet {0, 1, 3, -1 x 5}) and their streams start at page 2, with the shared flag
    cleared (their own pages are private).  At dec_prefix_pages = 3 the group is not used."""
    comp = [40, 47, 20, 0, 70]
    nnew = [1, 1, 1, 10, 1]
    tabs = [[5, 6, 7], [5, 6, 9], [8, 1], [5], [5, 6, 7, 2, 3]]
    kw = _kw(5, max_rows=16, max_blocks=8, dec_grid_waves=7, dec_min_pages=1, dec_wave_cap=7,
             pre_tile_q=32, pre_item_cap=8, pool_pages=64, dec_prefix_pages=2, dec_pre_cap=8)
    got, _ = _compare_pack(comp, nnew, tabs, kw)
    m = got["meta"]
    assert (int(m[1]), int(m[9]), int(m[10]), int(m[11])) == (4, 7, 8, 1)
    assert got["dec_prefix"][:4, :4].tolist() == [[2, 0, 1 | 1 << 16, 0], [2, 0, 1 | 1 << 16, 1],
                                                  [0, 0, 0, 0], [2, 0, 1 | 1 << 16, 2]]
    assert got["dec_pre_items"][:8].tolist() == [[0, h, 0, 2, 0, 1, 3] + [-1] * 5
                                                 for h in range(8)]
    flag = 1 << 30
    seqs = got["dec_seqs"][:4]
    assert [int(z) for z in seqs[:, 2]] == [41, 48, 21, 71]  # no flags: groups read their own
    # streams of 1, 1, 2, 3 pages cost 56, 56, 48, 72 positions (8 per page, 32 for a
    # stream's start, 16 more for a member's); 8 streams per sequence
    assert [int(z) for z in seqs[:, 3]] == [0, 448, 896, 1280]
    # W = 1856 positions in 7 shares starting at 0, 265, 530, 795, 1060, 1325, 1590; a
    # page belongs to the share holding its last position ((0, h): 56h+55; (1, h):
    # 503+56h; (2, h): 935+48h, 943+48h; (3, h): 1335+72h, +8, +16): {di, kvh, page
    # (absolute), pages streamed, page id}.  Share 3 holds pages of (1, 6..7) and
    # (2, 0..2).
    assert [list(map(int, w[:4])) + [int(w[7])] for w in got["dec_waves"][:7]] == [
        [0, 0, 2, 4, 7], [0, 4, 2, 5, 7], [1, 1, 2, 5, 9], [1, 6, 2, 8, 9],
        [2, 3, 0, 10, 8], [3, 0, 2, 12, 7], [3, 4, 2, 12, 7]]
    assert int(m[12]) == 1856 and int(m[6]) == 266
    off, _ = _compare_pack(comp, nnew, tabs, dict(kw, dec_prefix_pages=3))
    assert (int(off["meta"][9]), int(off["meta"][10]), int(off["meta"][11])) == (13, 0, 0)
    assert [bool(z & flag) for z in off["dec_seqs"][:4, 2]] == [True, True, False, True]


def test_pack_prefix_covers_every_page_once():
    """For every decode sequence and kv head, the prefix items of its group (pages
    [page0, page1) of the leader's table, which equal the member's) and the plan's shares
    of its stream together cover each of its pages exactly once, and each member is in
    exactly one octet slot of its group's items per (kv head, chunk)."""
    from tests.test_gpu_pack import rand_batch

    for seed in range(6):
        rng = np.random.default_rng(300 + seed)
        R = 60
        comp, nnew, tabs = rand_batch(rng, R, share="deep")
        kw = _kw(R, max_rows=max(1, int(np.sum(nnew))), dec_grid_waves=97, dec_min_pages=3,
                 dec_wave_cap=97, pre_tile_q=64, dec_prefix_pages=1, dec_pre_cap=64 * R)
        kw["pre_item_cap"] = kw["max_rows"] // 64 + R
        got, ref = _compare_pack(comp, nnew, tabs, kw)
        meta = got["meta"]
        nd, G, npx = int(meta[1]), int(meta[4]), int(meta[10])
        seqs, waves = got["dec_seqs"][:nd], got["dec_waves"][:G]
        drids = got["decode_rids"][:nd]
        count = {}
        for it in got["dec_pre_items"][:npx]:
            lead, kvh, p0, p1 = (int(x) for x in it[:4])
            for di in it[4:]:
                if di < 0:
                    continue
                r, rl = int(drids[di]), int(drids[lead])
                for p in range(p0, p1):
                    assert tabs[r][p] == tabs[rl][p]
                    count[(int(di), kvh, p)] = count.get((int(di), kvh, p), 0) + 1
        # walk the shares: runs (di, kvh, page) in stream order
        for w in waves:
            di, kvh, page, n = (int(x) for x in w[:4])
            while n > 0:
                r = int(drids[di])
                pages = comp[r] // 16 + 1
                P = int(got["dec_prefix"][di, 0])
                take = min(pages - page, n)
                for p in range(page, page + take):
                    count[(di, kvh, p)] = count.get((di, kvh, p), 0) + 1
                n -= take
                page = P if kvh < 7 else int(got["dec_prefix"][di + 1, 0]) if di + 1 < nd else 0
                kvh, di = (kvh + 1, di) if kvh < 7 else (0, di + 1)
        want = {(di, kvh, p) for di in range(nd) for kvh in range(8)
                for p in range(comp[int(drids[di])] // 16 + 1)}
        assert set(count) == want and all(v == 1 for v in count.values()), seed


def test_dec_share_known_answer():
    """The decode plan beside a concurrent prefill (dec_share), by hand.  With N = 1024,
    D = 783 x decode pages and P = prefill key-rows, the modelled decode time on G waves is
    D (36 G + 25 N) / (50 G), the prefill's P N / (N - G); G is the largest multiple of 32
    where the prefill is no slower, or one step more if the prefill there ends first.
    * 400 decode pages (D = 313200) beside a 400-row prompt on 583 cached keys
      (P = 400*583 + 400*401/2 = 313400): with D ~ P the times meet where
      36 G^2 + 39 N G - 25 N^2 = 0, G = 0.452 N = 463; 448 is the last multiple of 32
      below (50 P N 448 = 7.19e12 <= D (36*448 + 25 N)(N - 448) = 7.53e12), and the
      prefill at 480 (P N / 544 = 5.90e5) ends after the decode at 448
      (D * 41728 / 22400 = 5.83e5): 448 (1024 without dec_share).
    * One decode sequence of 100 keys (7 pages, D = 5481; 8 streams of 7 pages + 4 start
      positions, 88 in all) beside a 64-row prompt on 32 cached keys (P = 4128): the
      meeting point is far above the plan's 88 wavefronts: 88.
    * The same decode beside a 2000-row prompt on 10000 cached keys (P = 22001000): even
      G = 32 leaves the prefill slower, so the floor of 32 wavefronts."""
    base = dict(max_rows=65, max_blocks=256, pool_pages=4096, dec_grid_waves=1024,
                dec_min_pages=1, dec_wave_cap=1024, pre_tile_q=64, pre_item_cap=4)
    tabs3 = [np.arange(400, dtype=np.int32), np.arange(400, 462, dtype=np.int32)]
    c3 = dict(base, max_rows=401, max_blocks=512, pre_item_cap=16, dec_share=1)
    got = orc.pack([6399, 583], [1, 400], [0, 400, 462], np.concatenate(tabs3), **c3)
    assert got["meta"][4] == 448
    got = orc.pack([6399, 583], [1, 400], [0, 400, 462], np.concatenate(tabs3),
                   **dict(c3, dec_share=0))
    assert got["meta"][4] == 1024
    tabs = [np.arange(7, dtype=np.int32), np.arange(7, 13, dtype=np.int32)]
    got = orc.pack([99, 32], [1, 64], [0, 7, 13], np.concatenate(tabs), **dict(base, dec_share=1))
    assert got["meta"][4] == 88
    tabs2 = [np.arange(7, dtype=np.int32), np.arange(7, 7 + 751, dtype=np.int32)]
    big = dict(base, max_rows=2001, max_blocks=1024, pre_item_cap=40, dec_share=1)
    got = orc.pack([99, 10000], [1, 2000], [0, 7, 758], np.concatenate(tabs2), **big)
    assert got["meta"][4] == 32

def test_pack_known_answer():
    # request 0: decode at context 18 (pages 5,9); request 1: 3-row chunk on a 15-token
    # prefix (pages 2,7); request 2: 1-token fresh prompt = a decode; request 3: n = 0
    comp, nnew = [17, 15, 0, 4], [1, 3, 1, 0]
    tabs = [[5, 9], [2, 7], [11], [4]]
    kw = _kw(4, max_rows=8, max_blocks=3, dec_grid_waves=5, dec_min_pages=1, dec_wave_cap=5,
             pre_tile_q=32, pre_item_cap=4)
    got, _ = _compare_pack(comp, nnew, tabs, kw)
    assert got["cu_seqlens"][:5].tolist() == [0, 1, 4, 5, 5]
    assert got["positions"][:5].tolist() == [17, 15, 16, 17, 0]
    assert got["row_req"][:5].tolist() == [0, 1, 1, 1, 2]
    assert got["slot_mapping"][:5].tolist() == [9 * 16 + 1, 2 * 16 + 15, 7 * 16 + 0, 7 * 16 + 1,
                                                11 * 16]
    assert got["block_tables"][:12].tolist() == [5, 9, -1, 2, 7, -1, 11, -1, -1, 4, -1, -1]
    assert got["decode_rids"][:4].tolist() == [0, 2, -1, -1]
    assert got["prefill_rids"][:4].tolist() == [1, 3, -1, -1]
    assert got["meta"][:10].tolist() == [5, 2, 2, 3, 5, 1, 141, 0, 4, 3]
    # streams of 2 and 1 pages cost 48 and 40 positions (32 for a stream's start, 8 per
    # page): W = 8*(48+40) = 704 positions over 5 waves, shares from 0, 140, 281, 422, 563.
    # A page belongs to the share of its last position: (0, h) page 0 at 48h+39, page 1
    # at 48h+47, (1, h) page 0 at 423+40h; so 5, 6, 5, 4, 4 of the 24 page runs (share 3
    # starts at (1, 0)'s page, share 4 in (1, 4)'s start positions)
    assert got["dec_seqs"][:2].tolist() == [[0, 0, 18, 0], [2, 4, 1, 384]]
    assert got["dec_waves"][:5, :4].tolist() == [[0, 0, 0, 5], [0, 2, 1, 6], [0, 5, 1, 5],
                                                 [1, 0, 0, 4], [1, 4, 0, 4]]
    # {r, row, n_keys, first page id}: page 1 of request 0 is page id 9
    assert got["dec_waves"][:5, 4:].tolist() == [[0, 0, 18, 5], [0, 0, 18, 9], [0, 0, 18, 9],
                                                 [2, 4, 1, 11], [2, 4, 1, 11]]
    assert got["pre_items"][:1].tolist() == [[1, 0, 3, 18]]


def test_pack_shared_page_cost_known_answer():
    """The plan prices the pages of a shared sequence that is not the first with its first
    page at 5 positions instead of 8 (the first one's reads bring them into the caches).
    Decodes r0 (18 keys, pages 5 6) and r1 (41 keys, 5 8 9) share first page 5 (r0 first);
    r2 (2 keys, page 11) shares nothing.  Stream costs 2*8+32 = 48, 3*5+32 = 47,
    1*8+32 = 40; W = 8*135 = 1080 over 4 waves, shares from 0, 270, 540, 810.  Last
    positions of the pages: (0, h) 48h+39 and 48h+47; (1, h) 384+47h + 36, 41, 46;
    (2, h) 760+40h+39.  Share 0 takes (0, 0..4) (10 pages), share 1 (0, 5..7) and
    (1, 0..2) (15), share 2 (1, 3..7) and (2, 0) (16), share 3 (2, 1..7) (7)."""
    comp, nnew = [17, 40, 1], [1, 1, 1]
    tabs = [[5, 6], [5, 8, 9], [11]]
    kw = _kw(3, max_rows=4, max_blocks=3, dec_grid_waves=4, dec_min_pages=1, dec_wave_cap=4,
             pre_tile_q=32, pre_item_cap=4)
    got, _ = _compare_pack(comp, nnew, tabs, kw)
    flag = 1 << 30
    assert got["dec_seqs"][:3].tolist() == [[0, 0, 18 | flag, 0], [1, 1, 41 | flag, 384],
                                            [2, 2, 2, 760]]
    assert got["dec_waves"][:4, :4].tolist() == [[0, 0, 0, 10], [0, 5, 0, 15], [1, 3, 0, 16],
                                                 [2, 1, 0, 7]]
    assert got["dec_waves"][:4, 7].tolist() == [5, 5, 5, 11]
    m = got["meta"]
    assert (int(m[4]), int(m[6]), int(m[9]), int(m[12])) == (4, 270, 6, 1080)


@pytest.mark.parametrize("case,code", [("short", 1), ("wide", 2), ("rows", 3), ("page", 4),
                                       ("negative", 5), ("items", 6)])
def test_pack_status_codes(case, code):
    comp, nnew, tabs = [10, 0], [1, 40], [[1], [2, 3, 4]]
    kw = _kw(2, max_rows=64, max_blocks=8)
    if case == "short":
        tabs[1] = [2, 3]
    elif case == "wide":
        tabs[0] = list(range(9))
    elif case == "rows":
        kw["max_rows"] = 20
    elif case == "page":
        tabs[1] = [2, 5000, 4]
    elif case == "negative":
        nnew[0] = -1
    elif case == "items":
        kw["dec_wave_cap"] = 0
    got, ref = _compare_pack(comp, nnew, tabs, kw)
    assert got["status"] == code


def test_dec_waves_cover_every_run_once():
    rng = np.random.default_rng(5)
    comp = list(rng.integers(0, 3000, 37))
    tabs = [list(range(c // 16 + 1)) for c in comp]
    kw = _kw(37, max_rows=37, dec_grid_waves=61, dec_min_pages=1, dec_wave_cap=61)
    got = orc.pack(comp, [1] * 37, synth._assemble("x", comp, [1] * 37, [np.array(t) for t in tabs], 4096, 4096).bt_off,
                   np.concatenate(tabs), **kw)
    seen = []
    for di, kvh, page, n, *_ in got["dec_waves"][: got["meta"][4]]:
        while n > 0:
            pages = comp[got["dec_seqs"][di][0]] // 16 + 1
            take = min(n, pages - page)
            seen += [(di, kvh, p) for p in range(page, page + take)]
            n -= take
            page = 0
            kvh += 1
            if kvh == 8:
                kvh, di = 0, di + 1
    expect = [(di, kvh, p) for di in range(37) for kvh in range(8) for p in range(comp[di] // 16 + 1)]
    assert seen == expect


# ---------------------------------------------------------------------------------------
@pytest.mark.parametrize("seed", range(6))
def test_schedule_against_python_restatement(seed):
    rng = np.random.default_rng(seed)
    n = int(rng.integers(0, 300))
    comp = rng.integers(0, 3000, n).astype(np.int32)
    rem = np.where(rng.random(n) < 0.5, rng.integers(-2, 2, n), rng.integers(2, 900, n))
    ntok = (comp + rem).astype(np.int32)
    budget = int(rng.choice([-5, 0, 1, 512, 8192]))
    chunk = int(rng.choice([1, 64, 2048]))
    req, nn = orc.schedule(ntok, comp, budget, chunk)
    ref = pyref.build_batch(ntok.tolist(), comp.tolist(), budget, chunk)
    assert list(zip(req.tolist(), nn.tolist())) == ref


def test_schedule_config4_known_batch():
    cfg = synth.config4()
    req, nn = orc.schedule(cfg.num_tokens, cfg.computed, cfg.token_budget, cfg.prefill_chunk)
    assert len(req) == 261 and int(nn.sum()) == 6464
    rem = cfg.num_tokens[req] - cfg.computed[req]
    assert list(nn[:256]) == [1] * 256  # decodes first
    assert sorted(nn[256:259].tolist()) == [512, 700, 900]
    assert nn[259:].tolist() == [2048, 2048] and list(rem[259:]) == [4096, 4096]


# ---- sampling (fqo_sample, kernels.cu:184-327) ------------------------------------------

def _sample_numpy(lg, it, tp, u):
    """Independent formulation: numpy sort + cumsum + searchsorted, fp64; greedy rows by
    the thread-by-thread simulation of ArgmaxKernel."""
    if it <= 0:
        return pyref.argmax_kernel(lg)
    w = np.exp((lg.astype(np.float64) - lg.max()) * it)
    thr = 0.0
    if tp < 1:
        s = np.sort(w)[::-1]
        k = int(np.searchsorted(np.cumsum(s), tp * w.sum()))  # first k with cum >= need
        thr = s[min(k, len(s) - 1)]
    kept = np.where((w >= thr) & (w > 0), w, 0.0)
    cum = np.cumsum(kept)
    i = int(np.searchsorted(cum, u * cum[-1]))  # first i with cum >= target
    while i < len(kept) and kept[i] == 0.0:
        i += 1
    return min(i, len(lg) - 1)


def test_sample_known_answer():
    """logits 0..7, temperature 1: w = e^(l-7), sum 1.5814; u = 0.5 -> target 0.7907, the
    first seven weights sum to 0.5814, so token 7; u = 0 -> token 0; top_p = 0.5 keeps only
    token 7 (its weight 1 >= 0.79); greedy -> 7."""
    from oracle import oracle as orc

    lg = np.arange(8, dtype=np.float32)[None, :]
    assert orc.sample(lg, [1.0], [1.0], [0.5])[0][0] == 7
    assert orc.sample(lg, [1.0], [1.0], [0.0])[0][0] == 0
    assert orc.sample(lg, [1.0], [1.0], [0.30])[0][0] == 6   # 0.474 in (0.2141, 0.5814]
    pick, thr, mass = orc.sample(lg, [1.0], [0.5], [0.2])
    assert pick[0] == 7 and thr[0] == 1.0 and mass[0] == 1.0
    assert orc.sample(lg, [0.0], [1.0], [0.5])[0][0] == 7


def test_sample_closed_forms():
    from oracle import oracle as orc

    rng = np.random.default_rng(3)
    N = 1000
    # uniform logits, top_p = 1: the pick is ceil(u*N) - 1
    for u in (0.0005, 0.1234, 0.5, 0.99951):
        lg = np.full((1, N), 2.5, np.float32)
        assert orc.sample(lg, [0.7], [1.0], [u])[0][0] == int(np.ceil(u * N)) - 1
    # top_p -> 0 keeps only the largest weight: the argmax, whatever u
    lg = rng.standard_normal((4, N)).astype(np.float32)
    for b in range(4):
        assert orc.sample(lg[b:b + 1], [1.3], [1e-6], [rng.random()])[0][0] == int(np.argmax(lg[b]))
    # greedy ties in the reference's order: columns 17 and 400 sit on threads 17 and 144.
    # Step s moves slot t+s into slot t < s when strictly larger: 144 -> 16 (s = 128),
    # 16 -> 0 and 17 -> 1 (s = 16); at s = 1 slot 1's tie does not displace slot 0, so
    # column 400 wins although 17 is smaller
    lg = rng.standard_normal((1, N)).astype(np.float32)
    lg[0, [17, 400]] = 9.0
    assert orc.sample(lg, [0.0], [1.0], [0.3])[0][0] == 400
    # the same column on one thread: the first in its scan (256 and 512 on thread 0)
    lg = rng.standard_normal((1, N)).astype(np.float32)
    lg[0, [512, 256]] = 9.0
    assert orc.sample(lg, [0.0], [1.0], [0.3])[0][0] == 256
    # nothing above the kernel's -1e30 start: column 0
    assert orc.sample(np.full((1, N), -3e30, np.float32), [0.0], [1.0], [0.3])[0][0] == 0


def test_sample_against_numpy():
    from oracle import oracle as orc

    rng = np.random.default_rng(4)
    for trial in range(60):
        N = int(rng.integers(2, 300))
        lg = (rng.standard_normal((1, N)) * rng.choice([0.5, 3.0])).astype(np.float32)
        it = float(rng.choice([0.0, 0.5, 1.0, 2.0]))
        tp = float(rng.choice([1.0, 0.95, 0.6, 0.1]))
        u = float(rng.random())
        got = orc.sample(lg, [it], [tp], [u])[0][0]
        assert got == _sample_numpy(lg[0], it, tp, u), (trial, N, it, tp, u)


def test_greedy_tie_key_matches_the_thread_tree():
    """The GPU kernels order greedy ties by a key, (bit-reversed column % 256, column / 256);
    on random tie sets it picks what ArgmaxKernel's 256 strided scans and tree reduction
    pick (pyref.argmax_kernel), and the C oracle agrees with both."""
    def key(i):
        return (int(f"{i & 255:08b}"[::-1], 2), i >> 8)

    rng = np.random.default_rng(8)
    N = 3000
    rows = []
    for trial in range(40):
        lg = rng.standard_normal(N).astype(np.float32)
        ties = rng.choice(N, size=int(rng.integers(2, 7)), replace=False)
        lg[ties] = 7.5
        want = min(ties.tolist(), key=key)
        assert pyref.argmax_kernel(lg) == want, (trial, sorted(ties.tolist()))
        rows.append(lg)
    rows = np.stack(rows)
    got = orc.sample(rows, np.zeros(len(rows), np.float32), np.ones(len(rows), np.float32),
                     np.zeros(len(rows), np.float32))[0]
    assert [int(g) for g in got] == [pyref.argmax_kernel(r) for r in rows]


def test_pack_shared_first_page_flag():
    """FQA_DEC_SHARED (bit 30 of n_keys in dec_seqs and dec_waves): set on the decode
    sequences whose first page also starts another decode sequence.  Requests 0, 2 and 4
    are decodes whose first page is 7; request 1 decodes alone; request 3's first page is
    -1 (never shared); request 5 starts at page 7 too but is a prefill, which neither
    carries nor causes the flag."""
    comp = [20, 33, 16, 17, 40, 16]
    nnew = [1, 1, 1, 1, 1, 5]
    tabs = [[7, 3], [8, 9, 10], [7, 5], [-1, 6], [7, 3, 12], [7, 14]]
    kw = _kw(6, max_rows=16, max_blocks=4, dec_grid_waves=7, dec_min_pages=1, dec_wave_cap=7,
             pre_tile_q=32, pre_item_cap=8, pool_pages=64)
    got, _ = _compare_pack(comp, nnew, tabs, kw)
    flag = 1 << 30
    nd = int(got["meta"][1])
    seqs = got["dec_seqs"][:nd]
    assert [int(r) for r in seqs[:, 0]] == [0, 1, 2, 3, 4]
    assert [bool(z & flag) for z in seqs[:, 2]] == [True, False, True, False, True]
    assert [int(z & (flag - 1)) for z in seqs[:, 2]] == [21, 34, 17, 18, 41]
    for wv in got["dec_waves"][:int(got["meta"][4])]:
        assert (wv[6] & flag) == (seqs[wv[0], 2] & flag)
