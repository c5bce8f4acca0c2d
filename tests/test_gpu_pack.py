"""GPU pack, token-budget selection and gather vs the CPU oracle: bit-exact on random
ragged batches, edge cases (empty batch, 1-token prefills classified as decode, n=0
requests, shared prefix pages, maximal tables) and every status code."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from flashqwen_amd import synth
from tests import stepcase as sc


def rand_batch(rng, R, max_ctx=4096, pool_pages=4096, share=False):
    """share=True: tables of 4 pages or more start with the same 4 pages; share="deep":
    tables start with the same run of 1..all of their pages (one of 3 run sets)."""
    comp, nnew, tabs = [], [], []
    shared = rng.permutation(pool_pages)[:32].astype(np.int32)
    runs = [rng.permutation(pool_pages)[:synth.cdiv(max_ctx, synth.PAGE)].astype(np.int32)
            for _ in range(3)]
    for _ in range(R):
        kind = rng.integers(0, 4)
        if kind == 0:  # decode
            c, n = int(rng.integers(0, max_ctx - 1)), 1
        elif kind == 1:  # fresh prompt
            c, n = 0, int(rng.integers(0, 700))
        elif kind == 2:  # chunk continuation (prefill with cached prefix)
            c = int(rng.integers(1, 2000))
            n = int(rng.integers(2, min(600, max_ctx - c)))
        else:  # re-entering after preemption: computed 0, long
            c, n = 0, int(rng.integers(1, 300))
        need = synth.cdiv(c + n, synth.PAGE)
        extra = int(rng.integers(0, 3))
        nb = min(need + extra, synth.cdiv(max_ctx, synth.PAGE))
        t = rng.integers(0, pool_pages, size=nb).astype(np.int32)
        if share == "deep":
            k = int(rng.integers(1, nb + 1))
            t[:k] = runs[int(rng.integers(0, 3))][:k]
        elif share and nb >= 4:
            t[:4] = shared[:4]
        comp.append(c)
        nnew.append(n)
        tabs.append(t)
    return comp, nnew, tabs


def run_both(gpu, comp, nnew, tabs, *, max_rows=None, max_ctx=4096, pool_pages=4096,
             dec_grid_waves=64, dec_min_pages=2, pre_tile_q=64, max_reqs=None, dec_share=0,
             dec_prefix_pages=0, dec_pre_cap=4096):
    import torch

    from flashqwen_amd.step import AttnStep
    from oracle import oracle as orc

    cfg = synth._assemble("rand", comp, nnew, tabs, pool_pages, max_ctx)
    R = cfg.n_reqs
    max_reqs = max(R, 1) if max_reqs is None else max_reqs
    max_rows = max(int(np.sum(nnew)) if R else 0, 1) if max_rows is None else max_rows
    step = AttnStep(max_rows=max_rows, max_reqs=max_reqs, max_ctx=max_ctx, pool_pages=pool_pages,
                    device=gpu, dec_grid_waves=dec_grid_waves, dec_min_pages=dec_min_pages,
                    pre_tile_q=pre_tile_q, dec_share=bool(dec_share),
                    dec_prefix_pages=dec_prefix_pages, dec_pre_cap=dec_pre_cap)
    kw = dict(max_rows=max_rows, max_blocks=cfg.max_blocks, pool_pages=pool_pages,
              dec_grid_waves=dec_grid_waves, dec_min_pages=dec_min_pages,
              dec_wave_cap=step.dec_wave_cap, pre_tile_q=pre_tile_q, pre_item_cap=step.pre_cap,
              dec_share=dec_share, dec_prefix_pages=dec_prefix_pages,
              dec_pre_cap=step.dec_pre_cap)
    ref = orc.pack(cfg.computed, cfg.n_new, cfg.bt_off, cfg.bt_pages, **kw)
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(gpu)  # noqa: E731
    pages = cfg.bt_pages if len(cfg.bt_pages) else np.zeros(1, np.int32)
    step.prepare_inputs(t(cfg.computed if R else np.zeros(1, np.int32)),
                        t(cfg.n_new if R else np.zeros(1, np.int32)), t(cfg.bt_off), t(pages),
                        n_reqs=R)
    torch.cuda.synchronize()
    return step, ref, R, kw


def assert_pack_equal(step, ref, R, kw):
    meta = step.meta.cpu().numpy()
    assert np.array_equal(meta, ref["meta"]), (meta, ref["meta"])
    if meta[7] not in (0, 4):
        return
    T = int(meta[0])
    assert np.array_equal(step.cu_seqlens.cpu().numpy()[: R + 1], ref["cu_seqlens"][: R + 1])
    nd_seq = int(meta[1])
    assert np.array_equal(step.dec_seqs.cpu().numpy()[:nd_seq], ref["dec_seqs"][:nd_seq])
    for k in ("qlen", "decode_rids", "prefill_rids"):
        assert np.array_equal(getattr(step, k).cpu().numpy()[:R], ref[k][:R]), k
    for k in ("positions", "row_req", "slot_mapping"):
        assert np.array_equal(getattr(step, k).cpu().numpy()[:T], ref[k][:T]), k
    mb = kw["max_blocks"]
    assert np.array_equal(step.block_tables.cpu().numpy().reshape(-1)[: R * mb],
                          ref["block_tables"][: R * mb])
    nd, npi = int(meta[4]), int(meta[5])
    assert np.array_equal(step.dec_waves.cpu().numpy()[:nd], ref["dec_waves"][:nd])
    assert np.array_equal(step.pre_items.cpu().numpy()[:npi], ref["pre_items"][:npi])
    if kw.get("dec_prefix_pages", 0) > 0:
        npx = int(meta[10])
        assert np.array_equal(step.dec_prefix.cpu().numpy()[:nd_seq, :4],
                              ref["dec_prefix"][:nd_seq, :4])
        assert np.array_equal(step.dec_pre_items.cpu().numpy()[:npx], ref["dec_pre_items"][:npx])


@pytest.mark.gpu
@pytest.mark.parametrize("seed", range(12))
def test_pack_random(gpu, seed):
    rng = np.random.default_rng(seed)
    R = int(rng.choice([1, 3, 17, 64, 250, 700]))
    comp, nnew, tabs = rand_batch(rng, R, share=seed % 2 == 0)
    tile = int(rng.choice([32, 64, 128]))
    target = int(rng.choice([1, 7, 50, 2048]))
    share = seed % 3 == 1  # the decode plan for CUs shared with the prefill
    print(f"[test_pack_random] seed={seed} R={R} tile={tile} target={target} share={share}",
          flush=True)
    step, ref, R, kw = run_both(gpu, comp, nnew, tabs, pre_tile_q=tile, dec_grid_waves=target,
                                dec_min_pages=int(rng.choice([0, 1, 8])), dec_share=int(share))
    assert ref["status"] == 0
    assert_pack_equal(step, ref, R, kw)


@pytest.mark.gpu
@pytest.mark.parametrize("seed", range(8))
def test_pack_prefix_groups(gpu, seed):
    """Shared-prefix groups (dec_prefix_pages): tables sharing leading runs of any length,
    bit-exact against the oracle, with a prefix-item capacity that holds the plan and, on
    odd seeds, one item short of it (no groups then)."""
    rng = np.random.default_rng(500 + seed)
    R = int(rng.choice([2, 20, 90, 400]))
    comp, nnew, tabs = rand_batch(rng, R, share="deep")
    minp = int(rng.choice([1, 2, 8]))
    print(f"[test_pack_prefix_groups] seed={seed} R={R} min_pages={minp}", flush=True)
    step, ref, R, kw = run_both(gpu, comp, nnew, tabs, dec_grid_waves=int(rng.choice([7, 1024])),
                                dec_prefix_pages=minp, dec_share=seed % 3 == 0)
    assert ref["status"] in (0, 4)
    assert_pack_equal(step, ref, R, kw)
    npx = int(ref["meta"][10])
    if seed % 2 and npx > 0:
        step, ref, R, kw = run_both(gpu, comp, nnew, tabs, dec_prefix_pages=minp,
                                    dec_pre_cap=npx - 1)
        assert int(ref["meta"][10]) == int(ref["meta"][11]) == 0
        assert_pack_equal(step, ref, R, kw)


@pytest.mark.gpu
def test_pack_ties_in_prefill_order(gpu):
    # equal key counts across requests and tiles: the stable order must be reproduced
    comp = [0, 64, 0, 128, 32, 0]
    nnew = [128, 64, 192, 0, 96, 1]
    tabs = [np.arange(synth.cdiv(c + n, 16) + 1, dtype=np.int32) for c, n in zip(comp, nnew)]
    for tile in (32, 64, 128):
        step, ref, R, kw = run_both(gpu, comp, nnew, tabs, pre_tile_q=tile)
        assert_pack_equal(step, ref, R, kw)


@pytest.mark.gpu
def test_pack_edge_cases(gpu):
    # empty batch
    step, ref, R, kw = run_both(gpu, [], [], [], max_reqs=4)
    assert_pack_equal(step, ref, R, kw)
    assert step.meta.cpu().numpy()[0] == 0
    # 1-token prefill (computed 0, n 1) is a decode; n=0 is a prefill with no rows
    step, ref, R, kw = run_both(gpu, [0, 5, 0], [1, 0, 3], [np.array([7]), np.array([3]),
                                                          np.array([9])])
    assert_pack_equal(step, ref, R, kw)
    assert list(step.decode_rids.cpu().numpy()[:3]) == [0, -1, -1]
    assert list(step.prefill_rids.cpu().numpy()[:3]) == [1, 2, -1]
    # maximal table (max_ctx tokens)
    L = 4096
    step, ref, R, kw = run_both(gpu, [L - 1], [1], [np.arange(L // 16, dtype=np.int32)])
    assert_pack_equal(step, ref, R, kw)


@pytest.mark.gpu
@pytest.mark.parametrize("case", ["short", "wide", "rows", "negative", "page", "items"])
def test_pack_status(gpu, case):
    comp, nnew = [10, 0], [1, 40]
    tabs = [np.array([1], np.int32), np.array([2, 3, 4], np.int32)]
    kwargs = {}
    if case == "short":
        tabs[1] = np.array([2, 3], np.int32)
    elif case == "wide":
        tabs[0] = np.arange(300, dtype=np.int32)
    elif case == "rows":
        kwargs["max_rows"] = 20
    elif case == "negative":
        comp[0] = -3
    elif case == "page":
        tabs[1] = np.array([2, 5000, 4], np.int32)
    elif case == "items":
        comp = [4000] * 2
        nnew = [1, 1]
        tabs = [np.arange(251, dtype=np.int32)] * 2
        kwargs.update(dec_grid_waves=8, dec_min_pages=1)
    step, ref, R, kw = run_both(gpu, comp, nnew, tabs, **kwargs)
    code = {"short": 1, "wide": 2, "rows": 3, "negative": 5, "page": 4, "items": 6}[case]
    if case == "items":
        # capacity is sized by the bound; force overflow through a smaller cap
        from flashqwen_amd import _lib

        step.cfg.dec_wave_cap = 1
        kw["dec_wave_cap"] = 1
        from oracle import oracle as orc

        cfg = synth._assemble("x", comp, nnew, tabs, 4096, 4096)
        ref = orc.pack(cfg.computed, cfg.n_new, cfg.bt_off, cfg.bt_pages, **kw)
        import torch

        t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(gpu)  # noqa: E731
        step.prepare_inputs(t(cfg.computed), t(cfg.n_new), t(cfg.bt_off), t(cfg.bt_pages))
        torch.cuda.synchronize()
        assert _lib.META_STATUS == 7
    assert ref["status"] == code
    assert_pack_equal(step, ref, R, kw)


@pytest.mark.gpu
@pytest.mark.parametrize("fused", [True, False])
@pytest.mark.parametrize("seed", range(6))
def test_schedule_gather_pack(gpu, seed, fused):
    """fqa_schedule_gather + fqa_pack (fused) and fqa_schedule + fqa_gather_batch + fqa_pack
    == oracle selection + oracle pack."""
    import torch

    from flashqwen_amd.step import AttnStep
    from oracle import oracle as orc

    rng = np.random.default_rng(100 + seed)
    if seed == 0:
        cfg = synth.config4()
        budget, chunk = cfg.token_budget, cfg.prefill_chunk
        ntok, comp, tabs = cfg.num_tokens, cfg.computed, cfg.tables()
        pool = cfg.pool_pages
    else:
        n = int(rng.integers(1, 400))
        comp = rng.integers(0, 3000, size=n).astype(np.int32)
        rem = np.where(rng.random(n) < 0.6, 1, rng.integers(0, 900, size=n))
        ntok = (comp + rem).astype(np.int32)
        budget = int(rng.choice([0, 1, 100, 2048, 8192]))
        chunk = int(rng.choice([1, 64, 512, 2048]))
        pool = 8192
        tabs = [rng.integers(0, pool, size=synth.cdiv(int(c) + min(int(r), chunk) + 1, 16))
                .astype(np.int32) for c, r in zip(comp, rem)]
    print(f"[test_schedule_gather_pack] seed={seed} fused={fused} running={len(comp)} budget={budget} "
          f"chunk={chunk}", flush=True)
    run = synth._assemble("run", comp, np.zeros(len(comp), np.int32), tabs, pool, 8192)
    sel_req, sel_n = orc.schedule(ntok, comp, budget, chunk)
    T = int(sel_n.sum())
    max_rows = max(T, 1)
    step = AttnStep(max_rows=max_rows, max_reqs=len(comp), max_ctx=8192, pool_pages=pool,
                    device=gpu, dec_grid_waves=128, dec_min_pages=4)
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(gpu)  # noqa: E731
    step.schedule_and_prepare(t(ntok), t(comp), t(run.bt_off), t(run.bt_pages), budget, chunk,
                              fused=fused)
    torch.cuda.synchronize()
    Rb = int(step.n_sel.cpu().item())
    assert Rb == len(sel_req)
    assert np.array_equal(step.sel_req.cpu().numpy()[:Rb], sel_req)
    assert np.array_equal(step.sel_n.cpu().numpy()[:Rb], sel_n)
    sub = synth._assemble("sel", comp[sel_req], sel_n, [tabs[i] for i in sel_req], pool, 8192)
    assert np.array_equal(step.b_bt_off.cpu().numpy()[: Rb + 1], sub.bt_off)
    assert np.array_equal(step.b_bt_pages.cpu().numpy()[: len(sub.bt_pages)], sub.bt_pages)
    kw = dict(max_rows=max_rows, max_blocks=sub.max_blocks, pool_pages=pool,
              dec_grid_waves=128, dec_min_pages=4, dec_wave_cap=step.dec_wave_cap,
              pre_tile_q=step.pre_tile_q,
              pre_item_cap=step.pre_cap)
    ref = orc.pack(sub.computed, sub.n_new, sub.bt_off, sub.bt_pages, **kw)
    ref["meta"][8] = Rb
    assert_pack_equal(step, ref, Rb, kw)
    if seed == 0:
        assert T == 6464 and Rb == 261


@pytest.mark.gpu
def test_pack_at_maximum_sizes(gpu):
    """FQA_MAX_REQS (2048) requests in one step, mixed decode and prefill, over a table
    stride of 8192 pages (max_ctx 131072), with the decode plan on the full grid: bit-exact
    against the oracle."""
    rng = np.random.default_rng(2048)
    R, max_ctx, pool = 2048, 131072, 1 << 20
    comp, nnew, tabs = [], [], []
    for i in range(R):
        if i % 8 == 0:  # a prefill chunk on a cached prefix
            c, n = int(rng.integers(0, 100000)), int(rng.integers(2, 40))
        else:  # a decode, some at the longest context
            c, n = (max_ctx - 1 if i % 97 == 1 else int(rng.integers(0, 20000))), 1
        comp.append(c)
        nnew.append(n)
        tabs.append(rng.integers(0, pool, size=synth.cdiv(c + n, synth.PAGE)).astype(np.int32))
    print(f"[test_pack_at_maximum_sizes] R={R} rows={sum(nnew)} max_ctx={max_ctx}", flush=True)
    step, ref, R, kw = run_both(gpu, comp, nnew, tabs, max_ctx=max_ctx, pool_pages=pool,
                                dec_grid_waves=2048, dec_min_pages=8, pre_tile_q=32)
    assert ref["status"] == 0
    assert_pack_equal(step, ref, R, kw)
    assert int(step.meta.cpu().numpy()[1]) == R - R // 8
