"""GPU parity of the whole attention step (pack -> norm/rope/append -> decode + prefill)
against the CPU oracle, through the C ABI (libfqa.so via flashqwen_amd.step)."""
from __future__ import annotations

import numpy as np
import pytest

from flashqwen_amd import synth
from flashqwen_amd.synth import HEAD_DIM, N_Q, PAGE, QKV_STRIDE
from tests import stepcase as sc

PACK_KEYS_R = ("cu_seqlens", "qlen", "decode_rids", "prefill_rids")


def _t(x, dev):
    import torch

    return torch.from_numpy(np.ascontiguousarray(x)).to(dev)


def _host_u16(t) -> np.ndarray:
    import torch

    return t.view(torch.int16).cpu().numpy().view(np.uint16)


def make_pool(pages: int, seed: int, dev, layers: int = 1):
    import torch

    from flashqwen_amd.step import alloc_pool

    pool = alloc_pool(pages, layers, dev)
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    flat = pool.view(-1)
    chunk = 1 << 28
    for s in range(0, flat.numel(), chunk):
        e = min(s + chunk, flat.numel())
        flat[s:e] = torch.randn(e - s, generator=g, device=dev, dtype=torch.float32).to(
            torch.bfloat16)
    return pool


def gpu_chain(cfg, qkv_host, pool, wq, wk, dev, kw, schedule=False, side_stream=None):
    import torch

    from flashqwen_amd.step import AttnStep

    step = AttnStep(max_rows=kw["max_rows"], max_reqs=cfg.n_reqs, max_ctx=cfg.max_ctx,
                    pool_pages=cfg.pool_pages, device=dev,
                    dec_grid_waves=kw["dec_grid_waves"], dec_min_pages=kw["dec_min_pages"],
                    pre_tile_q=kw["pre_tile_q"], dec_share=bool(kw.get("dec_share", 0)),
                    dec_prefix_pages=kw.get("dec_prefix_pages", 0),
                    dec_pre_cap=kw.get("dec_pre_cap", 4096) or 4096)
    qkv = _t(qkv_host.view(np.int16), dev).view(torch.bfloat16)
    out = torch.zeros((kw["max_rows"], N_Q * HEAD_DIM), dtype=torch.bfloat16, device=dev)
    if schedule:
        step.schedule_and_prepare(_t(cfg.num_tokens, dev), _t(cfg.computed, dev),
                                  _t(cfg.bt_off, dev), _t(cfg.bt_pages, dev), cfg.token_budget,
                                  cfg.prefill_chunk)
    else:
        step.prepare_inputs(_t(cfg.computed, dev), _t(cfg.n_new, dev), _t(cfg.bt_off, dev),
                            _t(cfg.bt_pages, dev))
    step.run_layer(qkv, pool[0], _t(wq, dev), _t(wk, dev), out, side_stream=side_stream)
    torch.cuda.synchronize()
    return step, qkv, out


def check_pack(step, ref_pk, R, T, kw):
    meta = step.meta.cpu().numpy()
    assert np.array_equal(meta, ref_pk["meta"]), (meta, ref_pk["meta"])
    for k in PACK_KEYS_R:
        got = getattr(step, k).cpu().numpy()
        n = R + 1 if k == "cu_seqlens" else R
        assert np.array_equal(got[:n], ref_pk[k][:n]), k
    for k in ("positions", "row_req", "slot_mapping"):
        assert np.array_equal(getattr(step, k).cpu().numpy()[:T], ref_pk[k][:T]), k
    bt = step.block_tables.cpu().numpy().reshape(-1)[: R * kw["max_blocks"]]
    assert np.array_equal(bt, ref_pk["block_tables"][: R * kw["max_blocks"]])
    assert np.array_equal(step.dec_seqs.cpu().numpy()[: meta[1]], ref_pk["dec_seqs"][: meta[1]])
    nd, npi = int(meta[4]), int(meta[5])
    assert np.array_equal(step.dec_waves.cpu().numpy()[:nd], ref_pk["dec_waves"][:nd])
    assert np.array_equal(step.pre_items.cpu().numpy()[:npi], ref_pk["pre_items"][:npi])
    if kw.get("dec_prefix_pages", 0) > 0:
        npx = int(meta[10])
        assert np.array_equal(step.dec_prefix.cpu().numpy()[: meta[1], :4],
                              ref_pk["dec_prefix"][: meta[1], :4])
        assert np.array_equal(step.dec_pre_items.cpu().numpy()[:npx], ref_pk["dec_pre_items"][:npx])


def _check_step(cfg, sub, kw, seed, label, schedule=False, kernel_only=True):
    """Run the step on the GPU (cfg: the batch, or for schedule=True the running state it
    is selected from) and the oracle chain on `sub` (the batch itself); compare the pack
    bit-exactly, norm/RoPE within 1 ulp, V exactly on sampled rows, and the attention
    output (end to end, and optionally of the attention kernels alone) within tolerance."""
    from oracle import oracle as orc

    rng = np.random.default_rng(seed)
    T, R = sub.rows, sub.n_reqs
    qkv_h = synth.rand_bf16(rng, (T, QKV_STRIDE))
    wq, wk = synth.norm_weights()
    pool = make_pool(cfg.pool_pages, 1000 + seed, kw["device"])
    pool_h = _host_u16(pool).reshape(-1).copy()
    kwp = {k: v for k, v in kw.items() if k != "device"}

    ref = sc.oracle_chain(sub, qkv_h, pool_h, wq, wk, kwp)
    del pool_h
    step, qkv, out = gpu_chain(cfg, qkv_h, pool, wq, wk, kw["device"], kwp, schedule=schedule)

    check_pack(step, ref["pack"], R, T, kwp)

    # norm + rope: q in place, k/v into the pool (within 1 bf16 ulp; v exact)
    q_got = _host_u16(qkv)
    sc.assert_rope_close(q_got[:, : N_Q * HEAD_DIM], ref["qkv"][:, : N_Q * HEAD_DIM], "q")
    assert np.array_equal(q_got[:, N_Q * HEAD_DIM:], qkv_h[:, N_Q * HEAD_DIM:])  # k, v untouched
    pool_got = _host_u16(pool).reshape(-1)
    changed = pool_got != ref["pool"]
    if changed.any():
        sc.assert_rope_close(pool_got[changed], ref["pool"][changed], "pool")
    pages, toks = sc.written_mask(ref["pack"], T)
    for t in range(0, T, max(1, T // 64)):  # V exact on a sample of rows
        for kvh in range(8):
            base = ((pages[t] * 8 + kvh) * 2 + 1) * PAGE * HEAD_DIM
            idx = base + np.arange(HEAD_DIM) * PAGE + toks[t]
            assert np.array_equal(pool_got[idx], ref["pool"][idx])

    # attention end to end
    o_got = _host_u16(out)[:T]
    mx, mean = sc.att_errors(o_got, ref["out"])
    print(f"{label}: end-to-end max-abs {mx:.3e} mean-abs {mean:.3e}")
    assert mx <= sc.ATT_MAX_ABS and mean <= sc.ATT_MEAN_ABS
    if not kernel_only:
        return

    # attention alone: oracle attention on the GPU's post-append qkv and pool
    o_ref = np.zeros((T, N_Q * HEAD_DIM), np.uint16)
    pk = ref["pack"]
    orc.decode(q_got, pool_got.copy(), sub.pool_pages, pk["block_tables"], kwp["max_blocks"],
               pk["cu_seqlens"], pk["positions"], pk["decode_rids"], int(pk["meta"][1]), o_ref)
    absv = orc.prefill_absv(q_got, pool_got.copy(), sub.pool_pages, pk["block_tables"],
                            kwp["max_blocks"], pk["cu_seqlens"], pk["positions"],
                            pk["prefill_rids"], int(pk["meta"][2]), o_ref)
    mx, mean = sc.att_errors(o_got, o_ref)
    print(f"{label}: kernel-only max-abs {mx:.3e} mean-abs {mean:.3e}")
    assert mx <= sc.ATT_MAX_ABS and mean <= sc.ATT_MEAN_ABS
    prows = np.concatenate([np.arange(pk["cu_seqlens"][r], pk["cu_seqlens"][r + 1])
                            for r in pk["prefill_rids"][: int(pk["meta"][2])]] or
                           [np.zeros(0, np.int64)]).astype(np.int64)
    if prows.size:
        worst, steps = sc.assert_prefill_rows_close(o_got[prows], o_ref[prows], absv[prows],
                                                    label)
        print(f"{label}: prefill rows per element: worst |diff|/allowance {worst:.3f}, "
              f"worst {steps} bf16 steps where |out| >= 2^-6")
    drows = pk["cu_seqlens"][pk["decode_rids"][: int(pk["meta"][1])]]
    if drows.size:
        dmx, dmean = sc.att_errors(o_got[drows], o_ref[drows])
        print(f"{label}: decode rows kernel-only max-abs {dmx:.3e} mean-abs {dmean:.3e}")
        sc.assert_decode_rows_close(o_got[drows], o_ref[drows], label)


@pytest.mark.gpu
@pytest.mark.parametrize("cfgno,tile", [(1, 32), (2, 32), (3, 32), (3, 64)])
def test_step_parity(gpu, cfgno, tile):
    print(f"[test_step_parity] config{cfgno} tile{tile}", flush=True)
    cfg = synth.CONFIGS[cfgno]()
    kw = sc.pack_kwargs(cfg, dec_grid_waves=256 if cfgno == 1 else 2048, dec_min_pages=2,
                        pre_tile_q=tile)
    _check_step(cfg, cfg, dict(kw, device=gpu), 100 + cfgno, f"config{cfgno}")


@pytest.mark.gpu
def test_step_parity_scheduled(gpu):
    """Config 4: the GPU selects the batch from running state (fqa_schedule +
    fqa_gather_batch), packs and runs it: 2 chunked prefills on cached prefixes, 3 fresh
    prompts and 256 decodes in one step.  The oracle selects, packs and runs the same."""
    from oracle import oracle as orc

    print("[test_step_parity_scheduled] config4", flush=True)
    cfg = synth.config4()
    sel_req, sel_n = orc.schedule(cfg.num_tokens, cfg.computed, cfg.token_budget,
                                  cfg.prefill_chunk)
    tabs = cfg.tables()
    sub = synth._assemble("config4-selected", cfg.computed[sel_req], sel_n,
                          [tabs[i] for i in sel_req], cfg.pool_pages, cfg.max_ctx)
    kw = sc.pack_kwargs(sub, dec_grid_waves=2048, dec_min_pages=8)
    _check_step(cfg, sub, dict(kw, device=gpu), 104, "config4", schedule=True)


@pytest.mark.gpu
def test_decode_long_and_shared_prefix(gpu):
    """Config 5's decode batch on one layer: 32 sequences of 32768 tokens, each stream cut
    across several decode wavefronts (the combine merges more partials than one batch of
    loads holds), and 96 sequences sharing 4 prefixes of 128 pages through their block
    tables.  Pool sized to the pages the batch uses (70000 pages, 4.6 GB)."""
    print("[test_decode_long_and_shared_prefix] config5, 1 layer", flush=True)
    cfg = synth.config5(layers=1, pool_pages=70000)
    kw = sc.pack_kwargs(cfg, dec_grid_waves=1024, dec_min_pages=8)
    _check_step(cfg, cfg, dict(kw, device=gpu), 105, "config5", kernel_only=False)


@pytest.mark.gpu
@pytest.mark.parametrize("minp", [8, 1])
def test_decode_shared_prefix_groups(gpu, minp):
    """Config 5's decode batch with its shared prefixes attended once per group
    (dec_prefix_pages): 4 groups of 24 sequences whose first 128 pages are the same; each
    group's prefix items (8 kv heads x 8 chunks of 16 pages x 3 octets) leave partials that
    start every member's streams at page 128.  Plan bit-exact against the oracle, decode
    rows within tolerance and within one bf16 step of the oracle per element."""
    print(f"[test_decode_shared_prefix_groups] config5, 1 layer, min pages {minp}", flush=True)
    cfg = synth.config5(layers=1, pool_pages=70000)
    kw = sc.pack_kwargs(cfg, dec_grid_waves=1024, dec_min_pages=8, dec_prefix_pages=minp,
                        dec_pre_cap=4096)
    _check_step(cfg, cfg, dict(kw, device=gpu), 107, f"config5-prefix{minp}")


@pytest.mark.gpu
@pytest.mark.parametrize("seed", range(4))
def test_decode_prefix_random_groups(gpu, seed):
    """Random decode batches whose tables share leading runs of any length (groups of 2
    or more with prefixes from 1 page up, chunked prefixes, octets with fewer than 8
    members), beside prefill rows; the whole step against the oracle."""
    rng = np.random.default_rng(700 + seed)
    R = int(rng.choice([12, 40, 120]))
    pool_pages = 16384
    perm = iter(rng.permutation(pool_pages).astype(np.int32).tolist())
    runs = [[next(perm) for _ in range(128)] for _ in range(3)]  # shared leading runs
    comp, nnew, tabs = [], [], []
    for _ in range(R):
        dec = rng.random() < 0.7
        c = int(rng.integers(0, 2000))
        n = 1 if dec else int(rng.integers(2, 300))
        nb = synth.cdiv(c + n, PAGE)
        # a shared run covers only pages that hold cached keys of every reader (no row of
        # this step writes into them); the rest are the request's own
        k = min(int(rng.integers(0, nb + 1)), c // PAGE, 128)
        run = runs[int(rng.integers(0, 3))]
        tabs.append(np.array(run[:k] + [next(perm) for _ in range(nb - k)], np.int32))
        comp.append(c)
        nnew.append(n)
    cfg = synth._assemble(f"prefix-rand{seed}", comp, nnew, tabs, pool_pages, 4096)
    print(f"[test_decode_prefix_random_groups] seed={seed} R={R} rows={cfg.rows}", flush=True)
    kw = sc.pack_kwargs(cfg, dec_grid_waves=int(rng.choice([64, 1024])), dec_min_pages=2,
                        dec_prefix_pages=1, dec_pre_cap=4096)
    _check_step(cfg, cfg, dict(kw, device=gpu), 800 + seed, f"prefix-rand{seed}")


@pytest.mark.gpu
def test_pages_outside_pool_read_as_zeros(gpu):
    """Block-table entries outside the pool (one past the end, one negative) in two decode
    sequences and in a prefill's cached prefix: the pack flags the batch (status 4), and
    both attention kernels read those pages as zeros (keys score 0, add nothing to the
    numerator), as the oracle does; the rows' own pages are valid, so the append is
    unaffected."""
    print("[test_pages_outside_pool_read_as_zeros] config1 + 70-row prefill on a 40-token prefix",
          flush=True)
    base = synth.config1()
    rng = np.random.default_rng(31)
    used = set(base.bt_pages.tolist())
    free = np.array([p for p in rng.permutation(base.pool_pages) if p not in used][:7], np.int32)
    tabs = [t.copy() for t in base.tables()] + [free]
    tabs[3][5] = base.pool_pages + 7   # decode, 512 keys: page 5 of 32
    tabs[1][2] = -3                     # decode, 100 keys: page 2 of 7
    tabs[4][1] = base.pool_pages        # prefill: page 1 of the 40-token cached prefix
    cfg = synth._assemble("bad-pages", list(base.computed) + [40], list(base.n_new) + [70],
                          tabs, base.pool_pages, base.max_ctx)
    kw = sc.pack_kwargs(cfg, dec_grid_waves=64, dec_min_pages=2)
    _check_step(cfg, cfg, dict(kw, device=gpu), 131, "bad-pages")


@pytest.mark.gpu
def test_prefix_groups_with_pages_outside_pool(gpu):
    """A shared-prefix group whose common leading pages include one past the pool's end
    and one negative id: the pack flags the batch (status 4) and still plans the group,
    the prefix items read those pages as zeros, as every member's own stream would, and
    the decode rows match the oracle's."""
    rng = np.random.default_rng(77)
    pool_pages = 4096
    perm = iter(rng.permutation(pool_pages).astype(np.int32).tolist())
    run = [next(perm) for _ in range(20)]
    run[6] = pool_pages + 11
    run[13] = -5
    comp, nnew, tabs = [], [], []
    for i in range(6):
        c = int(rng.integers(20 * PAGE, 20 * PAGE + 300))
        nb = synth.cdiv(c + 1, PAGE)
        tabs.append(np.array(run + [next(perm) for _ in range(nb - 20)], np.int32))
        comp.append(c)
        nnew.append(1)
    cfg = synth._assemble("prefix-bad-pages", comp, nnew, tabs, pool_pages, 4096)
    print("[test_prefix_groups_with_pages_outside_pool] 6 decodes on a 20-page shared run",
          flush=True)
    kw = sc.pack_kwargs(cfg, dec_grid_waves=64, dec_min_pages=2, dec_prefix_pages=2,
                        dec_pre_cap=4096)
    from oracle import oracle as orc
    kwp = {k: v for k, v in kw.items() if k != "device"}
    pk = orc.pack(cfg.computed, cfg.n_new, cfg.bt_off, cfg.bt_pages, **kwp)
    assert int(pk["meta"][7]) == 4 and int(pk["meta"][11]) == 1  # flagged, one group
    _check_step(cfg, cfg, dict(kw, device=gpu), 177, "prefix-bad-pages")


@pytest.mark.gpu
def test_mixed_step_decode_on_side_stream(gpu):
    """Config 4 with the decode on a second stream, concurrent with the prefill: the output
    and the pool are bit-identical to the one-stream step (the two write disjoint rows).
    With dec_share the decode plan is cut for the CUs the prefill leaves: the pool and the
    prefill rows stay bit-identical, the decode rows within one bf16 step (other cuts of
    the same streams), and the plan equals the oracle's."""
    import torch

    from oracle import oracle as orc

    print("[test_mixed_step_decode_on_side_stream] config4", flush=True)
    cfg = synth.config4()
    sel_req, sel_n = orc.schedule(cfg.num_tokens, cfg.computed, cfg.token_budget,
                                  cfg.prefill_chunk)
    tabs = cfg.tables()
    sub = synth._assemble("config4-selected", cfg.computed[sel_req], sel_n,
                          [tabs[i] for i in sel_req], cfg.pool_pages, cfg.max_ctx)
    kw = sc.pack_kwargs(sub, dec_grid_waves=2048, dec_min_pages=8)
    rng = np.random.default_rng(105)
    qkv_host = synth.rand_bf16(rng, (sub.rows, QKV_STRIDE))
    wq, wk = synth.norm_weights()
    res = []
    for side, share in ((None, 0), (torch.cuda.Stream(device=gpu), 0),
                        (torch.cuda.Stream(device=gpu), 1)):
        pool = make_pool(cfg.pool_pages, 105, gpu)
        kws = dict(kw, dec_share=share)
        step, qkv, out = gpu_chain(cfg, qkv_host, pool, wq, wk, gpu, kws, schedule=True,
                                   side_stream=side)
        res.append((out.view(torch.int16).cpu().numpy(), pool.view(torch.int16).cpu().numpy()))
        if share:
            ref = orc.pack(sub.computed, sub.n_new, sub.bt_off, sub.bt_pages, **kws)
            check_pack(step, ref, sub.n_reqs, sub.rows, kws)
            waves = int(step.meta_host()[4])
            print(f"  dec_share: {waves} decode waves of {kw['dec_grid_waves']}", flush=True)
            assert 4 <= waves < kw["dec_grid_waves"] and waves % 4 == 0
            drows = ref["cu_seqlens"][ref["decode_rids"][: int(ref["meta"][1])]]
        del pool
    assert np.array_equal(res[0][0], res[1][0])
    assert np.array_equal(res[0][1], res[1][1])
    assert np.array_equal(res[0][1], res[2][1])
    prow = np.setdiff1d(np.arange(sub.rows), drows)
    assert np.array_equal(res[0][0][prow], res[2][0][prow])
    bits = lambda o: o[drows].view(np.uint16)  # noqa: E731
    sc.assert_decode_rows_close(bits(res[2][0]), bits(res[0][0]), "dec_share")


@pytest.mark.gpu
def test_decode_at_128k_context(gpu):
    """Decode sequences at 131072 and 65537 keys (8192 and 4097 pages per stream, each
    stream cut across many wavefronts) beside short ones, and a 3-row prefill chunk on a
    100000-token prefix: end to end against the oracle."""
    print("[test_decode_at_128k_context] 131072 / 65537 / 300 / 17 keys + 3-row chunk",
          flush=True)
    rng = np.random.default_rng(128)
    L = [131072, 65537, 300, 17]
    pool = 8192 + 4097 + 64 + 6300
    perm = rng.permutation(pool).astype(np.int32)
    tabs, o = [], 0
    for x in L + [100003]:
        k = synth.cdiv(x, PAGE)
        tabs.append(perm[o:o + k])
        o += k
    cfg = synth._assemble("128k", [x - 1 for x in L] + [100000], [1, 1, 1, 1, 3], tabs, pool,
                          131072)
    kw = sc.pack_kwargs(cfg, dec_grid_waves=1024, dec_min_pages=8)
    _check_step(cfg, cfg, dict(kw, device=gpu), 128, "128k")


@pytest.mark.gpu
def test_prefill_tiles_bit_identical(gpu):
    """Ragged prefill rows around the tile edges (2, 31, 32, 33, 63, 64, 65, 97, 128, 129 and
    300 rows, fresh and on cached prefixes that end inside a page): the 64-row items (two
    32-row blocks per wave) give bit-for-bit the output of the 32-row items, and both are
    within tolerance of the oracle."""
    import torch

    print("[test_prefill_tiles_bit_identical] 11 prompts, tiles 32 and 64", flush=True)
    rng = np.random.default_rng(64)
    n_new = [2, 31, 32, 33, 63, 64, 65, 97, 128, 129, 300]
    computed = [0, 0, 5, 16, 0, 1000, 31, 0, 2047, 3, 90]
    counts = [synth.cdiv(c + n, PAGE) for c, n in zip(computed, n_new)]
    pool_pages = sum(counts) + 40
    cfg = synth._assemble("tile-edges", computed, n_new, synth._place(rng, pool_pages, counts),
                          pool_pages, 4096)
    outs = {}
    for tile in (32, 64):
        kw = sc.pack_kwargs(cfg, dec_grid_waves=64, dec_min_pages=2, pre_tile_q=tile)
        _check_step(cfg, cfg, dict(kw, device=gpu), 640, f"tile-edges tile {tile}")
        pool = make_pool(cfg.pool_pages, 1640, gpu)
        qkv_h = synth.rand_bf16(np.random.default_rng(7), (cfg.rows, QKV_STRIDE))
        wq, wk = synth.norm_weights()
        _, _, out = gpu_chain(cfg, qkv_h, pool, wq, wk, gpu, kw)
        outs[tile] = out.view(torch.int16).cpu().numpy()[: cfg.rows]
        del pool
    assert np.array_equal(outs[32], outs[64])


def _floor_checksum(pool_u16, pool_pages, bt, max_blocks, dec_seqs, n_decode):
    """XOR of every 32-bit word of every (page, kv head) run a decode plan covers, each run
    once per decode sequence that reads it; pages outside the pool count as page 0."""
    runs = pool_u16.view(np.uint32).reshape(-1, PAGE * HEAD_DIM)  # one row per run (K+V)
    run_x = np.bitwise_xor.reduce(runs, axis=1)
    acc = np.uint32(0)
    for r, _row, z, _ in dec_seqs[:n_decode]:
        L = int(z) & ((1 << 30) - 1)
        ids = bt[r * max_blocks: r * max_blocks + (L + PAGE - 1) // PAGE].astype(np.int64)
        ids = np.where((ids >= 0) & (ids < pool_pages), ids, 0)
        idx = (ids[:, None] * 8 + np.arange(8)[None, :]).reshape(-1)
        acc ^= np.bitwise_xor.reduce(run_x[idx])
    return int(acc)


@pytest.mark.gpu
@pytest.mark.parametrize("cfgno,waves", [(1, 16), (2, 1024), (2, 2048), (2, 3000)])
def test_decode_read_floor_reads_every_run_once(gpu, cfgno, waves):
    """fqa_decode_read_floor (the bench's HBM floor for the decode) must read exactly the
    pages fqa_decode reads: the XOR of all lanes' folded words equals the XOR of all words
    of every (page, kv head) run of the plan, each once per decode sequence (bit-exact;
    a page skipped, read twice or read at a wrong address changes it).  Config 1 adds two
    block-table entries outside the pool, which both kernels read as page 0."""
    import torch

    print(f"[test_decode_read_floor_reads_every_run_once] config{cfgno} waves={waves}",
          flush=True)
    cfg = synth.CONFIGS[cfgno]()
    if cfgno == 1:
        tabs = [t.copy() for t in cfg.tables()]
        tabs[3][5] = cfg.pool_pages + 7
        tabs[1][2] = -3
        cfg = synth._assemble("bad-pages", list(cfg.computed), list(cfg.n_new), tabs,
                              cfg.pool_pages, cfg.max_ctx)
    kw = sc.pack_kwargs(cfg, dec_grid_waves=waves, dec_min_pages=2)
    kwp = {k: v for k, v in kw.items() if k != "device"}
    rng = np.random.default_rng(7)
    qkv_h = synth.rand_bf16(rng, (cfg.rows, QKV_STRIDE))
    wq, wk = synth.norm_weights()
    pool = make_pool(cfg.pool_pages, 77, gpu)
    step, _qkv, _out = gpu_chain(cfg, qkv_h, pool, wq, wk, gpu, kwp)
    step.workspace.zero_()
    step.decode_read_floor(pool[0])
    torch.cuda.synchronize()
    meta = step.meta.cpu().numpy()
    n_decode, n_waves = int(meta[1]), int(meta[4])
    assert n_decode == cfg.n_reqs and n_waves > 0
    sink = step.workspace.view(torch.int32).cpu().numpy().view(np.uint32)
    got = int(np.bitwise_xor.reduce(sink[: n_waves * 64]))
    want = _floor_checksum(_host_u16(pool).reshape(-1), cfg.pool_pages,
                           step.block_tables.cpu().numpy().reshape(-1), kwp["max_blocks"],
                           step.dec_seqs.cpu().numpy().reshape(-1, 4), n_decode)
    assert got == want, (hex(got), hex(want))


def _random_step(seed: int):
    """A random mixed step: 3-40 requests, each a decode (context 1-3000) or a prefill chunk
    (2-200 rows on a 0-1000-token prefix, at most 4 of them), some sharing their first
    pages with an earlier request's (full pages only, never appended to), page ids shuffled
    over a pool with free pages between them."""
    rng = np.random.default_rng(seed)
    R = int(rng.integers(3, 41))
    comp, new, tabs = [], [], []
    n_pre = 0
    for _ in range(R):
        if n_pre < 4 and rng.random() < 0.25:
            c = int(rng.integers(0, 1001)) if rng.random() < 0.6 else 0
            n = int(rng.integers(2, 201))
            n_pre += 1
        else:
            c = int(rng.integers(0, 3000))
            n = 1
        comp.append(c)
        new.append(n)
    need = [synth.cdiv(c + n, PAGE) for c, n in zip(comp, new)]
    pool = int(sum(need) * 1.5) + 64
    perm = rng.permutation(pool).astype(np.int32)
    o = 0
    for r in range(R):
        t = perm[o:o + need[r]].copy()
        o += need[r]
        full = comp[r] // PAGE  # pages this request reads but never writes
        if r > 0 and full > 0 and rng.random() < 0.3:
            src = int(rng.integers(0, r))
            k = min(full, comp[src] // PAGE)
            if k > 0:
                t[:k] = tabs[src][:k]
        tabs.append(t)
    return synth._assemble(f"random{seed}", comp, new, tabs, pool, 4096)


@pytest.mark.gpu
@pytest.mark.parametrize("seed", range(6))
def test_random_steps(gpu, seed):
    """Random mixed steps (decode contexts, prefill prefixes and chunk lengths, shared
    prefix pages, decode grid 16-2048 waves, minimum pages per wave, prefill tile, the
    decode planned for a share of the CUs, shared-prefix decode groups) end to end and
    kernel-only against the oracle; decode rows within one bf16 step."""
    cfg = _random_step(seed)
    rng = np.random.default_rng(1000 + seed)
    waves = int(rng.choice([16, 256, 1024, 2048]))
    min_pages = int(rng.choice([1, 2, 8]))
    tile = int(rng.choice([32, 64]))
    prefix = (0, 1, 2)[seed % 3]
    print(f"[test_random_steps] seed={seed} reqs={cfg.n_reqs} rows={cfg.rows} "
          f"waves={waves} min_pages={min_pages} tile={tile} dec_share={seed % 2} "
          f"dec_prefix_pages={prefix}", flush=True)
    kw = sc.pack_kwargs(cfg, dec_grid_waves=waves, dec_min_pages=min_pages, pre_tile_q=tile,
                        dec_share=seed % 2, dec_prefix_pages=prefix, dec_pre_cap=4096)
    _check_step(cfg, cfg, dict(kw, device=gpu), 500 + seed, f"random{seed}")


@pytest.mark.gpu
@pytest.mark.parametrize("prefix", [0, 1])
def test_decode_at_maximum_requests(gpu, prefix):
    """FQA_MAX_REQS (2048) decode sequences of 1-200 keys on the default 1024-wave grid: each
    wave walks many short streams (its segment loop reloads q and restarts the page
    rotation per stream), the combine runs on its largest grid, and some sequences share
    their first pages (prefix=1: those form shared-prefix groups).  End to end and
    kernel-only against the oracle."""
    from flashqwen_amd import _lib

    rng = np.random.default_rng(4096)
    R = _lib.FQA_MAX_REQS
    L = rng.integers(1, 201, size=R)
    need = [synth.cdiv(int(x), PAGE) for x in L]
    pool = sum(need) + 1000
    perm = rng.permutation(pool).astype(np.int32)
    tabs, o = [], 0
    for r in range(R):
        t = perm[o:o + need[r]].copy()
        o += need[r]
        full = (int(L[r]) - 1) // PAGE
        if r > 0 and full > 0 and rng.random() < 0.2:
            src = int(rng.integers(0, r))
            k = min(full, (int(L[src]) - 1) // PAGE)
            t[:k] = tabs[src][:k]
        tabs.append(t)
    cfg = synth._assemble("max-reqs", L - 1, np.ones(R, np.int32), tabs, pool, 4096)
    print(f"[test_decode_at_maximum_requests] R={R} keys={int(L.sum())} prefix={prefix}",
          flush=True)
    kw = sc.pack_kwargs(cfg, dec_grid_waves=1024, dec_min_pages=1, dec_prefix_pages=prefix,
                        dec_pre_cap=4096)
    _check_step(cfg, cfg, dict(kw, device=gpu), 2048, "max-reqs")


@pytest.mark.gpu
def test_invariant_under_page_relabelling_and_grid(gpu):
    """Two invariances of the path on a random mixed step (decodes, prefill chunks, shared
    prefix pages): relabelling every page id, with the pool's pages moved to match, leaves
    the attention output and the appended K/V bit-identical (the kernels do the same loads
    in the same order, only at other addresses); and the decode grid (where stream-K cuts
    the streams) changes decode rows by fp32 merge order only: within one bf16 step."""
    import torch

    cfg = _random_step(45)  # 38 requests, 4 prefill chunks, shared prefix pages
    kw = sc.pack_kwargs(cfg, dec_grid_waves=1024, dec_min_pages=1)
    kwp = {k: v for k, v in kw.items() if k != "device"}
    rng = np.random.default_rng(9)
    qkv_h = synth.rand_bf16(rng, (cfg.rows, QKV_STRIDE))
    wq, wk = synth.norm_weights()
    print(f"[test_invariant_under_page_relabelling_and_grid] reqs={cfg.n_reqs} rows={cfg.rows}",
          flush=True)
    pool = make_pool(cfg.pool_pages, 77, gpu)
    base = pool.clone()
    step, _q, out = gpu_chain(cfg, qkv_h, pool, wq, wk, gpu, kwp)
    out_a, pool_a = _host_u16(out)[: cfg.rows], pool

    # relabel: page p -> perm[p], and move the pool's pages with it
    perm = np.random.default_rng(10).permutation(cfg.pool_pages).astype(np.int32)
    cfg_b = synth._assemble("relabelled", cfg.computed, cfg.n_new,
                            [perm[t] for t in cfg.tables()], cfg.pool_pages, cfg.max_ctx)
    inv = np.empty_like(perm)
    inv[perm] = np.arange(cfg.pool_pages, dtype=np.int32)
    pool_b = base[:, torch.from_numpy(inv.astype(np.int64)).to(gpu)].contiguous()
    step_b, _q, out_b = gpu_chain(cfg_b, qkv_h, pool_b, wq, wk, gpu, kwp)
    assert np.array_equal(_host_u16(out_b)[: cfg.rows], out_a)
    moved_back = pool_b[:, torch.from_numpy(perm.astype(np.int64)).to(gpu)]
    assert torch.equal(moved_back.view(torch.int16), pool_a.view(torch.int16))

    # other decode grids: decode rows within one bf16 step of the 1024-wave result
    drows = step.cu_seqlens.cpu().numpy()[step.decode_rids.cpu().numpy()[
        : int(step.meta.cpu().numpy()[1])]]
    for waves in (7, 256, 3000):
        kw_g = sc.pack_kwargs(cfg, dec_grid_waves=waves, dec_min_pages=1)
        kwp_g = {k: v for k, v in kw_g.items() if k != "device"}
        _s, _q, out_g = gpu_chain(cfg, qkv_h, base.clone(), wq, wk, gpu, kwp_g)
        got = _host_u16(out_g)[: cfg.rows]
        sc.assert_decode_rows_close(got[drows], out_a[drows], f"grid {waves}")
        prow = np.setdiff1d(np.arange(cfg.rows), drows)
        assert np.array_equal(got[prow], out_a[prow])  # prefill rows do not depend on it
