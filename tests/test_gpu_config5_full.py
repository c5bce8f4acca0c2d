"""Config 5 at full size: one decode step over all 36 layers of a ~200 GB pool (84771 pages
per layer, 5.5 GB each, so every layer but the first sits beyond 5 GB of the allocation and
the last beyond 190 GB), then layers 0, 17 and 35 checked against the CPU oracle on those
layers' pages: norm/RoPE of q and k, the append of k and v, and the attention kernels on the
GPU's own post-append q and pool.  The decode runs as bench.py runs it: with the
shared-prefix groups (dec_prefix_pages 8: the 4 groups of 24 sequences attend their 128-page
prefix once per 8 members)."""
from __future__ import annotations

import numpy as np
import pytest

from flashqwen_amd import synth
from flashqwen_amd.synth import HEAD_DIM, N_Q, PAGE, QKV_STRIDE
from tests import stepcase as sc


@pytest.mark.gpu
def test_config5_36_layers_full_pool(gpu):
    import torch

    from flashqwen_amd.step import AttnStep, alloc_pool
    from oracle import oracle as orc

    torch.cuda.empty_cache()
    cfg = synth.config5()
    L, T, R = cfg.layers, cfg.rows, cfg.n_reqs
    print(f"[test_config5_36_layers_full_pool] layers={L} pages/layer={cfg.pool_pages} "
          f"pool={L * cfg.pool_pages * 65536 / 1e9:.1f} GB", flush=True)
    pool = alloc_pool(cfg.pool_pages, L, gpu)
    g = torch.Generator(device=gpu)
    g.manual_seed(55)
    flat = pool.view(-1)
    for s in range(0, flat.numel(), 1 << 30):
        flat[s: s + (1 << 30)].normal_(generator=g)
    rng = np.random.default_rng(56)
    qkv_h = synth.rand_bf16(rng, (L, T, QKV_STRIDE))
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(gpu)  # noqa: E731
    qkv = t(qkv_h.view(np.int16)).view(torch.bfloat16)
    out = torch.zeros((L, T, N_Q * HEAD_DIM), dtype=torch.bfloat16, device=gpu)
    wq, wk = synth.norm_weights()
    step = AttnStep(max_rows=T, max_reqs=R, max_ctx=cfg.max_ctx, pool_pages=cfg.pool_pages,
                    device=gpu, dec_prefix_pages=8)
    step.prepare_inputs(t(cfg.computed), t(cfg.n_new), t(cfg.bt_off), t(cfg.bt_pages))
    wq_d, wk_d = t(wq), t(wk)
    for l in range(L):
        step.run_layer(qkv[l], pool[l], wq_d, wk_d, out[l], prefill=False)
    torch.cuda.synchronize()
    print("  step done", flush=True)

    kw = sc.pack_kwargs(cfg, dec_grid_waves=step.dec_grid_waves, dec_min_pages=8,
                        dec_prefix_pages=8, dec_pre_cap=step.dec_pre_cap)
    pk = orc.pack(cfg.computed, cfg.n_new, cfg.bt_off, cfg.bt_pages, **kw)
    assert np.array_equal(step.meta_host(), pk["meta"])
    assert int(pk["meta"][11]) == 4 and int(pk["meta"][10]) > 0  # the 4 groups were found
    cos, sin = orc.rope_tables(cfg.max_ctx)
    pages, toks = sc.written_mask(pk, T)
    no_slot = np.full(T, -1, np.int32)
    for l in (0, 17, 35):
        q_got = qkv[l].view(torch.int16).cpu().numpy().view(np.uint16)
        pool_l = pool[l].view(torch.int16).reshape(-1).cpu().numpy().view(np.uint16)
        # norm + RoPE of q and k (the oracle appends nothing: no row has a slot)
        ref_q = qkv_h[l].copy()
        orc.qknorm_rope_append(ref_q, wq, wk, cos, sin, pk["positions"], no_slot, T,
                               np.zeros(sc.pool_elems(1), np.uint16), 1, write_k=True)
        sc.assert_rope_close(q_got[:, : N_Q * HEAD_DIM], ref_q[:, : N_Q * HEAD_DIM], f"q{l}")
        # the append: k (normalised) and v of every row at its slot
        for r in range(T):
            for kvh in range(8):
                run = (pages[r] * 8 + kvh) * 2 * PAGE * HEAD_DIM
                k_got = pool_l[run + toks[r] * HEAD_DIM: run + (toks[r] + 1) * HEAD_DIM]
                k_ref = ref_q[r, (N_Q + kvh) * HEAD_DIM: (N_Q + kvh + 1) * HEAD_DIM]
                sc.assert_rope_close(k_got, k_ref, f"k{l}")
                v_idx = run + PAGE * HEAD_DIM + np.arange(HEAD_DIM) * PAGE + toks[r]
                v_ref = qkv_h[l][r, (N_Q + 8 + kvh) * HEAD_DIM: (N_Q + 9 + kvh) * HEAD_DIM]
                assert np.array_equal(pool_l[v_idx], v_ref), (l, r, kvh)
        # attention kernels on the GPU's own post-append q and pool
        o_ref = np.zeros((T, N_Q * HEAD_DIM), np.uint16)
        orc.decode(q_got, pool_l, cfg.pool_pages, pk["block_tables"], kw["max_blocks"],
                   pk["cu_seqlens"], pk["positions"], pk["decode_rids"], R, o_ref)
        o_got = out[l].view(torch.int16).cpu().numpy().view(np.uint16)
        mx, mean = sc.att_errors(o_got, o_ref)
        print(f"  layer {l}: max-abs {mx:.3e} mean-abs {mean:.3e}", flush=True)
        assert mx <= sc.ATT_MAX_ABS and mean <= sc.ATT_MEAN_ABS, (l, mx, mean)
        sc.assert_decode_rows_close(o_got, o_ref, f"layer {l}")  # every row decodes
        del pool_l
    del pool, flat, qkv, out
    torch.cuda.empty_cache()
