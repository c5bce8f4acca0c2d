"""fqa_decode_noalloc (the decode with its partials in the library's fixed device array)
gives the same bytes as fqa_decode with a caller workspace, on two calls in a row, the
second with a smaller batch, and refuses plans larger than its array."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest
import torch

from flashqwen_amd import _lib, synth
from flashqwen_amd.step import AttnStep, alloc_pool


def _run(cfg, dev, seed, dec_grid_waves):
    lib = _lib.load()
    rng = np.random.default_rng(seed)
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(dev)  # noqa: E731
    qkv = t(synth.rand_bf16(rng, (cfg.rows, synth.QKV_STRIDE)).view(np.int16)).view(torch.bfloat16)
    pool = alloc_pool(cfg.pool_pages, 1, dev)
    pool.view(-1).normal_(generator=torch.Generator(device=dev).manual_seed(seed))
    step = AttnStep(max_rows=cfg.rows, max_reqs=cfg.n_reqs, max_ctx=cfg.max_ctx,
                    pool_pages=cfg.pool_pages, device=dev, dec_grid_waves=dec_grid_waves)
    step.prepare_inputs(t(cfg.computed), t(cfg.n_new), t(cfg.bt_off), t(cfg.bt_pages))
    wq, wk = synth.norm_weights()
    step.head_norm_rope_store_kv(qkv, pool[0], t(wq), t(wk))
    out_ws = torch.full((cfg.rows, 4096), float("nan"), dtype=torch.bfloat16, device=dev)
    out_na = torch.full_like(out_ws, float("inf"))
    step.attn_decode(qkv, pool[0], out_ws)
    args = (C.byref(step.dims), qkv.data_ptr(), pool[0].data_ptr(), step.pool_pages,
            step.block_tables.data_ptr(), step.max_blocks, step.dec_waves.data_ptr(),
            step.dec_seqs.data_ptr(), step.meta.data_ptr(), step.dec_wave_cap, cfg.n_reqs)
    rc = lib.fqa_decode_noalloc(*args, out_na.data_ptr(), step.stream)
    assert rc == _lib.FQA_OK
    torch.cuda.synchronize()
    meta = step.meta_host()
    assert meta[7] == 0 and meta[1] == cfg.n_reqs
    a = out_ws.view(torch.int16).cpu().numpy()
    b = out_na.view(torch.int16).cpu().numpy()
    print(f"  rows={cfg.rows} waves={int(meta[4])} cap={step.dec_wave_cap}", flush=True)
    assert np.array_equal(a, b)
    return step, args


@pytest.mark.gpu
def test_noalloc_decode_equals_workspace_decode(gpu):
    # config 2 over the full grid (2048 waves, streams cut into partials), then config 1
    # over a smaller one: the second call reuses the array the first left behind
    print("[test_noalloc_decode_equals_workspace_decode] config2", flush=True)
    _run(synth.config2(), gpu, 3, None)
    print("[test_noalloc_decode_equals_workspace_decode] config1", flush=True)
    step, args = _run(synth.config1(), gpu, 4, 16)
    lib = _lib.load()
    # a plan larger than the array is refused before any launch
    big = list(args)
    big[9] = _lib.FQA_DECODE_NOALLOC_MAX_WAVES + 1
    assert lib.fqa_decode_noalloc(*big, None, step.stream) == _lib.FQA_EINVAL
    # the largest plan the array holds: 4096 wavefronts over config 2 (every stream cut),
    # bit-equal to the workspace decode
    print("[test_noalloc_decode_equals_workspace_decode] config2 at the cap", flush=True)
    _, capargs = _run(synth.config2(), gpu, 5, _lib.FQA_DECODE_NOALLOC_MAX_WAVES)
    assert capargs[9] == _lib.FQA_DECODE_NOALLOC_MAX_WAVES
    # zero work: nothing launched, nothing looked up
    big[9] = 0
    assert lib.fqa_decode_noalloc(*big, None, step.stream) == _lib.FQA_OK
