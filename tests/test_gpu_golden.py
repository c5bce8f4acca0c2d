"""The HIP path on the committed golden step (tests/golden/step_small.npz): pack arrays
and the appended V bit-exact, the appended K within one bf16 ulp of the oracle's, the
attention output within the attention tolerance."""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

from tests import stepcase as sc

FIX = Path(__file__).resolve().parent / "golden" / "step_small.npz"


@pytest.mark.gpu
def test_gpu_matches_golden(gpu):
    import torch

    from flashqwen_amd.step import AttnStep
    from tests.golden import make_golden as mg

    print("[test_gpu_matches_golden]", flush=True)
    g = np.load(FIX)
    cfg, qkv, pool, wq, wk, kw = mg.inputs()
    step = AttnStep(max_rows=kw["max_rows"], max_reqs=cfg.n_reqs, max_ctx=cfg.max_ctx,
                    pool_pages=cfg.pool_pages, device=gpu, dec_grid_waves=kw["dec_grid_waves"],
                    dec_min_pages=kw["dec_min_pages"], pre_tile_q=kw["pre_tile_q"])
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(gpu)  # noqa: E731
    d_qkv = t(qkv.view(np.int16)).view(torch.bfloat16)
    d_pool = t(pool.view(np.int16)).view(torch.bfloat16)
    out = torch.zeros((cfg.rows, 4096), dtype=torch.bfloat16, device=gpu)
    step.prepare_inputs(t(cfg.computed), t(cfg.n_new), t(cfg.bt_off), t(cfg.bt_pages))
    step.run_layer(d_qkv, d_pool, t(wq), t(wk), out)
    torch.cuda.synchronize()
    T = cfg.rows
    assert step.meta_host()[:4].tolist() == g["meta"][:4].tolist()
    assert np.array_equal(step.positions[:T].cpu().numpy(), g["positions"])
    assert np.array_equal(step.slot_mapping[:T].cpu().numpy(), g["slot_mapping"])
    kv = mg.appended(d_pool.view(torch.int16).cpu().numpy().view(np.uint16),
                     g["slot_mapping"])
    assert np.array_equal(kv[:, :, 128:], g["kv"][:, :, 128:])  # V exact
    # K: within one bf16 ulp of the oracle's value (+1e-5 absolute for cancelling values)
    kg = (kv[:, :, :128].astype(np.uint32) << 16).view(np.float32)
    kr = (g["kv"][:, :, :128].astype(np.uint32) << 16).view(np.float32)
    ulp = np.ldexp(1.0, np.frexp(np.abs(kr))[1] - 8)
    assert np.all(np.abs(kg - kr) <= ulp + 1e-5)
    mx, mean = sc.att_errors(out.view(torch.int16).cpu().numpy().view(np.uint16), g["out"])
    print(f"max-abs {mx:.3e} mean-abs {mean:.3e}")
    assert mx <= sc.ATT_MAX_ABS and mean <= sc.ATT_MEAN_ABS
