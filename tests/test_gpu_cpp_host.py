"""The C++ host mirror (include/fqa_step.hpp: StepContext::PrepareInputs + RunLayer over the
C ABI) run as a compiled program on the GPU, checked against the CPU oracle."""
from __future__ import annotations

import subprocess
from pathlib import Path

import numpy as np
import pytest

from flashqwen_amd import synth
from tests import stepcase as sc

EXE = Path(__file__).resolve().parent / "cpp" / "step_cpp"


@pytest.mark.gpu
def test_cpp_step_matches_oracle(gpu, tmp_path):
    if not EXE.exists():
        pytest.fail(f"{EXE} not built (run __graft_entry__.build())")
    base = synth.config1()
    rng = np.random.default_rng(21)
    used = set(base.bt_pages.tolist())
    free = np.array([p for p in rng.permutation(base.pool_pages) if p not in used][:5], np.int32)
    # decodes of config 1 plus a 70-token fresh prompt (prefill)
    cfg = synth._assemble("cpp", list(base.computed) + [0], list(base.n_new) + [70],
                          base.tables() + [free], base.pool_pages, base.max_ctx)
    T, R = cfg.rows, cfg.n_reqs
    qkv = synth.rand_bf16(rng, (T, synth.QKV_STRIDE))
    pool = synth.rand_bf16(rng, sc.pool_elems(cfg.pool_pages))
    wq, wk = synth.norm_weights()
    with open(tmp_path / "in.bin", "wb") as f:
        np.array([R, T, cfg.max_ctx, cfg.pool_pages], np.int32).tofile(f)
        for a in (cfg.computed, cfg.n_new, cfg.bt_off, cfg.bt_pages):
            np.asarray(a, np.int32).tofile(f)
        qkv.tofile(f)
        wq.astype(np.float32).tofile(f)
        wk.astype(np.float32).tofile(f)
        pool.tofile(f)
    print(f"[test_cpp_step_matches_oracle] R={R} T={T}", flush=True)
    subprocess.run([str(EXE), str(tmp_path / "in.bin"), str(tmp_path / "out.bin")], check=True,
                   timeout=120)
    raw = np.fromfile(tmp_path / "out.bin", np.uint8)
    meta = raw[:64].view(np.int32)
    q_got = raw[64:64 + T * synth.QKV_STRIDE * 2].view(np.uint16).reshape(T, -1)
    o_got = raw[64 + T * synth.QKV_STRIDE * 2:].view(np.uint16).reshape(T, -1)
    kw = sc.pack_kwargs(cfg, dec_grid_waves=int(meta[4]) or 1, dec_min_pages=8)
    ref = sc.oracle_chain(cfg, qkv, pool, wq, wk, kw)
    assert meta[:4].tolist() == ref["pack"]["meta"][:4].tolist()
    assert meta[7] == 0
    sc.assert_rope_close(q_got[:, :4096], ref["qkv"][:, :4096], "q")
    mx, mean = sc.att_errors(o_got, ref["out"])
    assert mx <= sc.ATT_MAX_ABS and mean <= sc.ATT_MEAN_ABS, (mx, mean)
