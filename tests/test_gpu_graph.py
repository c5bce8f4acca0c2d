"""The step as a captured HIP graph (include/fqa_step.hpp: StepContext::UploadBatch +
StepGraph, the reference's GraphCache): one graph, captured once, replayed for every
batch of a scheduler-driven workload over 3 layers (prefills, decodes, preemption, so the
batch shape changes from step to step), with uploads and synchronisation between the
replays.  Every step's attention output and the final pools must be bit-identical to the
eager run of the same workload (tests/cpp/graph_cpp), and every replay's output of every
layer is checked against the CPU oracle replaying the same steps on its own pools."""
from __future__ import annotations

import os
import subprocess
from pathlib import Path

import numpy as np
import pytest
import torch

from flashqwen_amd import synth
from tests import stepcase as sc
from tests.test_sched import _script

EXE = Path(__file__).resolve().parent / "cpp" / "graph_cpp"


@pytest.mark.gpu
@pytest.mark.parametrize("dec_share,dec_prefix", [(0, 0), (1, 0), (0, 2)])
def test_step_graph_replays_match_eager(gpu, tmp_path, dec_share, dec_prefix):
    """dec_share=1: both runs plan each mixed batch's decode for the CUs the prefill leaves,
    and the eager run also queues decode on the side stream.  dec_prefix=2: decodes sharing
    at least 2 leading pages (the prefix-cache hits on the common 70-token prompt start)
    attend them once per group (fqa_decode_prefix), in the graph and eagerly."""
    if not EXE.exists():
        pytest.fail(f"{EXE} not built (run __graft_entry__.build())")
    rng = np.random.default_rng(78)
    base = [int(x) for x in rng.integers(0, 50000, size=70)]
    specs = []
    for i in range(10):
        tail = [int(x) for x in rng.integers(0, 50000, size=int(rng.integers(1, 60)))]
        prompt = (base + tail) if i % 2 == 0 else tail + base[:20]
        specs.append(dict(id=i + 1, arrival=int(i // 2) * 2, cancel=-1,
                          max_new=int(rng.integers(2, 9)), max_ctx=512, stop=[], prompt=prompt))
    (tmp_path / "s.txt").write_text(_script((20, 6, 96, 48, True), 16, specs) + "512\n")
    wq, wk = synth.norm_weights()
    np.concatenate([wq.astype(np.float32), wk.astype(np.float32)]).tofile(tmp_path / "w.bin")
    print(f"[test_step_graph_replays_match_eager] 10 seqs, 16 steps, 3 layers, "
          f"dec_share={dec_share} dec_prefix={dec_prefix}", flush=True)
    env = dict(os.environ, FQA_DEC_SHARE=str(dec_share), FQA_DEC_PREFIX=str(dec_prefix))
    r = subprocess.run([str(EXE), str(tmp_path / "s.txt"), str(tmp_path / "w.bin"),
                        str(tmp_path / "graph.bin")], capture_output=True, text=True,
                       timeout=120, env=env)
    print(r.stdout.strip(), r.stderr.strip())
    assert r.returncode == 0, (r.returncode, r.stdout, r.stderr)
    steps = int(r.stdout.split()[1])
    assert steps >= 10

    # the captured path against the oracle: every replay, every layer
    layers, n_blocks, budget, slots = 3, 20, 96, 6
    raw = np.fromfile(tmp_path / "graph.bin", np.uint8)
    o = 0

    def take(dtype, n):
        nonlocal o
        a = raw[o:o + n * np.dtype(dtype).itemsize].view(dtype)
        o += n * np.dtype(dtype).itemsize
        return a

    pools = [np.zeros(sc.pool_elems(n_blocks), np.uint16) for _ in range(layers)]
    n_checked = shared = grouped = 0
    # the decode grid StepContext takes by default: one wavefront per SIMD
    grid = 4 * torch.cuda.get_device_properties(gpu).multi_processor_count
    while o < raw.size:
        t, R, T = (int(x) for x in take(np.int32, 3))
        computed, n_new = take(np.int32, R), take(np.int32, R)
        off = take(np.int32, R + 1)
        pages = take(np.int32, int(off[-1]))
        per_layer = [(take(np.uint16, T * synth.QKV_STRIDE).reshape(T, -1),
                      take(np.uint16, T * 4096).reshape(T, -1)) for _ in range(layers)]
        meta = take(np.int32, 16)
        tables = [pages[off[i]:off[i + 1]] for i in range(R)]
        cfg = synth._assemble(f"step{t}", computed, n_new, tables, n_blocks, 512)
        kw = sc.pack_kwargs(cfg, max_rows=budget, dec_grid_waves=grid, dec_min_pages=8,
                            max_reqs=slots, dec_share=dec_share, dec_prefix_pages=dec_prefix,
                            dec_pre_cap=4096)
        for l, (qkv_in, attn) in enumerate(per_layer):
            ref = sc.oracle_chain(cfg, qkv_in, pools[l], wq, wk, kw)
            if l == 0:
                # rows, decode and prefill counts, the decode plan's wavefront count, and
                # its prefix items and groups
                assert meta[:5].tolist() == ref["pack"]["meta"][:5].tolist(), t
                assert meta[10:12].tolist() == ref["pack"]["meta"][10:12].tolist(), t
                grouped += int(meta[11]) > 0
                if dec_share:  # steps whose plan the share changed
                    from oracle import oracle as orc
                    whole = orc.pack(cfg.computed, cfg.n_new, cfg.bt_off, cfg.bt_pages,
                                     **dict(kw, dec_share=0))
                    shared += int(meta[4]) != int(whole["meta"][4])
                assert meta[7] == 0
            mx, mean = sc.att_errors(attn, ref["out"])
            assert mx <= sc.ATT_MAX_ABS and mean <= sc.ATT_MEAN_ABS, (t, l, mx, mean)
            pools[l] = ref["pool"]
            n_checked += 1
        print(f"graph step {t}: R={R} T={T} checked {layers} layers (last max-abs {mx:.2e})")
    assert n_checked == steps * layers
    # (this workload's batches are small: the share rarely moves their plans; config 4's
    # binding share is checked in test_gpu_path.py::test_mixed_step_decode_on_side_stream)
    print(f"steps whose decode plan the share changed: {shared}; with prefix groups: {grouped}")
    if dec_prefix:
        assert grouped > 0  # the groups were exercised
