"""The step as a captured HIP graph (include/fqa_step.hpp: StepContext::UploadBatch +
StepGraph, the reference's GraphCache): one graph, captured once, replayed for every
batch of a scheduler-driven workload over 3 layers (prefills, decodes, preemption, so the
batch shape changes from step to step), with uploads and synchronisation between the
replays.  Every step's attention output and the final pools must be bit-identical to the
eager run of the same workload (tests/cpp/graph_cpp)."""
from __future__ import annotations

import subprocess
from pathlib import Path

import numpy as np
import pytest

from flashqwen_amd import synth
from tests.test_sched import _script

EXE = Path(__file__).resolve().parent / "cpp" / "graph_cpp"


@pytest.mark.gpu
def test_step_graph_replays_match_eager(gpu, tmp_path):
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
    print("[test_step_graph_replays_match_eager] 10 seqs, 16 steps, 3 layers", flush=True)
    r = subprocess.run([str(EXE), str(tmp_path / "s.txt"), str(tmp_path / "w.bin")],
                       capture_output=True, text=True, timeout=120)
    print(r.stdout.strip(), r.stderr.strip())
    assert r.returncode == 0, (r.returncode, r.stdout, r.stderr)
    steps = int(r.stdout.split()[1])
    assert steps >= 10
