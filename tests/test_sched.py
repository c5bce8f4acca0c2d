"""The host scheduler and block allocator (include/fqa_sched.hpp, driven by tests/cpp/
sched_cpp) against an independent Python model (tests/sched_model.py) on scripted
workloads, with every step's selection also checked against the CPU oracle's BuildBatch
restatement (oracle/fqa_oracle.c, fqo_schedule).  Host code only: no GPU."""
from __future__ import annotations

import subprocess
from pathlib import Path

import numpy as np
import pytest

from tests import sched_model as sm

EXE = Path(__file__).resolve().parent / "cpp" / "sched_cpp"


def _script(cfg, n_steps, specs) -> str:
    nb, slots, budget, chunk, cache = cfg
    out = [f"{nb} {slots} {budget} {chunk} {int(cache)} {n_steps} {len(specs)}"]
    for s in specs:
        out.append(f"{s['id']} {s['arrival']} {s['cancel']} {s['max_new']} {s['max_ctx']} "
                   f"{len(s['stop'])} " + " ".join(map(str, s["stop"])) +
                   f" {len(s['prompt'])} " + " ".join(map(str, s["prompt"])))
    return "\n".join(out) + "\n"


def _cpp_trace(cfg, n_steps, specs) -> list[str]:
    if not EXE.exists():
        pytest.fail(f"{EXE} not built (run __graft_entry__.build())")
    r = subprocess.run([str(EXE)], input=_script(cfg, n_steps, specs), capture_output=True,
                       text=True, check=True, timeout=60)
    return r.stdout.strip().split("\n")


def _oracle_check(budget, chunk):
    from oracle import oracle as orc

    def check(snapshot, picked):
        ids = [s[0] for s in snapshot]
        ntok = np.array([s[1] for s in snapshot], np.int32)
        comp = np.array([s[2] for s in snapshot], np.int32)
        req, n = orc.schedule(ntok, comp, budget, chunk)
        assert [(ids[i], int(k)) for i, k in zip(req, n)] == picked, (snapshot, picked)
    return check


def _random_specs(rng, n_seqs, n_steps, shared_prompts):
    bases = [list(rng.integers(0, 50000, size=int(rng.integers(16, 80)))) for _ in range(3)]
    specs = []
    for i in range(n_seqs):
        if shared_prompts and rng.random() < 0.6:
            prompt = bases[int(rng.integers(0, 3))] + list(rng.integers(0, 50000, size=int(rng.integers(1, 40))))
        else:
            prompt = list(rng.integers(0, 50000, size=int(rng.integers(1, 120))))
        specs.append(dict(id=i + 1, arrival=int(rng.integers(0, n_steps // 2)),
                          cancel=int(rng.integers(1, n_steps)) if rng.random() < 0.1 else -1,
                          max_new=int(rng.integers(1, 24)),
                          max_ctx=int(rng.integers(len(prompt) + 1, len(prompt) + 40)),
                          stop=[int(x) for x in rng.integers(0, 50000, size=int(rng.integers(0, 3)))],
                          prompt=[int(x) for x in prompt]))
    return specs


@pytest.mark.parametrize("seed", range(16))
def test_trace_matches_model(seed):
    """Random arrivals, shared-prefix prompts, stops and cancellations; pools from ample to
    tight enough to preempt (and to retire a sequence that alone exceeds the pool)."""
    rng = np.random.default_rng(seed)
    n_steps = 60
    specs = _random_specs(rng, int(rng.integers(3, 24)), n_steps, shared_prompts=seed % 2 == 0)
    nb = int(rng.choice([6, 12, 24, 64, 512]))
    cfg = (nb, int(rng.integers(1, 9)), int(rng.choice([1, 7, 32, 64, 256])),
           int(rng.choice([1, 16, 48, 512])), bool(seed % 3 != 2))
    got = _cpp_trace(cfg, n_steps, specs)
    want = sm.run_trace(*cfg, n_steps, specs, selection_check=_oracle_check(cfg[2], cfg[3]))
    assert got == want, next((g, w) for g, w in zip(got, want) if g != w)


def test_preemption_known_answer():
    """Pool of 4 blocks, 2 slots, budget 64, chunk 64, no prefix cache; A = 40-token
    prompt (2 tokens to generate), B = 20-token prompt (1 token).  Derived by hand:
    step 0: order by rows to go is B, A.  B takes blocks 0, 1; A gets 2, 3 and finds the
      pool dry, so B (the youngest other running sequence) is preempted: 0, 1 go back to
      the free list and B to the front of the waiting queue.  A takes 0; the batch is
      rebuilt: A alone, 40 rows on blocks 2, 3, 0, sampling.  Free list: 1.
    step 1: B is re-admitted.  Order: A (1 row to go), B (20).  A is emitted, then B takes
      block 1 and finds the pool dry: A is preempted (2, 3, 0 freed, A waits with
      computed = 0), B takes 2, and the rebuilt batch is B alone on blocks 1, 2.  (The
      reference would keep A, already emitted, in the batch with its blocks freed.)
      B samples its one token and retires; all 4 blocks are free.
    step 2: A recomputes its 41 tokens on blocks 3, 0, 1 and finishes."""
    specs = [dict(id=1, arrival=0, cancel=-1, max_new=2, max_ctx=1000, stop=[],
                  prompt=list(range(100, 140))),
             dict(id=2, arrival=0, cancel=-1, max_new=1, max_ctx=1000, stop=[],
                  prompt=list(range(200, 220)))]
    cfg = (4, 2, 64, 64, False)
    want = ["B 0 40 1 1 0 40 3 2 3 0", "S 0 1 1", "F 0 free=1 running=1, waiting=2,",
            "B 1 20 1 2 0 20 2 1 2", "S 1 1 2", "R 1 2 1 0 21", "F 1 free=4 running= waiting=1,",
            "B 2 41 1 1 0 41 3 3 0 1", "S 2 1 1", "R 2 1 1 0 42", "F 2 free=4 running= waiting=",
            "F 3 free=4 running= waiting="]
    assert _cpp_trace(cfg, 4, specs) == want
    assert sm.run_trace(*cfg, 4, specs) == want


def test_prefix_cache_adopted():
    """A second sequence with the same 40-token prompt, arriving after the first has run,
    adopts the first two blocks (32 tokens) from the prefix cache: it starts at
    computed = 32 on the same block ids, and only its last 8 prompt rows are computed."""
    prompt = [int(x) for x in np.random.default_rng(7).integers(0, 50000, size=40)]
    specs = [dict(id=1, arrival=0, cancel=-1, max_new=1, max_ctx=1000, stop=[], prompt=prompt),
             dict(id=2, arrival=2, cancel=-1, max_new=1, max_ctx=1000, stop=[], prompt=prompt)]
    cfg = (16, 2, 64, 64, True)
    got = _cpp_trace(cfg, 4, specs)
    assert got == sm.run_trace(*cfg, 4, specs)
    b0 = next(l for l in got if l.startswith("B 0 ")).split()
    b2 = next(l for l in got if l.startswith("B 2 ")).split()
    assert b0[4:8] == ["1", "0", "40", "3"]
    assert b2[4:8] == ["2", "32", "8", "3"]          # 32 cached, 8 rows computed
    assert b2[8:10] == b0[8:10]                      # same two leading block ids


def test_hash_block_chain():
    """The block hash chain: deterministic, never 0, order- and parent-sensitive (the
    constants are the reference's; scheduler.cc:16-24)."""
    t = list(range(32))
    h1 = sm.hash_block(0, t, 0, 16)
    assert h1 == sm.hash_block(0, t, 0, 16) and h1 != 0
    assert sm.hash_block(h1, t, 16, 16) != sm.hash_block(0, t, 16, 16)
    assert sm.hash_block(0, t[::-1], 0, 16) != h1
