"""A serving loop in C++ (tests/cpp/serve_cpp): the host scheduler (include/fqa_sched.hpp)
builds every step's batch from live request state and the attention path runs it on the
GPU through the C++ step mirror (include/fqa_step.hpp), over one KV pool that persists
across steps.  Each step is replayed through the CPU oracle chain on the oracle's own
copy of the pool: pack counts equal, attention outputs within tolerance, at every step."""
from __future__ import annotations

import subprocess
from pathlib import Path

import numpy as np
import pytest

from flashqwen_amd import synth
from tests import sched_model as sm
from tests import stepcase as sc
from tests.test_sched import _script

EXE = Path(__file__).resolve().parent / "cpp" / "serve_cpp"


def _read_steps(path: Path):
    raw = np.fromfile(path, np.uint8)
    o, steps = 0, []

    def take(dtype, n):
        nonlocal o
        a = raw[o:o + n * np.dtype(dtype).itemsize].view(dtype)
        o += n * np.dtype(dtype).itemsize
        return a

    while o < raw.size:
        t, R, T = take(np.int32, 3)
        computed, n_new = take(np.int32, R), take(np.int32, R)
        off = take(np.int32, R + 1)
        pages = take(np.int32, int(off[-1]))
        qkv = take(np.uint16, T * synth.QKV_STRIDE).reshape(T, -1)
        attn = take(np.uint16, T * 4096).reshape(T, -1)
        meta = take(np.int32, 16)
        steps.append(dict(t=int(t), computed=computed, n_new=n_new, off=off, pages=pages,
                          qkv=qkv, attn=attn, meta=meta))
    return steps


def _serve_case(tmp_path, seed, n_seqs, n_blocks, slots, budget, chunk, steps, cancel_id):
    if not EXE.exists():
        pytest.fail(f"{EXE} not built (run __graft_entry__.build())")
    rng = np.random.default_rng(seed)
    base = [int(x) for x in rng.integers(0, 50000, size=70)]
    specs = []
    for i in range(n_seqs):  # shared 70-token prompt heads: later arrivals adopt cached blocks
        tail = [int(x) for x in rng.integers(0, 50000, size=int(rng.integers(1, 60)))]
        prompt = (base + tail) if i % 2 == 0 else tail + base[:20]
        specs.append(dict(id=i + 1, arrival=int(i // 2) * 2,
                          cancel=9 if i + 1 == cancel_id else -1,
                          max_new=int(rng.integers(2, 9)), max_ctx=512, stop=[],
                          prompt=prompt))
    script = _script((n_blocks, slots, budget, chunk, True), steps, specs) + "512\n"
    (tmp_path / "s.txt").write_text(script)
    wq, wk = synth.norm_weights()
    np.concatenate([wq.astype(np.float32), wk.astype(np.float32)]).tofile(tmp_path / "w.bin")
    print(f"[test_serving_loop_matches_oracle] {len(specs)} seqs, {steps} steps, pool "
          f"{n_blocks} pages", flush=True)
    subprocess.run([str(EXE), str(tmp_path / "s.txt"), str(tmp_path / "w.bin"),
                    str(tmp_path / "out.bin")], check=True, timeout=120)
    got = _read_steps(tmp_path / "out.bin")
    assert len(got) >= 8

    pool = np.zeros(sc.pool_elems(n_blocks), np.uint16)
    saw_prefill = saw_decode = saw_cached = False
    for st in got:
        tables = [st["pages"][st["off"][r]:st["off"][r + 1]] for r in range(len(st["n_new"]))]
        cfg = synth._assemble(f"step{st['t']}", st["computed"], st["n_new"], tables, n_blocks, 512)
        kw = sc.pack_kwargs(cfg, max_rows=budget, dec_grid_waves=int(st["meta"][4]) or 1,
                            dec_min_pages=8, max_reqs=slots)
        ref = sc.oracle_chain(cfg, st["qkv"], pool, wq, wk, kw)
        assert st["meta"][:4].tolist() == ref["pack"]["meta"][:4].tolist(), st["t"]
        assert st["meta"][7] == 0
        mx, mean = sc.att_errors(st["attn"], ref["out"])
        print(f"step {st['t']}: R={len(st['n_new'])} T={cfg.rows} max-abs {mx:.3e} mean-abs {mean:.3e}")
        assert mx <= sc.ATT_MAX_ABS and mean <= sc.ATT_MEAN_ABS, (st["t"], mx, mean)
        pool = ref["pool"]
        saw_prefill |= bool((st["n_new"] > 1).any())
        saw_decode |= bool((st["n_new"] == 1).any())
        saw_cached |= bool(((st["n_new"] > 1) & (st["computed"] > 0)).any())  # on cached keys
    assert saw_prefill and saw_decode and saw_cached

    # the batches are the scheduler model's decisions, and the workload preempts
    preempts = []

    class Counting(sm.Scheduler):
        def _grow(self, s, upto):
            ok, p = super()._grow(s, upto)
            preempts.append(p)
            return ok, p

    model_batches = []
    a = sm.Allocator(n_blocks)
    sch = Counting(a, slots, budget, chunk, True)
    live = {}
    for t in range(steps):
        for sp in specs:
            if sp["arrival"] == t:
                q = sm.Seq(sp["id"], sp["prompt"], sp["max_new"], sp["max_ctx"], sp["stop"])
                live[q.id] = q
                sch.waiting.append(q)
            if sp["cancel"] == t and sp["id"] in live:
                live[sp["id"]].cancelled = True
        sch.refill()
        batch = sch.build()
        if batch:
            model_batches.append((t, [c for _, c, _, _ in batch], [n for _, _, n, _ in batch]))
            smp = [q for q, c, n, _ in batch if c + n == len(q.tokens)]
            sch.apply(batch, {q.id: sm.sampled_token(q.id, t) for q in smp})
        sch.retired = []
    assert [(st["t"], st["computed"].tolist(), st["n_new"].tolist()) for st in got] == model_batches
    assert any(preempts)


@pytest.mark.gpu
def test_serving_loop_matches_oracle(gpu, tmp_path):
    """10 sequences over 16 steps on a 20-page pool (3 preemptions)."""
    _serve_case(tmp_path, 77, 10, 20, 6, 96, 48, 16, cancel_id=8)


@pytest.mark.gpu
def test_serving_loop_longer(gpu, tmp_path):
    """24 sequences over 40 steps: more slots, a larger budget and chunk, a 26-page pool
    (10 preemptions in the scheduler model; all 24 sequences retire)."""
    _serve_case(tmp_path, 78, 24, 26, 8, 128, 64, 40, cancel_id=5)
