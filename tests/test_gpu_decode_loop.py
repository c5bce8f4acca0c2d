"""The serving loop with tokens produced on the GPU (tests/cpp/decode_loop_cpp): host
scheduler -> pack -> per layer fqa_qkv_proj_append, attention, o_proj (fqa_gemm) ->
lm_head (fqa_gemm, fp32) -> fqa_sample for the sampled rows, fqa_gemm_argmax (lm_head
fused with the greedy pick) for the greedy ones -> Apply.  Checks: every greedy token is the
argmax of the float64 logits of the hidden row lm_head read (or, within fp32 rounding of
a tie, one of the two largest); every sampled token passes the sampler's own checks
against the fp64 oracle (tests/test_gpu_sample.py); two runs produce the same bytes."""
from __future__ import annotations

import subprocess
from pathlib import Path

import numpy as np
import pytest

from tests.test_sched import _script

EXE = Path(__file__).resolve().parent / "cpp" / "decode_loop_cpp"
VOCAB, HIDDEN, LAYERS = 4096, 512, 2


def _run(tmp: Path, script: str):
    tmp.mkdir(parents=True, exist_ok=True)
    (tmp / "s.txt").write_text(script)
    r = subprocess.run([str(EXE), str(tmp / "s.txt"), str(VOCAB), str(HIDDEN), str(LAYERS),
                        str(tmp)], capture_output=True, text=True, timeout=180)
    assert r.returncode == 0, r.stderr
    return (tmp / "steps.bin").read_bytes()


def _parse(raw: bytes):
    a = np.frombuffer(raw, np.uint8)
    o, steps = 0, []
    while o < a.size:
        t, n = np.frombuffer(a[o:o + 8].tobytes(), np.int32)
        o += 8
        rec = np.frombuffer(a[o:o + 20 * n].tobytes(), dtype=[("id", "<i4"), ("it", "<f4"),
                                                              ("tp", "<f4"), ("u", "<f4"),
                                                              ("tok", "<i4")])
        o += 20 * n
        hs = np.frombuffer(a[o:o + 2 * n * HIDDEN].tobytes(), np.uint16).reshape(n, HIDDEN)
        o += 2 * n * HIDDEN
        steps.append((int(t), rec, hs))
    return steps


def _f32(bits: np.ndarray) -> np.ndarray:
    return (bits.astype(np.uint32) << 16).view(np.float32)


@pytest.mark.gpu
def test_tokens_sampled_on_device(gpu, tmp_path):
    from tests.test_gpu_sample import _check_sampled

    if not EXE.exists():
        pytest.fail(f"{EXE} not built (run __graft_entry__.build())")
    rng = np.random.default_rng(31)
    specs = []
    for i in range(8):
        prompt = [int(x) for x in rng.integers(0, 50000, size=int(rng.integers(5, 90)))]
        specs.append(dict(id=i + 1, arrival=i // 3, cancel=-1, max_new=int(rng.integers(3, 7)),
                          max_ctx=256, stop=[], prompt=prompt))
    script = _script((64, 6, 96, 48, True), 14, specs) + "256\n"
    raw = _run(tmp_path / "a", script)
    assert raw == _run(tmp_path / "b", script)  # deterministic end to end
    w_lm = _f32(np.fromfile(tmp_path / "a" / "w_lm.bin", np.uint16)).reshape(VOCAB, HIDDEN)
    steps = _parse(raw)
    n_greedy = n_sampled = 0
    for t, rec, hs in steps:
        logits = _f32(hs).astype(np.float64) @ w_lm.astype(np.float64).T
        assert np.all((rec["tok"] >= 0) & (rec["tok"] < VOCAB))
        g = rec["it"] <= 0
        for i in np.nonzero(g)[0]:
            top2 = np.argsort(logits[i])[-2:]
            gap = logits[i][top2[1]] - logits[i][top2[0]]
            ok = rec["tok"][i] == top2[1] or (gap < 1e-4 * abs(logits[i][top2[1]]) and
                                              rec["tok"][i] == top2[0])
            assert ok, (t, int(rec["id"][i]), int(rec["tok"][i]), int(top2[1]), gap)
            n_greedy += 1
        s = np.nonzero(~g)[0]
        if s.size:
            lg = logits[s].astype(np.float32)
            got = rec["tok"][s]
            _check_sampled(lg, rec["it"][s].copy(), rec["tp"][s].copy(), rec["u"][s].copy(), got)
            n_sampled += s.size
    print(f"{len(steps)} steps with samples: {n_greedy} greedy, {n_sampled} sampled tokens")
    assert n_greedy >= 8 and n_sampled >= 8
