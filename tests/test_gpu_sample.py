"""fqa_sample on the GPU (LaunchSampleBatch, kernels.cu:184-327) against the fp64 oracle
(oracle/fqa_oracle.c, fqo_sample), through the C ABI.  Greedy rows: bit-exact.  Sampled
rows: nearly every pick must equal the oracle's exactly.  The kernel sums fp32 weights
(as the reference does), so a pick that differs is checked for what fp32 rounding cannot
change: the token is kept (weight >= the oracle's smallest kept weight, within 1e-5
relative), and its cumulative-mass interval in vocabulary order, computed in fp64,
contains the draw u * (kept mass) within 1e-4 of the kept mass."""
from __future__ import annotations

import numpy as np
import pytest

from tests import pyref

VOCAB = 151936  # Qwen3 vocabulary


def _run(lg, it, tp, u):
    import torch

    from flashqwen_amd.sample import sample

    t = lambda x: torch.from_numpy(np.ascontiguousarray(x, np.float32)).cuda()  # noqa: E731
    out = sample(t(lg), t(it), t(tp), t(u))
    torch.cuda.synchronize()
    return out.cpu().numpy()


def _check_sampled(lg, it, tp, u, got):
    from oracle import oracle as orc

    ref, thr, mass = orc.sample(lg, it, tp, u)
    exact = 0
    for b in range(lg.shape[0]):
        w = np.exp((lg[b].astype(np.float64) - lg[b].max()) * it[b])
        kept = np.where((w >= thr[b] * (1 - 1e-5)) & (w > 0), w, 0.0)
        g = int(got[b])
        assert 0 <= g < lg.shape[1]
        if g == ref[b]:
            exact += 1
            continue
        # a pick other than the oracle's: what fp32 rounding cannot change
        assert kept[g] > 0, (b, g, w[g], thr[b])
        cum = np.cumsum(kept)
        target, tol = u[b] * mass[b], 1e-4 * mass[b]
        lo = cum[g - 1] if g > 0 else 0.0
        assert lo - tol <= target <= cum[g] + tol, (b, g, int(ref[b]), lo, cum[g], target)
    return exact


@pytest.mark.gpu
def test_greedy_rows_bit_exact(gpu):
    from oracle import oracle as orc

    print("[test_greedy_rows_bit_exact] 64 rows x 151936", flush=True)
    rng = np.random.default_rng(11)
    B = 64
    lg = (rng.standard_normal((B, VOCAB)) * 4).astype(np.float32)
    # ties resolve in the reference's order (its thread tree, not the smallest index)
    lg[3, [5, 90000]] = 50.0          # threads 5 and 144: 90000 wins
    lg[9, [100, 300, 70001]] = 50.0   # threads 100, 44, 113
    lg[13, [512, 256, 1024]] = 50.0   # one thread: its first column, 256
    lg[7, :] = -np.inf                # all -inf: token 0
    lg[11, :] = -2e30                 # nothing above the kernel's -1e30 start: token 0
    lg[11, 77] = -1.5e30
    it = np.zeros(B, np.float32)
    got = _run(lg, it, np.ones(B, np.float32), rng.random(B).astype(np.float32))
    ref = orc.sample(lg, it, np.ones(B, np.float32), np.zeros(B, np.float32))[0]
    assert np.array_equal(got, ref)
    for r in (3, 9, 13):
        assert got[r] == pyref.argmax_kernel(lg[r]), r
    assert got[3] == 90000 and got[13] == 256 and got[7] == 0 and got[11] == 0


@pytest.mark.gpu
@pytest.mark.parametrize("vocab", [VOCAB, 1001, 64, 1])
def test_sampled_rows(gpu, vocab):
    print(f"[test_sampled_rows] vocab {vocab}", flush=True)
    rng = np.random.default_rng(12 + vocab)
    B = 96
    scale = rng.choice([0.5, 2.0, 6.0], size=B)
    lg = (rng.standard_normal((B, vocab)) * scale[:, None]).astype(np.float32)
    it = rng.choice([0.5, 1.0, 1.7], size=B).astype(np.float32)
    tp = rng.choice([1.0, 0.95, 0.8, 0.5, 0.1, 0.0], size=B).astype(np.float32)
    u = rng.random(B).astype(np.float32)
    u[:4] = [0.0, 0.5, 0.999999, 0.25]
    if vocab >= 64:  # masked tokens (-inf logits) weigh 0 and are never picked
        mask = rng.random((12, vocab)) < 0.3
        mask[:, 0] = False
        lg[4:16][mask] = -np.inf
    got = _run(lg, it, tp, u)
    exact = _check_sampled(lg, it, tp, u, got)
    print(f"vocab {vocab}: {exact}/{B} picks equal the fp64 oracle's")
    assert exact >= B - 3


@pytest.mark.gpu
def test_sampled_closed_forms(gpu):
    """Uniform logits, top_p = 1: token ceil(u*N) - 1 (up to one token of fp32 rounding);
    top_p = 0 keeps only the largest weight: the argmax."""
    rng = np.random.default_rng(13)
    B = 32
    u = rng.random(B).astype(np.float32)
    lg = np.full((B, VOCAB), 1.25, np.float32)
    got = _run(lg, np.ones(B, np.float32), np.ones(B, np.float32), u)
    want = np.ceil(u.astype(np.float64) * VOCAB).astype(np.int64) - 1
    assert np.all(np.abs(got - want) <= 1), (got, want)
    lg = rng.standard_normal((B, VOCAB)).astype(np.float32)
    got = _run(lg, np.full(B, 0.8, np.float32), np.zeros(B, np.float32), u)
    assert np.array_equal(got, lg.argmax(axis=1))


@pytest.mark.gpu
def test_top_p_boundary_bin_copied_or_reread(gpu):
    """Top-p rows whose boundary weight bin (weight bits 30..20) holds a few hundred weights
    (resolved from the LDS copy) and rows where it holds most of the vocabulary (more than
    the 16384 the copy holds: the row is read again).  Both against the fp64 oracle, and
    every run gives the same tokens (the histogram masses are exact integer sums)."""
    from oracle import oracle as orc

    print("[test_top_p_boundary_bin_copied_or_reread] 64 rows x 151936", flush=True)
    rng = np.random.default_rng(21)
    B = 64
    scale = np.where(np.arange(B) % 2 == 0, 4.0, 0.01)  # odd rows: nearly flat weights
    lg = (rng.standard_normal((B, VOCAB)) * scale[:, None]).astype(np.float32)
    it = np.ones(B, np.float32)
    tp = rng.choice([0.95, 0.8, 0.5], size=B).astype(np.float32)
    u = rng.random(B).astype(np.float32)
    _, thr, _ = orc.sample(lg, it, tp, u)
    w = np.exp((lg - lg.max(axis=1, keepdims=True)) * it[:, None]).astype(np.float32)
    tbin = (np.asarray(thr, np.float32).view(np.uint32) >> 20)[:, None]
    in_bin = ((w.view(np.uint32) >> 20) == tbin).sum(axis=1)
    assert (in_bin[0::2] < 16384).all() and (in_bin[1::2] > 16384).all(), in_bin
    got = _run(lg, it, tp, u)
    exact = _check_sampled(lg, it, tp, u, got)
    print(f"{exact}/{B} picks equal the fp64 oracle's; boundary bin sizes "
          f"{int(in_bin[0::2].max())} (copied) / {int(in_bin[1::2].min())} (re-read)")
    assert exact >= B - 3
    for _ in range(2):
        assert np.array_equal(_run(lg, it, tp, u), got)


@pytest.mark.gpu
def test_top_p_ties_and_extremes(gpu):
    """Logits on a coarse grid (many exactly equal weights, so whole runs of ties sit at
    the threshold and the boundary bin overflows the LDS copy on some rows), top_p near 1
    and near 0, and a vocabulary just above twice the copy's capacity."""
    print("[test_top_p_ties_and_extremes] 48 rows", flush=True)
    rng = np.random.default_rng(33)
    for vocab in (VOCAB, 2 * 16384 + 1):
        B = 24
        lg = (np.round(rng.standard_normal((B, vocab)) * 4) / 4).astype(np.float32)
        lg[:8] = np.round(lg[:8])  # integer logits: very large tie runs
        it = rng.choice([0.5, 1.0, 3.0], size=B).astype(np.float32)
        tp = np.array([0.999999, 1e-6, 0.5, 0.9, 0.75, 0.3] * 4, np.float32)
        u = rng.random(B).astype(np.float32)
        got = _run(lg, it, tp, u)
        exact = _check_sampled(lg, it, tp, u, got)
        print(f"vocab {vocab}: {exact}/{B} picks equal the fp64 oracle's")
        assert exact >= B - 2
