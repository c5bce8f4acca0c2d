"""The committed golden step (tests/golden/step_small.npz, written by
tests/golden/make_golden.py): the oracle reproduces it bit for bit, and its pack arrays
equal the hand-derived known answer for this batch."""
from __future__ import annotations

from pathlib import Path

import numpy as np

FIX = Path(__file__).resolve().parent / "golden" / "step_small.npz"


def test_golden_pack_known_answer():
    g = np.load(FIX)
    # decode at position 39: page index 2 of table [7, 2, 9] -> page 9, token 7
    # fresh prompt, 12 rows at positions 0..11 on page 4; chunk of 5 rows on a 16-token
    # cached prefix: positions 16..20, page index 1 of table [0, 5] -> page 5
    assert g["cu_seqlens"].tolist() == [0, 1, 13, 18]
    assert g["positions"].tolist() == [39] + list(range(12)) + list(range(16, 21))
    assert g["slot_mapping"].tolist() == [9 * 16 + 7] + list(range(64, 76)) + list(range(80, 85))
    assert g["meta"][:4].tolist() == [18, 1, 2, 12]  # rows, decodes, prefills, max qlen
    bt = g["block_tables"].reshape(3, -1)
    assert bt[0, :3].tolist() == [7, 2, 9] and (bt[0, 3:] == -1).all()
    assert bt[1, :2].tolist() == [4, 11] and (bt[1, 2:] == -1).all()


def test_oracle_reproduces_golden():
    from tests.golden import make_golden as mg

    g = np.load(FIX)
    e = mg.expected()
    for k in g.files:
        assert np.array_equal(g[k], e[k]), k
