"""bench.py's contract pieces that need no GPU: more than one GPU is refused with a JSON
error line, and the committed rocprof summaries carry the per-kernel traffic that the
headline line and the prefill lines read (so a renamed or added kernel cannot leave
`roofline.traffic` silently null)."""
from __future__ import annotations

import json
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    line = json.loads(r.stdout.strip().splitlines()[-1])
    assert "one GPU" in line["error"]


def test_committed_profiles_carry_the_line_traffic():
    import bench

    # the headline decode (config 5, shared-prefix groups: split kernel + combine)
    got, src = bench._profile_traffic(5, ["decode_split_kernel", "decode_combine_kernel"])
    assert got and src == "profiles/decode_config5.txt"
    # its bytes read are below the logical bytes (each shared prefix read once per 8
    # members) and above the unique K/V bytes of the layer
    assert 4.0e9 < got < 5.2e9
    for config, kernels in ((2, ["decode_split_kernel", "decode_combine_kernel"]),
                            (3, ["prefill_kernel"]), (4, ["prefill_kernel"])):
        got, src = bench._profile_traffic(config, kernels)
        assert got and src, config
    util = bench._profile_mfma_util(3)
    assert util and 0.2 < util["mfma_busy_of_active_cycles"] < 1.0
