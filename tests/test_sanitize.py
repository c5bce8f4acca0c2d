"""The host code of the library and its checker under AddressSanitizer +
UndefinedBehaviorSanitizer (host code only, no GPU):

* the CPU oracle (oracle/fqa_oracle.c) driven by tests/cpp/sanitize_oracle.c over random
  batches, every pack status code, the append, both attentions, selection and sampling;
* flashqwen_amd/csrc/fqa_host.cpp and include/fqa_compat.hpp (PrepareInputs, RopeTables,
  KvStore sizing, LaunchHeadNormRope's table bound, the rejections) driven by
  tests/cpp/sanitize_host.cpp over a stubbed device whose fqa_pack is the oracle's;
* the host scheduler include/fqa_sched.hpp through tests/cpp/sched_cpp.cpp on scripted
  workloads, whose traces must equal those of the plain build.

The programs are built with ROCm's clang (the HIP headers need it) into tests/cpp/san/;
any sanitizer report makes the program exit non-zero."""
from __future__ import annotations

import os
import subprocess
from pathlib import Path

import numpy as np
import pytest

from tests import test_sched as ts

ROOT = Path(__file__).resolve().parents[1]
OUT = ROOT / "tests" / "cpp" / "san"
CLANG = Path("/opt/rocm/llvm/bin/clang")
SAN = ["-O1", "-g", "-fno-omit-frame-pointer", "-fsanitize=address,undefined",
       "-fno-sanitize-recover=all"]
ENV = dict(os.environ, OMP_NUM_THREADS="2",
           ASAN_OPTIONS="detect_leaks=1:abort_on_error=0:exitcode=23",
           UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1:exitcode=24")

pytestmark = pytest.mark.skipif(not CLANG.exists(), reason="ROCm clang not present")


def _build(name: str, srcs: list[str], cxx: bool, extra: list[str] = ()) -> Path:
    OUT.mkdir(parents=True, exist_ok=True)
    exe = OUT / name
    objs = []
    for src in srcs:  # C sources as C99, the rest as C++17
        obj = OUT / (Path(src).name + ".o")
        c = src.endswith(".c")
        cmd = [str(CLANG) if c else str(CLANG) + "++", *SAN, "-fopenmp",
               "-std=c99" if c else "-std=c++17", "-D__HIP_PLATFORM_AMD__",
               "-I/opt/rocm/include", *extra, "-c", str(ROOT / src), "-o", str(obj)]
        subprocess.run(cmd, check=True, capture_output=True, text=True)
        objs.append(str(obj))
    link = [str(CLANG) + ("++" if cxx else ""), *SAN, "-fopenmp", "-o", str(exe), *objs, "-lm"]
    subprocess.run(link, check=True, capture_output=True, text=True)
    return exe


def _run(exe: Path, stdin: str | None = None) -> str:
    # the OpenMP runtime's own thread-pool allocation is not freed at exit: not ours
    supp = OUT / "lsan.supp"
    supp.write_text("leak:libomp.so\n")
    env = dict(ENV, LSAN_OPTIONS=f"suppressions={supp}")
    r = subprocess.run([str(exe)], input=stdin, capture_output=True, text=True, env=env,
                       timeout=300)
    assert r.returncode == 0, (exe.name, r.returncode, r.stderr[-4000:])
    return r.stdout


def test_oracle_under_sanitizers():
    exe = _build("sanitize_oracle", ["tests/cpp/sanitize_oracle.c", "oracle/fqa_oracle.c"],
                 cxx=False)
    out = _run(exe)
    assert out.strip().endswith("ok")
    # every status code of the pack was reached (0, 1 short table, 3 rows, 4 page range,
    # 5 negative, 6 plan capacity)
    codes = {int(l.rsplit("=", 1)[1]) for l in out.splitlines() if l.startswith("step ")}
    assert codes == {0, 1, 3, 4, 5, 6}, codes


def test_host_and_compat_under_sanitizers():
    exe = _build("sanitize_host", ["tests/cpp/sanitize_host.cpp",
                                   "flashqwen_amd/csrc/fqa_host.cpp", "oracle/fqa_oracle.c"],
                 cxx=True)
    assert _run(exe).strip() == "ok"


def test_scheduler_under_sanitizers():
    exe = _build("sched_cpp", ["tests/cpp/sched_cpp.cpp"], cxx=True)
    plain = ROOT / "tests" / "cpp" / "sched_cpp"
    if not plain.exists():
        pytest.fail(f"{plain} not built (run __graft_entry__.build())")
    for seed in range(6):
        rng = np.random.default_rng(seed)
        n_steps = 60
        specs = ts._random_specs(rng, int(rng.integers(3, 24)), n_steps,
                                 shared_prompts=seed % 2 == 0)
        nb = int(rng.choice([6, 12, 24, 64, 512]))
        cfg = (nb, int(rng.integers(1, 9)), int(rng.choice([1, 7, 32, 64, 256])),
               int(rng.choice([1, 16, 48, 512])), bool(seed % 3 != 2))
        script = ts._script(cfg, n_steps, specs)
        want = subprocess.run([str(plain)], input=script, capture_output=True, text=True,
                              check=True, timeout=60).stdout
        assert _run(exe, script) == want
