"""Build libfqa.so (the gfx950 HIP library behind include/fqa.h) in-tree with hipcc.

Every source is compiled for gfx950 only, with packed-fp32 instruction selection
switched off, then linked into one shared library next to this file.
"""
from __future__ import annotations

import os
import subprocess
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
LIB = PKG / "libfqa.so"
OBJ = PKG / "_build"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    # NaN semantics off (infinities kept): fmaxf on MFMA results then needs no
    # canonicalising v_max x,x, and the kernels never test for NaN
    "-fno-honor-nans",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _run(cmd: list[str]) -> None:
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in r.stderr.splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError(f"build failed: {' '.join(cmd)}\n{err}")
    if err.strip():
        print(err)


def build(verbose: bool = False) -> Path:
    OBJ.mkdir(exist_ok=True)
    srcs = sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cpp"))
    objs = [OBJ / (s.name + ".o") for s in srcs]
    cmds = [[HIPCC, *FLAGS, "-c", str(s), "-o", str(o)] for s, o in zip(srcs, objs)]
    with ThreadPoolExecutor(max_workers=min(8, len(cmds))) as ex:
        list(ex.map(_run, cmds))
    tmp = LIB.with_suffix(".so.tmp")
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-o", str(tmp), *map(str, objs)])
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


def build_cpp_driver() -> Path:
    """tests/cpp/step_cpp: a C++ program driving the path through include/fqa_step.hpp."""
    root = PKG.parent
    src = root / "tests" / "cpp" / "step_cpp.cpp"
    exe = src.with_suffix("")
    _run([HIPCC, "-O2", "-std=c++17", "-o", str(exe), str(src), f"-L{PKG}", "-lfqa",
          "-Wl,-rpath,$ORIGIN/../../flashqwen_amd"])
    return exe


def build_serve_driver() -> Path:
    """tests/cpp/serve_cpp: host scheduler + C++ step mirror serving loop on the GPU."""
    root = PKG.parent
    src = root / "tests" / "cpp" / "serve_cpp.cpp"
    exe = src.with_suffix("")
    _run([HIPCC, "-O2", "-std=c++17", "-o", str(exe), str(src), f"-L{PKG}", "-lfqa",
          "-Wl,-rpath,$ORIGIN/../../flashqwen_amd"])
    return exe


def build_graph_driver() -> Path:
    """tests/cpp/graph_cpp: eager vs captured-graph steps through include/fqa_step.hpp."""
    root = PKG.parent
    src = root / "tests" / "cpp" / "graph_cpp.cpp"
    exe = src.with_suffix("")
    _run([HIPCC, "-O2", "-std=c++17", "-o", str(exe), str(src), f"-L{PKG}", "-lfqa",
          "-Wl,-rpath,$ORIGIN/../../flashqwen_amd"])
    return exe


def build_decode_loop_driver() -> Path:
    """tests/cpp/decode_loop_cpp: the serving loop with projections, lm_head and sampling
    on the GPU (tokens produced on the device)."""
    root = PKG.parent
    src = root / "tests" / "cpp" / "decode_loop_cpp.cpp"
    exe = src.with_suffix("")
    _run([HIPCC, "-O2", "-std=c++17", "-o", str(exe), str(src), f"-L{PKG}", "-lfqa",
          "-Wl,-rpath,$ORIGIN/../../flashqwen_amd"])
    return exe


def build_compat_driver() -> Path:
    """tests/cpp/compat_cpp: the reference's RunLayersBody attention calls, compiled against
    include/fqa_compat.hpp (the reference's Launch* signatures)."""
    root = PKG.parent
    src = root / "tests" / "cpp" / "compat_cpp.cpp"
    exe = src.with_suffix("")
    _run([HIPCC, "-O2", "-std=c++17", "-Wall", "-o", str(exe), str(src), f"-L{PKG}", "-lfqa",
          "-Wl,-rpath,$ORIGIN/../../flashqwen_amd"])
    return exe


def build_sched_driver() -> Path:
    """tests/cpp/sched_cpp: a host program driving include/fqa_sched.hpp (no HIP)."""
    root = PKG.parent
    src = root / "tests" / "cpp" / "sched_cpp.cpp"
    exe = src.with_suffix("")
    _run(["g++", "-O2", "-std=c++17", "-Wall", "-Wextra", "-o", str(exe), str(src)])
    return exe


if __name__ == "__main__":
    build(verbose=True)
