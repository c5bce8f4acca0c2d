"""The C ABI without a GPU: libfqa.so loads, exports every function include/fqa.h declares,
its host-side helpers are exact, and rejected calls return error codes before any launch."""
from __future__ import annotations

import ctypes as C
import re
from pathlib import Path

import numpy as np
import pytest

from flashqwen_amd import _lib
from flashqwen_amd.step import make_dims

HEADER = Path(__file__).resolve().parents[1] / "include" / "fqa.h"


def declared_functions() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(fqa_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    names = declared_functions()
    assert len(names) >= 12
    for n in names:
        assert hasattr(lib, n), n
    assert set(names) == set(_lib.SIGNATURES), "ctypes table and header disagree"
    assert lib.fqa_version().startswith(b"fqa")


def test_rope_tables_bit_identical_to_oracle():
    from oracle import oracle as orc

    lib = _lib.load()
    for max_pos in (1, 17, 4096):
        cos = np.empty((max_pos, 64), np.float32)
        sin = np.empty_like(cos)
        assert lib.fqa_rope_tables(max_pos, 128, 1e6, cos.ctypes.data, sin.ctypes.data) == 0
        oc, os_ = orc.rope_tables(max_pos)
        assert np.array_equal(cos.view(np.uint32), oc.view(np.uint32))
        assert np.array_equal(sin.view(np.uint32), os_.view(np.uint32))


def test_sizes_and_bounds():
    lib = _lib.load()
    d = make_dims()
    assert lib.fqa_pool_bytes(C.byref(d), 12500) == 12500 * 64 * 1024
    assert lib.fqa_pool_bytes(C.byref(d), 84771) == 84771 * 65536  # > 2^31 elements ok
    assert lib.fqa_dec_wave_bound(64, 2048) == 2048
    assert lib.fqa_pre_item_bound(16, 8192, 32) == 8192 // 32 + 16
    assert lib.fqa_decode_workspace_bytes(C.byref(d), 2048) == 2 * 2048 * 4 * 130 * 4


def test_rejected_calls_return_codes_without_launching():
    lib = _lib.load()
    d = make_dims()
    bad = make_dims()
    bad.head_dim = 64
    null = None
    # pack: null structs, too many requests, bad tile, zero grid waves
    assert lib.fqa_pack(null, null, null, null) == _lib.FQA_EINVAL
    b = _lib.FqaBatch(null, null, null, null, null, _lib.FQA_MAX_REQS + 1)
    cfg = _lib.FqaPackCfg(8, 8, 8, 16, 1, 16, 32, 8)
    out = _lib.FqaPackOut()
    assert lib.fqa_pack(C.byref(b), C.byref(cfg), C.byref(out), null) == _lib.FQA_EINVAL
    b.n_reqs = 1
    cfg.pre_tile_q = 48
    assert lib.fqa_pack(C.byref(b), C.byref(cfg), C.byref(out), null) == _lib.FQA_EINVAL
    cfg.pre_tile_q = 32
    cfg.dec_grid_waves = 0
    assert lib.fqa_pack(C.byref(b), C.byref(cfg), C.byref(out), null) == _lib.FQA_EINVAL
    # shapes other than Qwen3-8B's are refused
    assert lib.fqa_decode(C.byref(bad), null, null, 1, null, 1, null, null, null, 4, 4, null,
                          null, null) == _lib.FQA_EUNSUPPORTED
    assert lib.fqa_prefill(C.byref(bad), null, null, 1, null, 1, null, null, null, null, 32, 1,
                           null, null) == _lib.FQA_EUNSUPPORTED
    assert lib.fqa_qknorm_rope_append(C.byref(bad), *([null] * 5 + [1] + [null] * 3 + [1, null, 1,
                                                        0, null])) == _lib.FQA_EUNSUPPORTED
    # unsupported prefill tile; null pointers with work to do
    assert lib.fqa_prefill(C.byref(d), null, null, 1, null, 1, null, null, null, null, 128, 1, null,
                           null) == _lib.FQA_EUNSUPPORTED
    assert lib.fqa_decode(C.byref(d), null, null, 1, null, 1, null, null, null, 4, 4, null, null,
                          null) == _lib.FQA_EINVAL
    assert lib.fqa_schedule(null, null, _lib.FQA_MAX_REQS + 1, 1, 1, null, null, null,
                            null) == _lib.FQA_EINVAL
    assert lib.fqa_schedule(null, null, 4, 1, 0, null, null, null, null) == _lib.FQA_EINVAL
    # the fused selection + gather: the same bounds, and every pointer its work needs
    i32 = (C.c_int32 * 8)()
    assert lib.fqa_schedule_gather(null, null, _lib.FQA_MAX_REQS + 1, 1, 1, i32, i32, i32, i32,
                                   i32, i32, i32, i32, i32, 8, null) == _lib.FQA_EINVAL
    assert lib.fqa_schedule_gather(i32, i32, 4, 1, 0, i32, i32, i32, i32, i32, i32, i32, i32,
                                   i32, 8, null) == _lib.FQA_EINVAL
    assert lib.fqa_schedule_gather(i32, i32, 4, 1, 1, i32, null, i32, i32, i32, i32, i32, i32,
                                   i32, 8, null) == _lib.FQA_EINVAL
    assert lib.fqa_schedule_gather(null, i32, 4, 1, 1, i32, i32, i32, i32, i32, i32, i32, i32,
                                   i32, 8, null) == _lib.FQA_EINVAL
    assert lib.fqa_rope_tables(4, 127, 1e6, null, null) == _lib.FQA_EINVAL


@pytest.mark.parametrize("name", ["fqa_pack", "fqa_decode", "fqa_prefill",
                                  "fqa_qknorm_rope_append", "fqa_schedule"])
def test_zero_work_is_ok(name):
    """Zero-size calls are no-ops that succeed (the reference's launchers return early on
    R <= 0 / n_decode <= 0, attn_cute.cu:155,247)."""
    lib = _lib.load()
    d = make_dims()
    meta = (C.c_int32 * 16)()
    if name == "fqa_decode":
        rc = lib.fqa_decode(C.byref(d), None, None, 1, None, 1, None, None, meta, 0, 0, None,
                            None, None)
    elif name == "fqa_prefill":
        rc = lib.fqa_prefill(C.byref(d), None, None, 1, None, 1, None, None, None, meta, 32, 0,
                             None, None)
    elif name == "fqa_qknorm_rope_append":
        rc = lib.fqa_qknorm_rope_append(C.byref(d), None, None, None, None, None, 8, None, None,
                                        meta, 0, None, 1, 0, None)
    else:
        pytest.skip("launches a kernel even for empty input (covered on the GPU)")
    assert rc == _lib.FQA_OK


def test_gemm_rejections_without_gpu():
    """fqa_gemm rejects unsupported shapes and bad arguments before any launch, and sizes
    its split-K workspace."""
    from flashqwen_amd import _lib

    lib = _lib.load()
    assert lib.fqa_gemm(None, 64, None, 64, None, 128, 4, 100, 64, 0, None, 0, None) == _lib.FQA_EUNSUPPORTED
    assert lib.fqa_gemm(None, 64, None, 64, None, 128, 4, 128, 60, 0, None, 0, None) == _lib.FQA_EUNSUPPORTED
    assert lib.fqa_gemm(None, 64, None, 64, None, 128, -1, 128, 64, 0, None, 0, None) == _lib.FQA_EINVAL
    assert lib.fqa_gemm(None, 64, None, 64, None, 128, 0, 128, 64, 0, None, 0, None) == _lib.FQA_OK
    assert lib.fqa_gemm(None, 64, None, 64, None, 128, 4, 128, 64, 0, None, 0, None) == _lib.FQA_EINVAL
    # 48 tiles of QKV at M=256: K split 5 ways (240 workgroups), fp32 partials
    assert lib.fqa_gemm_workspace_bytes(256, 6144, 4096) == 5 * 256 * 6144 * 4
    assert lib.fqa_gemm_workspace_bytes(8192, 6144, 4096) == 0
    assert lib.fqa_gemm_workspace_bytes(1, 128, 64) == 0  # one k step cannot be split


def test_sample_and_fused_qkv_rejections_without_gpu():
    """fqa_sample and fqa_qkv_proj_append refuse bad arguments before any launch; empty
    calls succeed."""
    lib = _lib.load()
    null = None
    # sample: vocab out of range, stride below vocab, null pointers with rows; 0 rows ok
    assert lib.fqa_sample(null, 4, 0, 8, null, null, null, null, null) == _lib.FQA_EINVAL
    assert lib.fqa_sample(null, 4, (1 << 24) + 1, 1 << 25, null, null, null, null,
                          null) == _lib.FQA_EINVAL
    assert lib.fqa_sample(null, 4, 16, 8, null, null, null, null, null) == _lib.FQA_EINVAL
    assert lib.fqa_sample(null, 4, 16, 16, null, null, null, null, null) == _lib.FQA_EINVAL
    assert lib.fqa_sample(null, 0, 16, 16, null, null, null, null, null) == _lib.FQA_OK
    # fused QKV: other shapes, null meta, null pointers with rows; 0 rows ok
    d = make_dims()
    bad = make_dims()
    bad.n_kv_heads = 4
    meta = (C.c_int32 * 16)()
    args = lambda dims, rows, meta_: (C.byref(dims), null, 64, null, 64, rows, 64, null, null,  # noqa: E731
                                      null, null, null, 8, null, null, meta_, null, 1, 0, null,
                                      0, null)
    assert lib.fqa_qkv_proj_append(*args(bad, 4, meta)) == _lib.FQA_EUNSUPPORTED
    assert lib.fqa_qkv_proj_append(*args(d, 4, None)) == _lib.FQA_EINVAL
    assert lib.fqa_qkv_proj_append(*args(d, 4, meta)) == _lib.FQA_EINVAL
    assert lib.fqa_qkv_proj_append(*args(d, -1, meta)) == _lib.FQA_EINVAL
    assert lib.fqa_qkv_proj_append(*args(d, 0, meta)) == _lib.FQA_OK


def test_header_is_plain_c(tmp_path):
    """include/fqa.h is the C ABI: it compiles as C99 with -Wall -Wextra -pedantic, and a C
    program calling it links against libfqa.so."""
    import shutil
    import subprocess
    from pathlib import Path

    if shutil.which("gcc") is None:
        pytest.skip("no gcc")
    root = Path(__file__).resolve().parents[1]
    src = tmp_path / "c_abi.c"
    src.write_text('#include "fqa.h"\n'
                   "int main(void) {\n"
                   "  return fqa_gemm_workspace_bytes(256, 6144, 4096) > 0 && fqa_version() ? 0 : 1;\n"
                   "}\n")
    exe = tmp_path / "c_abi"
    r = subprocess.run(["gcc", "-std=c99", "-Wall", "-Wextra", "-pedantic", "-Werror",
                        f"-I{root / 'include'}", str(src), "-o", str(exe),
                        f"-L{root / 'flashqwen_amd'}", "-lfqa",
                        f"-Wl,-rpath,{root / 'flashqwen_amd'}"], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    assert subprocess.run([str(exe)]).returncode == 0


def test_gemm_argmax_rejections_without_gpu():
    from flashqwen_amd import _lib

    lib = _lib.load()
    assert lib.fqa_gemm_argmax(None, 64, None, 64, 4, 100, 64, None, None, 0, None) == _lib.FQA_EUNSUPPORTED
    assert lib.fqa_gemm_argmax(None, 64, None, 64, 4, 128, 64, None, None, 0, None) == _lib.FQA_EINVAL
    assert lib.fqa_gemm_argmax(None, 64, None, 64, 0, 128, 64, None, None, 0, None) == _lib.FQA_OK
    # lm_head at 256 rows: 1187 tiles of 256 x 128, one (max, column) pair per tile and row
    assert lib.fqa_gemm_argmax_workspace_bytes(256, 151936, 4096) == 1187 * 256 * 8
