"""ctypes binding of libfqa.so (include/fqa.h).

The library is the product: every compute call of this package goes through it.  If
the shared library is missing the import fails loudly; there is no Python fallback.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libfqa.so"

FQA_OK = 0
FQA_EINVAL = -1
FQA_EUNSUPPORTED = -2
FQA_ELAUNCH = -3
FQA_ENOSPACE = -4
FQA_PAGE_TOKENS = 16
FQA_MAX_REQS = 2048
FQA_DECODE_NOALLOC_MAX_WAVES = 4096
FQA_PRE_TILE_Q = 64  # prefill rows per work item the step helpers plan with (fqa.h)

META_ROWS, META_N_DECODE, META_N_PREFILL, META_MAX_QLEN = 0, 1, 2, 3
META_DEC_WAVES, META_PRE_ITEMS, META_DEC_WAVE_PAGES, META_STATUS = 4, 5, 6, 7
META_REQS, META_DEC_PAGES = 8, 9
META_DEC_PRE_ITEMS, META_DEC_GROUPS = 10, 11
META_LEN = 16

PACK_OK, PACK_SHORT_TABLE, PACK_WIDE_TABLE, PACK_ROWS = 0, 1, 2, 3
PACK_PAGE_RANGE, PACK_NEGATIVE, PACK_ITEMS = 4, 5, 6

P = C.c_void_p
I32 = C.c_int32
I64 = C.c_int64


class FqaDims(C.Structure):
    _fields_ = [
        ("n_q_heads", I32),
        ("n_kv_heads", I32),
        ("head_dim", I32),
        ("page_size", I32),
        ("qkv_stride", I32),
        ("eps", C.c_float),
        ("scale", C.c_float),
    ]


class FqaBatch(C.Structure):
    _fields_ = [
        ("computed", P),
        ("n_new", P),
        ("bt_off", P),
        ("bt_pages", P),
        ("n_reqs_dev", P),
        ("n_reqs", I32),
    ]


class FqaPackOut(C.Structure):
    _fields_ = [
        ("cu_seqlens", P),
        ("qlen", P),
        ("positions", P),
        ("row_req", P),
        ("slot_mapping", P),
        ("block_tables", P),
        ("decode_rids", P),
        ("prefill_rids", P),
        ("dec_seqs", P),
        ("dec_waves", P),
        ("pre_items", P),
        ("meta", P),
        ("dec_prefix", P),
        ("dec_pre_items", P),
    ]


class FqaPackCfg(C.Structure):
    _fields_ = [
        ("max_rows", I32),
        ("max_blocks", I32),
        ("pool_pages", I64),
        ("dec_grid_waves", I32),
        ("dec_min_pages", I32),
        ("dec_wave_cap", I32),
        ("pre_tile_q", I32),
        ("pre_item_cap", I32),
        ("dec_share", I32),
        ("dec_prefix_pages", I32),
        ("dec_pre_cap", I32),
    ]


# name -> (restype, argtypes); exactly the declarations of include/fqa.h
SIGNATURES = {
    "fqa_rope_tables": (C.c_int, [I32, I32, C.c_float, P, P]),
    "fqa_pool_bytes": (I64, [C.POINTER(FqaDims), I64]),
    "fqa_pool_pages": (C.c_int, [C.POINTER(FqaDims), C.c_uint64, C.c_uint64, C.c_float, I32, I32,
                                 C.POINTER(I64)]),
    "fqa_pool_pages_device": (C.c_int, [C.POINTER(FqaDims), C.c_float, I32, I32, C.POINTER(I64)]),
    "fqa_dec_wave_bound": (I32, [I32, I32]),
    "fqa_dec_default_waves": (I32, [I32]),
    "fqa_pre_item_bound": (I32, [I32, I32, I32]),
    "fqa_decode_workspace_bytes": (I64, [C.POINTER(FqaDims), I32]),
    "fqa_schedule": (C.c_int, [P, P, I32, I32, I32, P, P, P, P]),
    "fqa_gather_batch": (C.c_int, [P, P, P, I32, P, P, P, P, P, P, P, I32, P]),
    "fqa_schedule_gather": (C.c_int, [P, P, I32, I32, I32, P, P, P, P, P, P, P, P, P, I32, P]),
    "fqa_pack": (C.c_int, [C.POINTER(FqaBatch), C.POINTER(FqaPackCfg), C.POINTER(FqaPackOut), P]),
    "fqa_qknorm_rope_append": (
        C.c_int,
        [C.POINTER(FqaDims), P, P, P, P, P, I32, P, P, P, I32, P, I64, I32, P],
    ),
    "fqa_qknorm_rope": (C.c_int, [C.POINTER(FqaDims), P, P, P, P, P, I32, P, P, I32, P]),
    "fqa_store_kv": (C.c_int, [C.POINTER(FqaDims), P, P, P, P, I32, P, I64, P]),
    "fqa_decode": (
        C.c_int,
        [C.POINTER(FqaDims), P, P, I64, P, I32, P, P, P, I32, I32, P, P, P],
    ),
    "fqa_decode_noalloc": (
        C.c_int,
        [C.POINTER(FqaDims), P, P, I64, P, I32, P, P, P, I32, I32, P, P],
    ),
    "fqa_prefill": (
        C.c_int,
        [C.POINTER(FqaDims), P, P, I64, P, I32, P, P, P, P, I32, I32, P, P],
    ),
    "fqa_sample": (C.c_int, [P, I32, I32, I64, P, P, P, P, P]),
    "fqa_gemm_workspace_bytes": (I64, [I32, I32, I32]),
    "fqa_gemm": (C.c_int, [P, I64, P, I64, P, I64, I32, I32, I32, I32, P, I64, P]),
    "fqa_qkv_proj_append": (
        C.c_int,
        [C.POINTER(FqaDims), P, I64, P, I64, I32, I32, P, P, P, P, P, I32, P, P, P, P, I64, I32,
         P, I64, P],
    ),
    "fqa_gemm_argmax_workspace_bytes": (I64, [I32, I32, I32]),
    "fqa_gemm_argmax": (C.c_int, [P, I64, P, I64, I32, I32, I32, P, P, I64, P]),
    "fqa_decode_read_floor": (C.c_int, [P, I64, P, I32, P, P, P, I32, P, P]),
    "fqa_decode_read_floor_prefix": (C.c_int, [P, I64, P, I32, P, P, P, P, I32, P, P]),
    "fqa_decode_prefix_workspace_bytes": (I64, [C.POINTER(FqaDims), I32, I32]),
    "fqa_decode_prefix": (
        C.c_int,
        [C.POINTER(FqaDims), P, P, I64, P, I32, P, P, P, P, P, I32, I32, I32, P, P, P],
    ),
    "fqa_version": (C.c_char_p, []),
}

_lib = None


def load() -> C.CDLL:
    """Load libfqa.so once; raise if it was not built (no fallback exists)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise ImportError(
                f"{LIB_PATH} is missing: build it with `python -m flashqwen_amd.build` "
                "(the attention path has no non-HIP implementation)"
            )
        lib = C.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


class FqaError(RuntimeError):
    pass


def check(rc: int, what: str) -> None:
    if rc != FQA_OK:
        names = {FQA_EINVAL: "EINVAL", FQA_EUNSUPPORTED: "EUNSUPPORTED", FQA_ELAUNCH: "ELAUNCH",
                 FQA_ENOSPACE: "ENOSPACE"}
        raise FqaError(f"{what} failed: {names.get(rc, rc)}")
