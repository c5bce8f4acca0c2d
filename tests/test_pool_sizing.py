"""Pool sizing (fqa_pool_pages), the KvStore constructor's arithmetic (kv_store.cu:10-33):
pages = (total * fraction - used) / (layers * 2 * 16 * kv_dim * 2 B), refused when fewer
than one max_ctx sequence fits."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from flashqwen_amd import _lib
from flashqwen_amd.step import make_dims

GB = 10**9
PER_PAGE_36 = 36 * 2 * 16 * 1024 * 2  # one page of every Qwen3-8B layer: 2.25 MiB


def pages_of(total, used, fraction, layers=36, max_ctx=32768):
    lib = _lib.load()
    out = C.c_int64(-7)
    rc = lib.fqa_pool_pages(C.byref(make_dims()), total, used, fraction, layers, max_ctx,
                            C.byref(out))
    return rc, out.value


def test_288gb_known_answers():
    # 288 GB, 90% cap, 20 GB already used (weights + scratch): 239.2 GB for the pool.
    # float(288e9) * 0.9f is 259.2e9 within float rounding; by hand: 259200000000 rounds
    # to the float 259199991808 (ulp 32768), so avail = 239199991808 B, / 2359296 B
    # = 101386.3 -> 101386 pages (1,622,176 tokens).
    rc, n = pages_of(288 * GB, 20 * GB, 0.9)
    assert rc == _lib.FQA_OK
    assert n == 101386
    # the whole device, nothing used: 288e9 / 2359296 = 122070.3
    assert pages_of(288 * GB, 0, 1.0) == (_lib.FQA_OK, 122070)
    # config 5's ~200 GB pool: 200e9 / (36 x 64 KiB) = 84771 pages
    assert pages_of(200 * GB, 0, 1.0)[1] == 84771


def test_float_product_like_the_reference():
    """The reference multiplies size_t by float, so the budget is a float product; with a
    double product the page count differs for some sizes. Check against numpy float32."""
    rng = np.random.default_rng(0)
    for _ in range(200):
        total = int(rng.integers(1, 400)) * GB + int(rng.integers(0, 1 << 30))
        used = int(rng.integers(0, total))
        frac = float(np.float32(rng.uniform(0.05, 1.0)))
        layers = int(rng.integers(1, 64))
        budget = int(np.float32(total) * np.float32(frac))
        avail = max(budget - used, 0)
        want = avail // (layers * 2 * 16 * 1024 * 2)
        rc, n = pages_of(total, used, frac, layers=layers, max_ctx=16)
        assert n == want, (total, used, frac, layers)
        assert rc == (_lib.FQA_OK if want >= 1 else _lib.FQA_ENOSPACE)


def test_refuses_when_one_sequence_does_not_fit():
    # max_ctx 32768 needs 2048 pages = 4.83 GB at 36 layers
    need = 2048 * PER_PAGE_36
    rc, n = pages_of(need, 0, 1.0)
    assert (rc, n) == (_lib.FQA_OK, 2048)
    # one byte short (through `used`: total - 1 would round back up in the float product)
    rc, n = pages_of(need, 1, 1.0)
    assert (rc, n) == (_lib.FQA_ENOSPACE, 2047)
    # used beyond the budget: nothing left, count 0
    assert pages_of(100 * GB, 95 * GB, 0.9) == (_lib.FQA_ENOSPACE, 0)
    # partial last page does not count; max_ctx not a multiple of 16 rounds up
    assert pages_of(3 * PER_PAGE_36, 1, 1.0, max_ctx=33)[0] == _lib.FQA_ENOSPACE
    assert pages_of(3 * PER_PAGE_36, 0, 1.0, max_ctx=33) == (_lib.FQA_OK, 3)


def test_rejected_arguments():
    lib = _lib.load()
    d = make_dims()
    out = C.c_int64()
    assert lib.fqa_pool_pages(None, GB, 0, 0.9, 36, 4096, C.byref(out)) == _lib.FQA_EINVAL
    assert lib.fqa_pool_pages(C.byref(d), GB, 0, 0.9, 36, 4096, None) == _lib.FQA_EINVAL
    for frac in (0.0, -0.5, float("nan"), float("inf")):
        assert lib.fqa_pool_pages(C.byref(d), GB, 0, frac, 36, 4096, C.byref(out)) == _lib.FQA_EINVAL
    assert lib.fqa_pool_pages(C.byref(d), GB, 0, 0.9, 0, 4096, C.byref(out)) == _lib.FQA_EINVAL
    assert lib.fqa_pool_pages(C.byref(d), GB, 0, 0.9, 36, 0, C.byref(out)) == _lib.FQA_EINVAL
    assert lib.fqa_pool_pages_device(C.byref(d), 0.9, 36, 4096, None) == _lib.FQA_EINVAL


def test_fraction_above_one_accepted():
    """The reference's constructor takes any fraction (kv_store.cu:10-33): above 1 the
    budget is larger than the device, and the pages follow the same formula."""
    rc, pages = pages_of(288 * GB, 20 * GB, 1.5)
    assert rc == _lib.FQA_OK
    budget = int(np.float32(np.float32(288 * GB) * np.float32(1.5)))
    assert pages == (budget - 20 * GB) // (36 * 2 * 16 * 1024 * 2)


@pytest.mark.gpu
def test_device_sizing_matches_mem_get_info(gpu):
    """fqa_pool_pages_device reads hipMemGetInfo on the current device: the same count as
    fqa_pool_pages over torch's reading of it (no allocation in between)."""
    import torch

    lib = _lib.load()
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    free, total = torch.cuda.mem_get_info(gpu)
    out = C.c_int64()
    rc = lib.fqa_pool_pages_device(C.byref(make_dims()), 0.9, 36, 32768, C.byref(out))
    rc2, want = pages_of(total, total - free, 0.9)
    assert rc == rc2 == _lib.FQA_OK
    assert abs(out.value - want) <= 1  # free memory may move by a page-size crumb
    # the pool fits the 90% cap beside what is in use, and the next page would not
    per = 36 * 2 * 16 * 1024 * 2
    assert out.value * per + (total - free) <= 0.9 * total + per
    assert (out.value + 2) * per + (total - free) > 0.9 * total
    assert total > 250 * GB  # an MI355X: 288 GB of HBM
    print(f"device total {total / GB:.1f} GB, free {free / GB:.1f} GB -> {out.value} pages")
