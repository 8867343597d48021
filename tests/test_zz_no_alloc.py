"""px_flat_search_device_noalloc (the entry point that allocates nothing) against
px_flat_search_device, through the C ABI on device buffers: two calls in a row on each
index, the second with a smaller input, to the parity rule (bit for bit on integer data,
whose keys are exact in fp32), with and without a filter, on a dim that is not a multiple
of 8 (queries padded inside the fixed scratch), plus the limits it rejects."""
import ctypes

import numpy as np
import pytest

import oracle
from conftest import assert_parity
from proxima_amd import FlatIndex, Metric, _lib, datagen

pytestmark = pytest.mark.gpu


class _Dev:
    def __init__(self):
        self.lib = _lib.load()
        self.ptrs = []

    def put(self, arr):
        arr = np.ascontiguousarray(arr)
        p = ctypes.c_void_p()
        assert self.lib.px_dev_alloc(ctypes.byref(p), max(arr.nbytes, 16)) == 0
        self.ptrs.append(p)
        if arr.nbytes:
            assert self.lib.px_dev_upload(p, arr.ctypes.data, arr.nbytes) == 0
        return p

    def empty(self, nbytes):
        p = ctypes.c_void_p()
        assert self.lib.px_dev_alloc(ctypes.byref(p), max(nbytes, 16)) == 0
        self.ptrs.append(p)
        return p

    def get(self, p, shape, dtype):
        out = np.empty(shape, dtype=dtype)
        assert self.lib.px_dev_download(out.ctypes.data, p, out.nbytes) == 0
        return out

    def free(self):
        for p in self.ptrs:
            self.lib.px_dev_free(p)
        self.ptrs = []


@pytest.fixture
def dev(gpu):
    d = _Dev()
    yield d
    d.free()


def _both(dev, idx, q, k, mask=None):
    """(ids, dists) of px_flat_search_device and of the no-allocation entry point."""
    lib = dev.lib
    nq = len(q)
    dq = dev.put(q.astype(np.float32))
    dm = dev.put(mask.view(np.uint8)) if mask is not None else None
    out = []
    for fn in (lib.px_flat_search_device, lib.px_flat_search_device_noalloc):
        di, dd = dev.empty(nq * k * 8), dev.empty(nq * k * 4)
        rc = fn(idx._h, dq, nq, k, dm, di, dd)
        assert rc == 0, _lib.last_error()
        out.append((dev.get(di, (nq, k), np.int64), dev.get(dd, (nq, k), np.float32)))
    return out


def _key_of(data, queries, metric):
    def key_of(qi, row):
        if metric == oracle.L2:
            return float(oracle.l2_sqr(queries[qi], data[row]))
        return -float(oracle.inner_product(queries[qi], data[row]))
    return key_of


def test_noalloc_equals_device_search_integer_l2(dev):
    data = datagen.sift_like(100_000, 128, 801)
    q = datagen.sift_like(1000, 128, 802)
    idx = FlatIndex(128, Metric.L2)
    idx.add(data)
    for nq, k in ((1000, 10), (100, 5)):  # the second call smaller
        print(f"no-alloc L2 sift nq={nq} k={k}", flush=True)
        (ids, d), (ids2, d2) = _both(dev, idx, q[:nq], k)
        assert np.array_equal(ids, ids2)
        assert np.array_equal(d.view(np.uint32), d2.view(np.uint32))
        o_ids, o_d, _ = oracle.flat_search(data, q[:nq], k, oracle.L2)
        assert np.array_equal(ids2, o_ids) and np.array_equal(d2, o_d)


def test_noalloc_filtered_and_padded_dim(dev):
    dim = 100  # padded to 104 inside the scratch
    data = datagen.unit_gaussian(30_000, dim, 811)
    q = datagen.unit_gaussian(300, dim, 812)
    mask = datagen.mask(30_000, 0.2, 813)
    idx = FlatIndex(dim, Metric.InnerProduct)
    idx.add(data)
    for nq, k, m in ((300, 40, mask), (20, 7, None)):
        print(f"no-alloc IP dim={dim} nq={nq} k={k} mask={m is not None}", flush=True)
        (ids, d), (ids2, d2) = _both(dev, idx, q[:nq], k, mask=m)
        o_ids, o_d, _ = oracle.flat_search(data, q[:nq], k, oracle.IP, mask=m)
        key_of = _key_of(data, q[:nq], oracle.IP)
        assert_parity(ids2, d2, ids, d, key_of)
        assert_parity(ids2, d2, o_ids, o_d, key_of)
        if m is not None:
            assert m[ids2[ids2 >= 0]].all()


def test_noalloc_limits(dev):
    lib = dev.lib
    data = datagen.gaussian(2000, 16, 821)
    idx = FlatIndex(16, Metric.L2)
    idx.add(data)
    dq = dev.put(datagen.gaussian(4, 16, 822))
    di, dd = dev.empty(4 * 200 * 8), dev.empty(4 * 200 * 4)
    assert lib.px_flat_search_device_noalloc(idx._h, dq, 4, 121, None, di, dd) == _lib.PX_ERR_BAD_K
    assert "k <= 120" in _lib.last_error()
    # more queries than the fixed scratch holds lists for: rejected before any search
    assert lib.px_flat_search_device_noalloc(idx._h, dq, 1 << 28, 10, None, di, dd) == \
        _lib.PX_ERR_ARG
    assert "limit" in _lib.last_error()
    # still usable after the rejections
    assert lib.px_flat_search_device_noalloc(idx._h, dq, 4, 10, None, di, dd) == 0
    ids = dev.get(di, (4, 10), np.int64)
    o_ids, _, _ = oracle.flat_search(data, datagen.gaussian(4, 16, 822), 10, oracle.L2)
    assert np.array_equal(ids, o_ids)


def test_noalloc_fresh_handle_allocates_nothing(dev):
    # On a fresh handle (rows added, no search yet, so no workspace exists) the entry point
    # must not need one: the library's own device allocations are capped at 1 byte
    # (PX_DEVICE_BUDGET, checked at every allocation it makes), so any allocation on the
    # way would fail the call. The caller's buffers (px_dev_alloc) are not counted.
    import os

    lib = dev.lib
    data = datagen.sift_like(60_000, 128, 831)
    q = datagen.sift_like(200, 128, 832)
    mask = datagen.mask(60_000, 0.3, 833)
    o = {m is not None: oracle.flat_search(data, q, 10, oracle.L2, mask=m)[:2]
         for m in (None, mask)}
    idx = FlatIndex(128, Metric.L2)
    idx.add(data)
    dq = dev.put(q)
    dm = dev.put(mask.view(np.uint8))
    di, dd = dev.empty(200 * 10 * 8), dev.empty(200 * 10 * 4)
    os.environ["PX_DEVICE_BUDGET"] = "1"
    try:
        for m, dmask in ((False, None), (True, dm)):
            print(f"no-alloc fresh handle under a 1-byte budget mask={m}", flush=True)
            rc = lib.px_flat_search_device_noalloc(idx._h, dq, 200, 10, dmask, di, dd)
            assert rc == 0, _lib.last_error()
            ids, d = dev.get(di, (200, 10), np.int64), dev.get(dd, (200, 10), np.float32)
            assert np.array_equal(ids, o[m][0]) and np.array_equal(d, o[m][1]), m
        # the allocating entry point does need its workspace: refused under the same cap
        assert lib.px_flat_search_device(idx._h, dq, 200, 10, None, di, dd) != 0
    finally:
        del os.environ["PX_DEVICE_BUDGET"]


def test_noalloc_nonfinite_query(dev):
    # same checks as px_flat_search_device (flat.rs:114-117): a NaN or infinite query value
    # fails with PX_ERR_NONFINITE before any output is written
    lib = dev.lib
    data = datagen.gaussian(20_000, 64, 841)
    q = datagen.gaussian(50, 64, 842)
    idx = FlatIndex(64, Metric.L2)
    idx.add(data)
    for bad in (np.nan, np.inf, -np.inf):
        qb = q.copy()
        qb[17, 5] = bad
        dq = dev.put(qb)
        di = dev.put(np.full((50, 10), 777, dtype=np.int64))
        dd = dev.put(np.full((50, 10), 7.5, dtype=np.float32))
        print(f"no-alloc non-finite query value {bad}", flush=True)
        assert lib.px_flat_search_device_noalloc(idx._h, dq, 50, 10, None, di, dd) == \
            _lib.PX_ERR_NONFINITE
        assert (dev.get(di, (50, 10), np.int64) == 777).all()
        assert (dev.get(dd, (50, 10), np.float32) == 7.5).all()
    # and the handle still serves finite queries
    dq = dev.put(q)
    di, dd = dev.empty(50 * 10 * 8), dev.empty(50 * 10 * 4)
    assert lib.px_flat_search_device_noalloc(idx._h, dq, 50, 10, None, di, dd) == 0
    o_ids, o_d, _ = oracle.flat_search(data, q, 10, oracle.L2)
    assert_parity(dev.get(di, (50, 10), np.int64), dev.get(dd, (50, 10), np.float32), o_ids, o_d,
                  _key_of(data, q, oracle.L2))
