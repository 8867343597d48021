"""A stage-sync wait that gives up fails the search, on every scan that has one.

The barrier-free scans (the collect scans, and the per-split lists of k + 8 <= 32) order
their stage buffers by a bounded wait: a wave polls the other waves' committed stages and,
after a limit of polls, goes on and reports it. These tests lower the limit from the host
(px_flat_set_spin_limit: one poll) so that the waves of a workgroup holding few live query
slots -- the padding waves of its last query tile stage the corpus and run ahead of the
live ones -- give up, while every kernel still runs to its end. The search must then fail
with PX_ERR_DEVICE ("stage sync"), leave its device outputs as they were, and a search on the
same handle with the limit restored must equal the oracle (flat.rs:106-148 restated).
Covered: the lists in fp32 and fp16 (128-dim rows) and of 384-dim rows (flat_list16q_kernel,
the queries resident in registers), the bounded collect scan in fp32 and fp16, the sampled
collect scan of 128-dim rows (its sample and collect scans) and of 384-dim rows (its sample
scan on flat_scan_kernel, its collect scan on flat_list16q_kernel), the no-allocation entry
point, and the host-array form.
"""
import ctypes

import numpy as np
import pytest

import oracle
from conftest import assert_parity
from proxima_amd import FlatIndex, Metric, _lib, datagen

pytestmark = pytest.mark.gpu

SENTINEL_ID = 0x5A5A5A5A5A5A5A5A
SENTINEL_D = np.float32(-12345.5)


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


def _key_of(data, queries, metric):
    def key_of(qi, row):
        if metric == oracle.L2:
            return float(oracle.l2_sqr(queries[qi], data[row]))
        return float(-oracle.inner_product(queries[qi], data[row]))
    return key_of


def _give_up_then_recover(dev, data, q, k, metric, path, f16=False, mask=None,
                          noalloc=False):
    """One search with the limit at one poll (must fail, outputs untouched), then one with
    the kernels' own limit (must match the oracle)."""
    lib = dev.lib
    nq = len(q)
    idx = FlatIndex(data.shape[1], Metric.L2 if metric == oracle.L2 else Metric.InnerProduct)
    idx.add(data)
    idx._scan_f16(f16)
    dq = dev.put(q)
    dm = dev.put(mask.view(np.uint8)) if mask is not None else None
    fn = lib.px_flat_search_device_noalloc if noalloc else lib.px_flat_search_device
    di = dev.put(np.full((nq, k), SENTINEL_ID, dtype=np.int64))
    dd = dev.put(np.full((nq, k), SENTINEL_D, dtype=np.float32))
    print(f"case give-up path={path} n={data.shape[0]} dim={data.shape[1]} nq={nq} k={k} "
          f"f16={f16} mask={mask is not None} noalloc={noalloc}", flush=True)
    idx._spin_limit(1)
    rc = fn(idx._h, dq, nq, k, dm, di, dd)
    msg = _lib.last_error()
    assert rc == _lib.PX_ERR_DEVICE, (rc, msg)
    assert "stage sync" in msg, msg
    t = idx._last_timing()
    assert t["path"] == path, t
    assert t["scan_f16"] == f16, t
    assert (dev.get(di, (nq, k), np.int64) == SENTINEL_ID).all(), "ids written"
    assert (dev.get(dd, (nq, k), np.float32) == SENTINEL_D).all(), "distances written"

    idx._spin_limit(0)
    rc = fn(idx._h, dq, nq, k, dm, di, dd)
    assert rc == 0, _lib.last_error()
    assert idx._last_timing()["path"] == path
    ids, d = dev.get(di, (nq, k), np.int64), dev.get(dd, (nq, k), np.float32)
    o_ids, o_d, _ = oracle.flat_search(data, q, k, metric, mask=mask)
    assert_parity(ids, d, o_ids, o_d, _key_of(data, q, metric))
    return idx


# 100 queries: one query tile of 256 slots with four live waves and four padding ones
def test_lists_fp32(dev):
    data = datagen.gaussian(200_000, 128, 501)
    _give_up_then_recover(dev, data, datagen.gaussian(100, 128, 502), 10, oracle.L2, "lists")


def test_lists_fp16(dev):
    data = datagen.sift_like(200_000, 128, 503)
    _give_up_then_recover(dev, data, datagen.sift_like(100, 128, 504), 10, oracle.L2, "lists",
                          f16=True)


def test_lists_filtered_ip(dev):
    data = datagen.unit_gaussian(200_000, 128, 505)
    mask = datagen.mask(200_000, 0.5, 506)
    _give_up_then_recover(dev, data, datagen.unit_gaussian(100, 128, 507), 24, oracle.IP,
                          "lists", mask=mask)


def test_lists_384(dev):
    # 40 queries on 384-dim rows: one query tile of 128 slots (16 a wave), five of its eight
    # waves padding
    data = datagen.unit_gaussian(200_000, 384, 518)
    _give_up_then_recover(dev, data, datagen.unit_gaussian(40, 384, 519), 10, oracle.IP,
                          "lists")


def test_noalloc_lists(dev):
    data = datagen.gaussian(200_000, 128, 508)
    _give_up_then_recover(dev, data, datagen.gaussian(100, 128, 509), 10, oracle.L2, "lists",
                          noalloc=True)


# 2,088 queries over 100,000 rows: 28 splits (bounded first round); the last query tile
# holds 40 queries, so six of its eight waves are padding
def test_bounded_collect_fp32(dev):
    data = datagen.gaussian(100_000, 128, 510)
    _give_up_then_recover(dev, data, datagen.gaussian(2088, 128, 511), 10, oracle.L2,
                          "collect-bounded")


def test_bounded_collect_fp16(dev):
    data = datagen.sift_like(100_000, 128, 512)
    _give_up_then_recover(dev, data, datagen.sift_like(2088, 128, 513), 10, oracle.L2,
                          "collect-bounded", f16=True)


def test_sampled_collect_128(dev):
    # k' = 58 past the lists on 300 queries: sample scan, ladder, collect scan, select
    data = datagen.gaussian(200_000, 128, 514)
    _give_up_then_recover(dev, data, datagen.gaussian(300, 128, 515), 50, oracle.L2,
                          "collect-sampled")


def test_sampled_collect_384(dev):
    # rows of three 128-dim chunks (k = 16, 300,000 rows): the sample scan on
    # flat_scan_kernel's collect mode, the collect scan on flat_list16q_kernel's
    data = datagen.unit_gaussian(300_000, 384, 516)
    _give_up_then_recover(dev, data, datagen.unit_gaussian(300, 384, 517), 16, oracle.IP,
                          "collect-sampled")


def test_host_arrays_raise(gpu):
    data = datagen.gaussian(200_000, 128, 518)
    q = datagen.gaussian(100, 128, 519)
    idx = FlatIndex(128, Metric.L2)
    idx.add(data)
    idx._spin_limit(1)
    print("case give-up host arrays", flush=True)
    with pytest.raises(RuntimeError, match="stage sync"):
        idx.search_batch(q, k=10)
    idx._spin_limit(0)
    ids, d = idx.search_batch(q, k=10)
    o_ids, o_d, _ = oracle.flat_search(data, q, 10, oracle.L2)
    assert_parity(ids, d, o_ids, o_d, _key_of(data, q, oracle.L2))


def test_spin_limit_argument(gpu):
    idx = FlatIndex(8, Metric.L2)
    with pytest.raises(ValueError):
        idx._spin_limit(-1)
