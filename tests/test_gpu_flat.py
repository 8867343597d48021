"""GPU parity of the FlatIndex path (libproxima_px.so) against the CPU oracle.

Parity rule: ids identical at every rank except where the two candidates' keys differ by
less than 1e-5 relative; distances within 1e-4 relative. The oracle orders candidates by
(key, id), so exact ties go to the lower row id -- the GPU must do the same.
"""
import ctypes

import numpy as np
import pytest

import oracle
from conftest import assert_parity
from proxima_amd import FlatIndex, Metric, _lib, datagen

pytestmark = pytest.mark.gpu


def _oracle_key(data, queries, metric):
    def key_of(qi, row):
        if metric == oracle.L2:
            return float(oracle.l2_sqr(queries[qi], data[row]))
        return float(-oracle.inner_product(queries[qi], data[row]))
    return key_of


def _run(data, queries, k, metric, mask=None):
    m = Metric.L2 if metric == oracle.L2 else Metric.InnerProduct
    idx = FlatIndex(data.shape[1], m)
    idx.add(data)
    if mask is None:
        ids, d = idx.search_batch(queries, k=k)
    else:
        ids, d = idx.search_batch_filtered(queries, mask, k=k)
    o_ids, o_d, _ = oracle.flat_search(data, queries, k, metric, mask=mask)
    return ids, d, o_ids, o_d


def _check(data, queries, k, metric, mask=None, allow_exempt=True):
    ids, d, o_ids, o_d = _run(data, queries, k, metric, mask)
    print(f"case n={data.shape[0]} dim={data.shape[1]} nq={queries.shape[0]} k={k} "
          f"metric={metric} mask={'yes' if mask is not None else 'no'}", flush=True)
    return assert_parity(ids, d, o_ids, o_d, _oracle_key(data, queries, metric),
                         allow_exempt=allow_exempt)


def test_config1_full_l2(gpu):
    data = datagen.corpus(1)
    q = datagen.queries(1)
    _check(data, q, 10, oracle.L2)


@pytest.mark.parametrize("metric", [oracle.L2, oracle.IP])
@pytest.mark.parametrize("k", [1, 10, 37, 100, 128])
def test_gaussian_k_sweep(gpu, metric, k):
    data = datagen.gaussian(6000, 64, 77)
    q = datagen.gaussian(70, 64, 78)
    _check(data, q, k, metric)


def test_config2_reduced_ip(gpu):
    # the 100,000 x 384 unit-Gaussian workload on its first 30,000 rows and 200 queries
    data = datagen.corpus(2, rows=30_000)
    q = datagen.queries(2, rows=200)
    _check(data, q, 10, oracle.IP)


@pytest.mark.parametrize("k", [10, 100])
def test_config3_reduced_sift_integers_bit_exact(gpu, k):
    # SIFT-like integers: every partial sum < 2^24, so keys are exact in any order and ids
    # must match the oracle's (key, id) order with no exemption at all.
    data = datagen.corpus(3, rows=200_000)
    q = datagen.queries(3, rows=256)
    ids, d, o_ids, o_d = _run(data, q, k, oracle.L2)
    assert np.array_equal(ids, o_ids)
    assert np.array_equal(d, o_d)


@pytest.mark.parametrize("dim", [1, 4, 7, 12, 24, 100, 130, 200, 256, 384, 1000, 2051])
def test_odd_dims(gpu, dim):
    data = datagen.gaussian(3000, dim, 11 + dim)
    q = datagen.gaussian(40, dim, 12 + dim)
    for metric in (oracle.L2, oracle.IP):
        _check(data, q, 10, metric)


@pytest.mark.parametrize("dim", [3, 200, 256, 384, 1000, 2051])
def test_odd_dims_collect_path(gpu, dim):
    # 260 queries and k = 20: the threshold-collect path, with 1, 2-3 (the queries resident in
    # registers) and 8 / 17 query chunks
    data = datagen.gaussian(4000, dim, 21 + dim)
    q = datagen.gaussian(260, dim, 22 + dim)
    for metric in (oracle.L2, oracle.IP):
        _check(data, q, 20, metric)


@pytest.mark.parametrize("p", [0.0, 0.001, 0.2, 0.5, 1.0])
def test_filtered(gpu, p):
    data = datagen.gaussian(20_000, 48, 5)
    q = datagen.gaussian(50, 48, 6)
    mask = datagen.mask(20_000, p, 7)
    for metric in (oracle.L2, oracle.IP):
        _check(data, q, 10, metric, mask=mask)


@pytest.mark.parametrize("dim", [256, 384])
def test_filtered_resident_query_lists(gpu, dim):
    # lists of 32 over rows of 129-384 padded dims (the queries resident in registers, every
    # chunk full) behind a filter, both metrics
    data = datagen.gaussian(12_000, dim, 90 + dim)
    q = datagen.gaussian(60, dim, 91 + dim)
    mask = datagen.mask(12_000, 0.3, 92)
    for metric in (oracle.L2, oracle.IP):
        _check(data, q, 10, metric, mask=mask)


def test_filtered_large_k_and_sparse(gpu):
    data = datagen.sift_like(50_000, 128, 9)
    q = datagen.sift_like(64, 128, 10)
    mask = datagen.mask(50_000, 0.1, 11)
    ids, d, o_ids, o_d = _run(data, q, 100, oracle.L2, mask)
    assert np.array_equal(ids, o_ids)
    assert np.array_equal(d, o_d)
    assert mask[ids[ids >= 0]].all()


def test_ties_go_to_lower_id(gpu):
    # many exact duplicates: rows repeat with period 7, so every key is tied 1,000-fold
    base = datagen.sift_like(7, 32, 3)
    data = np.tile(base, (1000, 1))
    q = datagen.sift_like(20, 32, 4)
    for metric in (oracle.L2, oracle.IP):
        ids, d, o_ids, o_d = _run(data, q, 25, metric)
        assert np.array_equal(ids, o_ids), metric
        assert np.array_equal(d, o_d), metric


def test_all_rows_identical(gpu):
    data = np.ones((5000, 16), dtype=np.float32)
    q = np.full((3, 16), 2.0, dtype=np.float32)
    ids, d, o_ids, o_d = _run(data, q, 50, oracle.L2)
    assert np.array_equal(ids, np.tile(np.arange(50), (3, 1)))
    assert np.array_equal(ids, o_ids) and np.array_equal(d, o_d)


def test_k_larger_than_n_pads(gpu):
    data = datagen.gaussian(5, 8, 1)
    q = datagen.gaussian(3, 8, 2)
    for metric in (oracle.L2, oracle.IP):
        ids, d, o_ids, o_d = _run(data, q, 12, metric)
        assert (ids[:, 5:] == -1).all()
        pad = np.float32(3.4028235e38) if metric == oracle.L2 else np.float32(-3.4028235e38)
        assert (d[:, 5:] == pad).all()
        assert np.array_equal(ids, o_ids)


def test_reference_padding_known_answer(gpu):
    # crates/core/src/flat.rs:323-338
    idx = FlatIndex(4, Metric.L2)
    idx.add(np.array([[0, 0, 0, 0], [1, 1, 1, 1]], dtype=np.float32))
    ids, d = idx.search(np.zeros(4, dtype=np.float32), k=5)
    assert ids.tolist() == [0, 1, -1, -1, -1]
    assert d[0] == 0.0 and d[1] == 2.0
    assert (d[2:] == np.float32(3.4028235e38)).all()


def test_reference_filtered_padding_known_answer(gpu):
    # crates/core/src/flat.rs:370-383
    idx = FlatIndex(4, Metric.L2)
    idx.add(np.array([[0] * 4, [1] * 4, [2] * 4], dtype=np.float32))
    ids, d = idx.search_filtered(np.zeros(4, dtype=np.float32),
                                 np.array([True, False, False]), k=5)
    assert ids.tolist() == [0, -1, -1, -1, -1]
    assert (d[1:] == np.float32(3.4028235e38)).all()


def test_self_is_nearest_reference(gpu):
    # crates/core/src/flat.rs:252-267 (200 x 16, SplitMix seed 42, uniform [-1, 1])
    data = datagen.uniform_pm1(200, 16, 42)
    idx = FlatIndex(16, Metric.L2)
    idx.add(data)
    ids, d = idx.search_batch(data, k=1)
    assert np.array_equal(ids[:, 0], np.arange(200))
    assert (np.abs(d[:, 0]) < 1e-3).all()
    assert (d[:, 0] == 0.0).all()  # exact re-rank: distance to itself is exactly 0


def test_batch_matches_single_reference(gpu):
    # crates/core/src/flat.rs:294-321 (500 x 12 IP, 33 queries, k=5)
    data = datagen.uniform_pm1(500, 12, 3)
    q = datagen.uniform_pm1(33, 12, 88)
    idx = FlatIndex(12, Metric.InnerProduct)
    idx.add(data)
    bids, bd = idx.search_batch(q, k=5, num_threads=4)
    for qi in range(33):
        sids, sd = idx.search(q[qi], k=5)
        assert bids[qi].tolist() == sids.tolist()
        assert np.abs(bd[qi] - sd).max() < 1e-4
        assert (np.diff(sd) <= 1e-4).all()


def test_incremental_add_and_regrowth(gpu):
    data = datagen.gaussian(5000, 40, 21)
    q = datagen.gaussian(30, 40, 22)
    idx = FlatIndex(40, Metric.L2)
    for lo in range(0, 5000, 700):
        idx.add(data[lo:lo + 700])
        ids, d = idx.search_batch(q, k=7)
        o_ids, o_d, _ = oracle.flat_search(data[:lo + 700], q, 7, oracle.L2)
        assert_parity(ids, d, o_ids, o_d, _oracle_key(data, q, oracle.L2))
    assert np.array_equal(idx.vectors(), data)


def test_empty_index_and_zero_k(gpu):
    idx = FlatIndex(8, Metric.InnerProduct)
    ids, d = idx.search(np.zeros(8, dtype=np.float32), k=3)
    assert ids.tolist() == [-1, -1, -1]
    assert (d == np.float32(-3.4028235e38)).all()
    idx.add(datagen.gaussian(10, 8, 1))
    ids, d = idx.search_batch(datagen.gaussian(4, 8, 2), k=0)
    assert ids.shape == (4, 0) and d.shape == (4, 0)


def test_k_above_seam_limit_searches(gpu):
    # the reference's FlatIndex takes any k: every row in order, then padding
    data = datagen.gaussian(300, 8, 1)
    idx = FlatIndex(8, Metric.L2)
    idx.add(data)
    q = np.zeros(8, dtype=np.float32)
    ids, d = idx.search(q, k=_lib.PX_MAX_K + 1)
    o_ids, o_d, _ = oracle.flat_search(data, q[None, :], _lib.PX_MAX_K + 1, oracle.L2)
    assert np.array_equal(ids, o_ids[0]) and np.array_equal(d, o_d[0])
    assert (ids[300:] == -1).all() and (d[300:] == np.finfo(np.float32).max).all()


def test_knn_gpu_seam_raw_keys(gpu):
    # crates/core/src/gpu.rs:10-15 signatures; keys are raw (squared L2 / negated IP)
    lib = _lib.load()
    data = datagen.gaussian(3000, 32, 31)
    q = datagen.gaussian(25, 32, 32)
    h = lib.knn_gpu_create(_lib.f32p(data), 3000, 32)
    assert h
    try:
        for metric in (oracle.L2, oracle.IP):
            ids = np.empty((25, 10), dtype=np.int64)
            keys = np.empty((25, 10), dtype=np.float32)
            rc = lib.knn_gpu_search(h, _lib.f32p(q), 25, 10, metric,
                                    ids.ctypes.data_as(ctypes.POINTER(ctypes.c_longlong)),
                                    _lib.f32p(keys))
            assert rc == 0, _lib.last_error()
            o_ids, _, o_keys = oracle.flat_search(data, q, 10, metric)
            assert np.array_equal(ids, o_ids)
            assert np.array_equal(keys, o_keys)
        assert lib.knn_gpu_search(h, _lib.f32p(q), 25, 0, 0, None, None) == -1
    finally:
        lib.knn_gpu_free(h)


def test_device_pointer_entry(gpu):
    lib = _lib.load()
    data = datagen.gaussian(4000, 100, 41)
    q = datagen.gaussian(50, 100, 42)
    mask = datagen.mask(4000, 0.3, 43)
    idx = FlatIndex(100, Metric.L2)
    idx.add(data)
    ptrs = []

    def dev(arr):
        p = ctypes.c_void_p()
        assert lib.px_dev_alloc(ctypes.byref(p), max(arr.nbytes, 1)) == 0
        ptrs.append(p)
        assert lib.px_dev_upload(p, arr.ctypes.data, arr.nbytes) == 0
        return p

    try:
        dq, dm = dev(q), dev(mask.view(np.uint8))
        ids = np.empty((50, 10), dtype=np.int64)
        dd = np.empty((50, 10), dtype=np.float32)
        di, ddist = dev(ids), dev(dd)
        rc = lib.px_flat_search_device(idx._h, dq, 50, 10, dm, di, ddist)
        assert rc == 0, _lib.last_error()
        assert lib.px_dev_download(ids.ctypes.data, di, ids.nbytes) == 0
        assert lib.px_dev_download(dd.ctypes.data, ddist, dd.nbytes) == 0
        h_ids, h_d = idx.search_batch_filtered(q, mask, k=10)
        assert np.array_equal(ids, h_ids) and np.array_equal(dd, h_d)
    finally:
        for p in ptrs:
            lib.px_dev_free(p)


@pytest.mark.parametrize("nq,k,masked,path", [
    (200, 10, False, "lists"),   # the check is read back with the search's last wait
    (200, 10, True, "lists"),    # a filter: resolved before the mask is compacted
    (2048, 10, False, "collect-bounded"),
    (300, 200, False, "collect-sampled"),
    (5, 10, False, "vector"),
])
def test_device_query_nonfinite_leaves_outputs(gpu, nq, k, masked, path):
    # flat.rs:114-117 rejects a NaN or infinite query before searching: the device form
    # returns PX_ERR_NONFINITE with the outputs unwritten, whichever path the batch takes,
    # and the next, finite batch is searched normally
    lib = _lib.load()
    data = datagen.gaussian(40_000, 64, 44)
    q = datagen.gaussian(nq, 64, 45)
    mask = datagen.mask(40_000, 0.5, 46) if masked else None
    idx = FlatIndex(64, Metric.L2)
    idx.add(data)
    ptrs = []

    def dev(arr):
        p = ctypes.c_void_p()
        assert lib.px_dev_alloc(ctypes.byref(p), max(arr.nbytes, 1)) == 0
        ptrs.append(p)
        assert lib.px_dev_upload(p, arr.ctypes.data, arr.nbytes) == 0
        return p

    try:
        sentinel_i = np.full((nq, k), 1234567, dtype=np.int64)
        sentinel_d = np.full((nq, k), 7.5, dtype=np.float32)
        di, dd = dev(sentinel_i), dev(sentinel_d)
        dm = dev(mask.view(np.uint8)) if masked else None
        for bad in (np.nan, np.inf, -np.inf):
            qb = q.copy()
            qb[nq // 2, 17] = bad
            print(f"case nonfinite device query nq={nq} k={k} masked={masked} {bad}", flush=True)
            rc = lib.px_flat_search_device(idx._h, dev(qb), nq, k, dm, di, dd)
            assert rc == _lib.PX_ERR_NONFINITE, (rc, _lib.last_error())
            got_i, got_d = np.empty_like(sentinel_i), np.empty_like(sentinel_d)
            assert lib.px_dev_download(got_i.ctypes.data, di, got_i.nbytes) == 0
            assert lib.px_dev_download(got_d.ctypes.data, dd, got_d.nbytes) == 0
            assert np.array_equal(got_i, sentinel_i) and np.array_equal(got_d, sentinel_d)
        assert lib.px_flat_search_device(idx._h, dev(q), nq, k, dm, di, dd) == 0, _lib.last_error()
        ids, dist = np.empty_like(sentinel_i), np.empty_like(sentinel_d)
        assert lib.px_dev_download(ids.ctypes.data, di, ids.nbytes) == 0
        assert lib.px_dev_download(dist.ctypes.data, dd, dist.nbytes) == 0
        if masked:
            h_ids, h_d = idx.search_batch_filtered(q, mask, k=k)
        else:
            h_ids, h_d = idx.search_batch(q, k=k)
        assert np.array_equal(ids, h_ids) and np.array_equal(dist, h_d)
        assert idx._last_timing()["path"] == path
    finally:
        for p in ptrs:
            lib.px_dev_free(p)


@pytest.mark.parametrize("k", [24, 25, 48, 49, 112, 113, 120])
def test_list_capacity_boundaries(gpu, k):
    # k' = k + 8 crosses the list classes (32 int ids | 56 and 120 with 16-bit offsets | 128)
    data = datagen.sift_like(20_000, 40, 51)
    q = datagen.sift_like(45, 40, 52)
    for metric in (oracle.L2, oracle.IP):
        ids, d, o_ids, o_d = _run(data, q, k, metric)
        assert np.array_equal(ids, o_ids), (k, metric)
        assert np.array_equal(d, o_d), (k, metric)


def test_large_k_many_splits_16bit_offsets(gpu):
    # 300k rows at k=100: at least five splits of <= 65,472 rows, positions stored as 16-bit
    # offsets from each split's start
    data = datagen.sift_like(300_000, 16, 61)
    q = datagen.sift_like(40, 16, 62)
    for metric in (oracle.L2, oracle.IP):
        ids, d, o_ids, o_d = _run(data, q, 100, metric)
        assert np.array_equal(ids, o_ids), metric
        assert np.array_equal(d, o_d), metric


def test_large_k_filtered_multichunk(gpu):
    # dim 200 (two 128-dim query chunks), 30% filter, k=100 and k=40
    data = datagen.gaussian(40_000, 200, 71)
    q = datagen.gaussian(30, 200, 72)
    mask = datagen.mask(40_000, 0.3, 73)
    for k in (40, 100):
        for metric in (oracle.L2, oracle.IP):
            _check(data, q, k, metric, mask=mask)


def test_merge_bound_with_many_ties(gpu):
    # 0/1 rows: thousands of rows share each distance, so more than 256 split candidates sit
    # at the scan's published bound and the merge sorts all of them; ties to the lower row
    rng = np.random.default_rng(74)
    data = rng.integers(0, 2, size=(30_000, 16)).astype(np.float32)
    q = rng.integers(0, 2, size=(40, 16)).astype(np.float32)
    for metric in (oracle.L2, oracle.IP):
        ids, d, o_ids, o_d = _run(data, q, 10, metric)
        assert np.array_equal(ids, o_ids), metric
        assert np.array_equal(d, o_d), metric


def test_merge_bound_gaussian_many_splits(gpu):
    # a query tile spread over many splits (each publishing its bounds): the merge sorts
    # only the candidates at or below them
    data = datagen.gaussian(200_000, 64, 75)
    q = datagen.gaussian(20, 64, 76)
    for k in (1, 10, 20):
        _check(data, q, k, oracle.L2)
