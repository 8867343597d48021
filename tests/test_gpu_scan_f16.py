"""GPU parity of the scans that use the fp16 copy of exact rows.

When every value of the rows and of a batch's queries is exactly an fp16 zero or normal
number -- integer-valued descriptors such as the SIFT-like workload's are -- every product
q_i * x_i is exact in fp16 as in fp32, so the collect scan (flat_collect_kernel) and the
per-split list scan (flat_scan_kernel, on at least 65,536 rows) multiply on the fp16 matrix
cores with fp32 accumulation; their candidates are re-ranked in the reference's arithmetic
(distance.rs:3-39) exactly as on the fp32 scans. The vector-ALU scan of at most 16 queries
reads the copy widened to the same fp32 values. Results must equal the oracle's
(flat.rs:106-148) bit for bit on integer data and the fp32 scans', and the scans must fall
back to fp32 whenever a row or a query is not exact in fp16 (rounded, past 65504, or an fp16
subnormal).
"""
import numpy as np
import pytest

import oracle
from conftest import assert_parity
from proxima_amd import FlatIndex, Metric, datagen

pytestmark = pytest.mark.gpu


def _key_of(data, queries, metric):
    def key_of(qi, row):
        if metric == oracle.L2:
            return float(oracle.l2_sqr(queries[qi], data[row]))
        return float(-oracle.inner_product(queries[qi], data[row]))
    return key_of


def _index(data, metric):
    idx = FlatIndex(data.shape[1], Metric.L2 if metric == oracle.L2 else Metric.InnerProduct)
    idx.add(data)
    return idx


def _run(idx, q, k, mask=None):
    if mask is None:
        ids, d = idx.search_batch(q, k=k)
    else:
        ids, d = idx.search_batch_filtered(q, mask, k=k)
    info = idx._last_timing()
    return ids, d, info


def _same(a_ids, a_d, b_ids, b_d):
    return np.array_equal(a_ids, b_ids) and np.array_equal(a_d.view(np.uint32), b_d.view(np.uint32))


@pytest.mark.parametrize("metric", [oracle.L2, oracle.IP])
@pytest.mark.parametrize("k", [100, 1000])
def test_integer_rows_f16_equals_oracle_and_fp32(gpu, metric, k):
    # the sampled collect path (threshold sample scan, ladder, collect scan)
    data = datagen.sift_like(100_000, 128, 701)
    q = datagen.sift_like(1000, 128, 702)
    idx = _index(data, metric)
    print(f"case sift-like 100000 x 128, 1000 queries, k={k}, metric={metric}", flush=True)
    ids, d, info = _run(idx, q, k)
    print(f"  path {info['path']}, f16 {info['scan_f16']}, rounds {info['collect_rounds']}",
          flush=True)
    assert info["path"].startswith("collect")
    assert info["scan_f16"]
    o_ids, o_d, _ = oracle.flat_search(data, q, k, metric)
    assert np.array_equal(ids, o_ids)
    assert np.array_equal(d.view(np.uint32), o_d.view(np.uint32))
    idx._scan_f16(False)
    ids32, d32, info32 = _run(idx, q, k)
    assert not info32["scan_f16"] and info32["path"] == info["path"]
    assert _same(ids, d, ids32, d32)


def test_integer_rows_filtered(gpu):
    data = datagen.sift_like(120_000, 128, 711)
    q = datagen.sift_like(600, 128, 712)
    mask = datagen.mask(120_000, 0.3, 713)
    idx = _index(data, oracle.L2)
    for k in (10, 200):
        print(f"case sift-like filtered 30%, k={k}", flush=True)
        ids, d, info = _run(idx, q, k, mask)
        print(f"  path {info['path']}, f16 {info['scan_f16']}", flush=True)
        o_ids, o_d, _ = oracle.flat_search(data, q, k, oracle.L2, mask=mask)
        assert np.array_equal(ids, o_ids)
        assert np.array_equal(d.view(np.uint32), o_d.view(np.uint32))
        assert info["scan_f16"] == info["path"].startswith("collect")


@pytest.mark.parametrize("metric", [oracle.L2, oracle.IP])
def test_bounded_path(gpu, metric):
    # the 1M x 128 workload's route (collect-bounded: no sample, the splits' shared bound):
    # 2,048 queries over 60,000 rows (32 splits)
    data = datagen.sift_like(60_000, 128, 721)
    q = datagen.sift_like(2048, 128, 722)
    idx = _index(data, metric)
    for k in (1, 10, 16):
        print(f"case sift-like 60000 x 128, 2048 queries, k={k}, metric={metric}", flush=True)
        ids, d, info = _run(idx, q, k)
        print(f"  path {info['path']}, f16 {info['scan_f16']}", flush=True)
        assert info["path"] == "collect-bounded" and info["scan_f16"]
        o_ids, o_d, _ = oracle.flat_search(data, q, k, metric)
        assert np.array_equal(ids, o_ids)
        assert np.array_equal(d.view(np.uint32), o_d.view(np.uint32))


@pytest.mark.parametrize("n", [57_560, 57_600, 57_686, 57_816, 59_000])
def test_bounded_path_split_ends(gpu, n):
    # the scan runs whole stages of four 32-row tiles, then a split's last partial stage with
    # per-tile checks. Splits hold a multiple of 64 rows (an even tile count); with 2,048
    # queries these row counts give 60-62 splits of 960 rows (30 tiles: two past the last
    # whole stage) and a last split of 920, 960, 86, 216 and 440 rows (29, 30, 3, 7 and 14
    # tiles), so a partial stage of each length, and a split shorter than one stage, is met
    data = datagen.sift_like(n, 128, 731)
    q = datagen.sift_like(2048, 128, 732)
    idx = _index(data, oracle.L2)
    print(f"case sift-like {n} x 128, 2048 queries, k=10, L2", flush=True)
    ids, d, info = _run(idx, q, 10)
    print(f"  path {info['path']}, f16 {info['scan_f16']}, splits {info['splits']}", flush=True)
    assert info["path"] == "collect-bounded" and info["scan_f16"]
    o_ids, o_d, _ = oracle.flat_search(data, q, 10, oracle.L2)
    assert np.array_equal(ids, o_ids)
    assert np.array_equal(d.view(np.uint32), o_d.view(np.uint32))


def test_fp16_exact_fractions_and_signs(gpu):
    # multiples of 1/16 with signs: exact in fp16 (normal numbers or zero), not integers
    rng = np.random.default_rng(731)
    data = (rng.integers(-400, 400, size=(60_000, 128)) / 16.0).astype(np.float32)
    q = (rng.integers(-400, 400, size=(700, 128)) / 16.0).astype(np.float32)
    for metric in (oracle.L2, oracle.IP):
        idx = _index(data, metric)
        print(f"case fractions metric={metric}", flush=True)
        ids, d, info = _run(idx, q, 100)
        assert info["scan_f16"]
        o_ids, o_d, _ = oracle.flat_search(data, q, 100, metric)
        assert_parity(ids, d, o_ids, o_d, _key_of(data, q, metric))
        idx._scan_f16(False)
        ids32, d32, _ = _run(idx, q, 100)
        assert_parity(ids32, d32, o_ids, o_d, _key_of(data, q, metric))


def test_fallback_when_not_exact(gpu):
    rows = datagen.sift_like(40_000, 128, 741)
    q = datagen.sift_like(400, 128, 742)
    k = 100
    cases = {
        "rounded query value": (rows, np.where(np.arange(128) == 5, q + 0.3, q).astype(np.float32)),
        "query past 65504": (rows, np.where(np.arange(128) == 7, 70000.0, q).astype(np.float32)),
        "query fp16 subnormal": (rows, np.where(np.arange(128) == 9, 2.0 ** -20, q).astype(np.float32)),
        "gaussian rows": (datagen.gaussian(40_000, 128, 743), q),
    }
    for name, (data, qq) in cases.items():
        print(f"case fallback: {name}", flush=True)
        idx = _index(data, oracle.L2)
        ids, d, info = _run(idx, qq, k)
        assert info["path"].startswith("collect")
        assert not info["scan_f16"], name
        o_ids, o_d, _ = oracle.flat_search(data, qq, k, oracle.L2)
        assert_parity(ids, d, o_ids, o_d, _key_of(data, qq, oracle.L2))


def test_inexact_rows_added_later_drop_the_fp16_copy(gpu):
    a = datagen.sift_like(30_000, 128, 751)
    b = datagen.gaussian(5_000, 128, 752)
    q = datagen.sift_like(300, 128, 753)
    idx = _index(a, oracle.L2)
    _, _, info = _run(idx, q, 100)
    assert info["scan_f16"]
    idx.add(b)
    print("case rows added that are not exact in fp16", flush=True)
    ids, d, info = _run(idx, q, 100)
    assert not info["scan_f16"]
    both = np.concatenate([a, b])
    o_ids, o_d, _ = oracle.flat_search(both, q, 100, oracle.L2)
    assert_parity(ids, d, o_ids, o_d, _key_of(both, q, oracle.L2))


def test_exact_rows_added_later_keep_the_fp16_copy(gpu):
    # the fp16 copy grows with the rows (a second add past the first allocation)
    a = datagen.sift_like(20_000, 128, 761)
    b = datagen.sift_like(50_000, 128, 762)
    q = datagen.sift_like(300, 128, 763)
    idx = _index(a, oracle.L2)
    idx.add(b)
    print("case exact rows added twice", flush=True)
    ids, d, info = _run(idx, q, 150)
    assert info["scan_f16"]
    both = np.concatenate([a, b])
    o_ids, o_d, _ = oracle.flat_search(both, q, 150, oracle.L2)
    assert np.array_equal(ids, o_ids)
    assert np.array_equal(d.view(np.uint32), o_d.view(np.uint32))


@pytest.mark.parametrize("nq", [1, 5, 16])
def test_few_queries_read_the_fp16_rows(gpu, nq):
    # batches of at most 16 queries take the vector-ALU scan; with the fp16 copy of the rows
    # it reads half the bytes and widens them to the same fp32 values: bit-identical keys,
    # whatever the queries hold (here not exact in fp16)
    data = datagen.sift_like(150_000, 128, 771)
    q = (datagen.sift_like(nq, 128, 772) + 0.37).astype(np.float32)
    mask = datagen.mask(150_000, 0.4, 773)
    for metric in (oracle.L2, oracle.IP):
        idx = _index(data, metric)
        for k, m in ((10, None), (100, None), (10, mask)):
            print(f"case few queries nq={nq} k={k} metric={metric} mask={m is not None}", flush=True)
            ids, d, info = _run(idx, q, k, m)
            assert info["path"] == "vector" and info["scan_f16"]
            o_ids, o_d, _ = oracle.flat_search(data, q, k, metric, mask=m)
            assert_parity(ids, d, o_ids, o_d, _key_of(data, q, metric))
            idx._scan_f16(False)
            ids32, d32, info32 = _run(idx, q, k, m)
            idx._scan_f16(True)
            assert not info32["scan_f16"]
            assert _same(ids, d, ids32, d32)


@pytest.mark.parametrize("metric", [oracle.L2, oracle.IP])
@pytest.mark.parametrize("nq,k", [(32, 10), (100, 1), (200, 40), (255, 100), (40, 120)])
def test_list_path_in_fp16(gpu, metric, nq, k):
    # batches of 17..255 queries (and other list-path cases) over at least 65,536 rows of
    # 128 dims take the per-split lists in fp16 (each list capacity: k' = k + 8 of 32, 56,
    # 120 and 128); results bit-identical to the oracle and to the fp32 lists
    data = datagen.sift_like(120_000, 128, 781)
    q = datagen.sift_like(nq, 128, 782)
    idx = _index(data, metric)
    print(f"case lists fp16 nq={nq} k={k} metric={metric}", flush=True)
    ids, d, info = _run(idx, q, k)
    assert info["path"] == "lists" and info["scan_f16"], info
    o_ids, o_d, _ = oracle.flat_search(data, q, k, metric)
    assert np.array_equal(ids, o_ids)
    assert np.array_equal(d.view(np.uint32), o_d.view(np.uint32))
    idx._scan_f16(False)
    ids32, d32, info32 = _run(idx, q, k)
    assert info32["path"] == "lists" and not info32["scan_f16"]
    assert _same(ids, d, ids32, d32)


def test_list_path_in_fp16_filtered_and_fallback(gpu):
    data = datagen.sift_like(100_000, 128, 791)
    q = datagen.sift_like(64, 128, 792)
    mask = datagen.mask(100_000, 0.7, 793)
    idx = _index(data, oracle.L2)
    print("case lists fp16 filtered", flush=True)
    ids, d, info = _run(idx, q, 10, mask)
    assert info["path"] == "lists" and info["scan_f16"]
    o_ids, o_d, _ = oracle.flat_search(data, q, 10, oracle.L2, mask=mask)
    assert np.array_equal(ids, o_ids) and np.array_equal(d.view(np.uint32), o_d.view(np.uint32))
    # queries not exact in fp16: the fp32 lists
    qf = (q + 0.25).astype(np.float32)
    qf[3, 7] += 0.001
    ids, d, info = _run(idx, qf, 10)
    assert info["path"] == "lists" and not info["scan_f16"]
    o_ids, o_d, _ = oracle.flat_search(data, qf, 10, oracle.L2)
    assert_parity(ids, d, o_ids, o_d, _key_of(data, qf, oracle.L2))
    # fewer than 65,536 rows: the lists stay on fp32 (the exactness check would cost what
    # the fp16 scan saves)
    small = _index(data[:50_000], oracle.L2)
    _, _, info = _run(small, q, 10)
    assert info["path"] == "lists" and not info["scan_f16"]


def test_list_path_fp16_device_nonfinite(gpu):
    # the device form's finiteness check is answered by the fp16 pass's read-back on this
    # path: a NaN or infinite query still fails with PX_ERR_NONFINITE, outputs unwritten
    import ctypes
    from proxima_amd import _lib
    lib = _lib.load()
    nq, k = 200, 10
    data = datagen.sift_like(80_000, 128, 801)
    q = datagen.sift_like(nq, 128, 802)
    idx = _index(data, oracle.L2)
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
        for bad in (np.nan, np.inf):
            qb = q.copy()
            qb[nq // 2, 17] = bad
            print(f"case fp16 lists device nonfinite {bad}", flush=True)
            rc = lib.px_flat_search_device(idx._h, dev(qb), nq, k, None, di, dd)
            assert rc == _lib.PX_ERR_NONFINITE, (rc, _lib.last_error())
            got_i = np.empty_like(sentinel_i)
            assert lib.px_dev_download(got_i.ctypes.data, di, got_i.nbytes) == 0
            assert np.array_equal(got_i, sentinel_i)
        assert lib.px_flat_search_device(idx._h, dev(q), nq, k, None, di, dd) == 0, _lib.last_error()
        assert idx._last_timing()["path"] == "lists" and idx._last_timing()["scan_f16"]
        ids = np.empty_like(sentinel_i)
        assert lib.px_dev_download(ids.ctypes.data, di, ids.nbytes) == 0
        o_ids, _, _ = oracle.flat_search(data, q, k, oracle.L2)
        assert np.array_equal(ids, o_ids)
    finally:
        for p in ptrs:
            lib.px_dev_free(p)


def test_knn_seam_and_reload_in_fp16(gpu, tmp_path):
    # the reference's C seam (knn_gpu_create / knn_gpu_search, raw keys, metric per call)
    # and a FlatIndex saved and loaded again both keep the fp16 copy of exact rows: raw
    # keys equal to the oracle's for both metrics on one handle, and a reloaded index's
    # search takes the fp16 scan with the same results
    from proxima_amd import _lib
    lib = _lib.load()
    data = datagen.sift_like(70_000, 128, 811)
    q = datagen.sift_like(300, 128, 812)
    k = 10
    g = lib.knn_gpu_create(_lib.f32p(data), 70_000, 128)
    assert g
    try:
        for metric in (oracle.L2, oracle.IP):
            print(f"case knn seam fp16 metric={metric}", flush=True)
            ids = np.zeros((300, k), dtype=np.int64)
            keys = np.zeros((300, k), dtype=np.float32)
            rc = lib.knn_gpu_search(g, _lib.f32p(q), 300, k, metric, _lib.i64p(ids), _lib.f32p(keys))
            assert rc == 0, _lib.last_error()
            o_ids, _, o_keys = oracle.flat_search(data, q, k, metric)
            assert np.array_equal(ids, o_ids)
            assert np.array_equal(keys, o_keys)
    finally:
        lib.knn_gpu_free(g)
    idx = _index(data, oracle.L2)
    path = str(tmp_path / "flat.sfidx")
    idx.save(path)
    back = FlatIndex.load(path)
    print("case reloaded index fp16", flush=True)
    ids, d, info = _run(back, q, 100)
    assert info["scan_f16"]
    ids0, d0, _ = _run(idx, q, 100)
    assert _same(ids, d, ids0, d0)


def test_padded_dims_and_large_integers(gpu):
    # 125 dims pad to 128 with zero columns (exact in fp16): the copy and both scans hold
    rng = np.random.default_rng(821)
    d125 = rng.integers(0, 256, size=(80_000, 125)).astype(np.float32)
    q125 = rng.integers(0, 256, size=(400, 125)).astype(np.float32)
    idx = _index(d125, oracle.L2)
    for k, nq in ((100, 400), (10, 100)):
        print(f"case 125 dims k={k} nq={nq}", flush=True)
        ids, d, info = _run(idx, q125[:nq], k)
        assert info["scan_f16"]
        o_ids, o_d, _ = oracle.flat_search(d125, q125[:nq], k, oracle.L2)
        assert np.array_equal(ids, o_ids)
        assert np.array_equal(d.view(np.uint32), o_d.view(np.uint32))
    # integers up to 2047 are exact in fp16, but their sums pass 2^24: fp32 accumulation
    # rounds, in the fp16 MFMA's order as in the fp32 one's -- the parity rule, with its
    # near-tie exemption, as for any rounded data
    big = rng.integers(0, 2048, size=(70_000, 128)).astype(np.float32)
    qb = rng.integers(0, 2048, size=(300, 128)).astype(np.float32)
    for metric in (oracle.L2, oracle.IP):
        idx = _index(big, metric)
        print(f"case integers to 2047 metric={metric}", flush=True)
        ids, d, info = _run(idx, qb, 50)
        assert info["scan_f16"]
        o_ids, o_d, _ = oracle.flat_search(big, qb, 50, metric)
        assert_parity(ids, d, o_ids, o_d, _key_of(big, qb, metric))


# values at the edges of "exact in fp16" (zero, or a normal fp16 number: magnitude in
# [2^-14, 65504] with at most 11 significant bits), and just past them
_EDGE_EXACT = {
    "-0.0": -0.0,
    "2^-14, the smallest normal": 2.0 ** -14,
    "2^-14 (1 + 2^-10), its last significant bit": 2.0 ** -14 * (1 + 2.0 ** -10),
    "65504, the largest": 65504.0,
    "-65504": -65504.0,
}
_EDGE_INEXACT = {
    "1 + 2^-11, twelve significant bits": 1 + 2.0 ** -11,
    "65520, rounds past 65504": 65520.0,
    "65536 = 2^16": 65536.0,
    "2^-15, an fp16 subnormal": 2.0 ** -15,
}


def test_exactness_edges(gpu):
    edges = {**_EDGE_EXACT, **_EDGE_INEXACT}
    # the table itself against numpy's fp16: round trip, and not subnormal
    for name, v in edges.items():
        v32 = np.float32(v)
        with np.errstate(over="ignore"):  # 65520 and 65536 become fp16 infinities
            r = np.float16(v32).astype(np.float32)
        fits = bool(r == v32) and (v32 == 0 or abs(v32) >= 2.0 ** -14)
        assert fits == (name in _EDGE_EXACT), name
    rng = np.random.default_rng(851)
    base = rng.integers(0, 256, size=(40_000, 128)).astype(np.float32)
    q = rng.integers(0, 256, size=(1000, 128)).astype(np.float32)
    k = 100
    # one edge value in one row of an integer corpus (the copy is made on the device)
    for name, v in edges.items():
        data = base.copy()
        data[17, 3] = v
        idx = _index(data, oracle.L2)
        ids, d, info = _run(idx, q[:400], k)
        print(f"case row edge {name}: path {info['path']}, f16 {info['scan_f16']}", flush=True)
        assert info["path"].startswith("collect")
        assert info["scan_f16"] == (name in _EDGE_EXACT), name
        o_ids, o_d, _ = oracle.flat_search(data, q[:400], k, oracle.L2)
        assert_parity(ids, d, o_ids, o_d, _key_of(data, q[:400], oracle.L2))
    # one edge value in the last query of a batch: 400 x 128 values are tested on the
    # host, 1000 x 128 on the device
    idx = _index(base, oracle.L2)
    for nq in (400, 1000):
        for name, v in edges.items():
            qq = q[:nq].copy()
            qq[nq - 1, 5] = v
            ids, d, info = _run(idx, qq, k)
            print(f"case query edge {name}, nq={nq}: path {info['path']}, f16 {info['scan_f16']}",
                  flush=True)
            assert info["path"].startswith("collect")
            assert info["scan_f16"] == (name in _EDGE_EXACT), (name, nq)
            o_ids, o_d, _ = oracle.flat_search(base, qq, k, oracle.L2)
            assert_parity(ids, d, o_ids, o_d, _key_of(base, qq, oracle.L2))


def test_exactness_edges_on_the_lists(gpu):
    # the per-split lists (200 queries, k = 10, 80,000 rows): host arrays are tested on the
    # host, the device form by the lists' own pass (finiteness and fp16 exactness in one
    # read-back)
    import ctypes
    from proxima_amd import _lib
    lib = _lib.load()
    nq, k = 200, 10
    data = datagen.sift_like(80_000, 128, 861)
    q = datagen.sift_like(nq, 128, 862)
    idx = _index(data, oracle.L2)
    ptrs = []

    def dev(arr):
        p = ctypes.c_void_p()
        assert lib.px_dev_alloc(ctypes.byref(p), max(arr.nbytes, 1)) == 0
        ptrs.append(p)
        assert lib.px_dev_upload(p, arr.ctypes.data, arr.nbytes) == 0
        return p

    try:
        di = dev(np.zeros((nq, k), dtype=np.int64))
        dd = dev(np.zeros((nq, k), dtype=np.float32))
        for name, v in {**_EDGE_EXACT, **_EDGE_INEXACT}.items():
            qq = q.copy()
            qq[nq - 1, 9] = v
            o_ids, o_d, _ = oracle.flat_search(data, qq, k, oracle.L2)
            ids, d, info = _run(idx, qq, k)
            print(f"case lists query edge {name}: host f16 {info['scan_f16']}", flush=True)
            assert info["path"] == "lists" and info["scan_f16"] == (name in _EDGE_EXACT), name
            assert_parity(ids, d, o_ids, o_d, _key_of(data, qq, oracle.L2))
            rc = lib.px_flat_search_device(idx._h, dev(qq), nq, k, None, di, dd)
            assert rc == 0, _lib.last_error()
            info = idx._last_timing()
            print(f"  device form f16 {info['scan_f16']}", flush=True)
            assert info["path"] == "lists" and info["scan_f16"] == (name in _EDGE_EXACT), name
            ids = np.empty((nq, k), dtype=np.int64)
            d = np.empty((nq, k), dtype=np.float32)
            assert lib.px_dev_download(ids.ctypes.data, di, ids.nbytes) == 0
            assert lib.px_dev_download(d.ctypes.data, dd, d.nbytes) == 0
            assert_parity(ids, d, o_ids, o_d, _key_of(data, qq, oracle.L2))
    finally:
        for p in ptrs:
            lib.px_dev_free(p)
