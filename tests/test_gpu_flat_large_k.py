"""GPU parity of the threshold-collect and full-sort paths of FlatIndex searches.

The reference's FlatIndex takes any k (flat.rs:106-148 keeps a heap of k); so does the
library: up to PX_MAX_K on the fused scans, past it by sorting every key. For k' = k + 8
past 128, and for k >= 16 in batches of at least 256 queries where the lists do not win
(the lists keep k' <= 56 on rows of more than 128 padded dims below 262,144 rows, and on
rows of at most 128 padded dims while n_eff * (k' - 16) < 1.04M), it samples a subset of
the rows spread evenly over the corpus for per-query thresholds, appends every row at or
below them in one collect scan, and finishes each query whose candidate set is complete
and large enough; the others go round again with a looser or tighter threshold.
Unfiltered batches of at least 256 queries with k + 8 <= 24 on rows of at most 128 padded
dims over at most 48 splits take no sample: their first round is bounded by the splits'
shared bound alone. These tests compare with the oracle at the parity rule, bit for bit
on integer-valued data (exact in fp32) and on the full-sort path, and force each kind of
extra round with data laid out against the sample or the bound.
"""
import ctypes

import numpy as np
import pytest

import oracle
from conftest import assert_parity, sample_positions
from proxima_amd import FlatIndex, Metric, _lib, datagen

pytestmark = pytest.mark.gpu


def _key_of(data, queries, metric):
    def key_of(qi, row):
        if metric == oracle.L2:
            return float(oracle.l2_sqr(queries[qi], data[row]))
        return float(-oracle.inner_product(queries[qi], data[row]))
    return key_of


def _rounds(idx) -> int:
    r = ctypes.c_int(-1)
    assert idx._lib.px_flat_last_rounds(idx._h, ctypes.byref(r)) == 0
    return r.value


def _search(data, queries, k, metric, mask=None):
    idx = FlatIndex(data.shape[1], Metric.L2 if metric == oracle.L2 else Metric.InnerProduct)
    idx.add(data)
    if mask is None:
        ids, d = idx.search_batch(queries, k=k)
    else:
        ids, d = idx.search_batch_filtered(queries, mask, k=k)
    return idx, ids, d


def _check(data, queries, k, metric, mask=None, exact=False):
    print(f"case n={data.shape[0]} dim={data.shape[1]} nq={queries.shape[0]} k={k} "
          f"metric={metric} mask={'yes' if mask is not None else 'no'}", flush=True)
    idx, ids, d = _search(data, queries, k, metric, mask)
    o_ids, o_d, _ = oracle.flat_search(data, queries, k, metric, mask=mask)
    assert_parity(ids, d, o_ids, o_d, _key_of(data, queries, metric), allow_exempt=not exact)
    if exact:
        assert np.array_equal(ids, o_ids)
        assert np.array_equal(d.view(np.uint32), o_d.view(np.uint32))
    return _rounds(idx)


@pytest.mark.parametrize("k", [121, 300, 1000, 4096])
def test_sift_like_exact(gpu, k):
    data = datagen.sift_like(60_000, 128, 31)
    q = datagen.sift_like(48, 128, 32)
    rounds = _check(data, q, k, oracle.L2, exact=True)
    assert rounds >= 1


def test_first_k_past_the_lists_and_last_list_k(gpu):
    # k = 120 is the last k on the per-split lists (k' = 128), k = 121 the first collected
    data = datagen.sift_like(20_000, 96, 33)
    q = datagen.sift_like(40, 96, 34)
    for k in (120, 121):
        idx, ids, d = _search(data, q, k, oracle.L2)
        o_ids, o_d, _ = oracle.flat_search(data, q, k, oracle.L2)
        assert np.array_equal(ids, o_ids) and np.array_equal(d, o_d), k
        assert (_rounds(idx) == 0) == (k == 120)


def test_batch_routing_boundary(gpu):
    # batches of >= 256 queries switch from the per-split lists to the collect path at k = 16,
    # except that with one 128-dim query chunk k' = k + 8 <= 56 stays on the lists while
    # n_eff (k' - 16) < 1,040,000 (30,000 rows: k' <= 50)
    data = datagen.sift_like(30_000, 64, 49)
    q = datagen.sift_like(300, 64, 50)
    for k, collected in ((15, False), (16, False), (42, False), (43, True), (48, True),
                         (49, True), (100, True)):
        idx, ids, d = _search(data, q, k, oracle.L2)
        o_ids, o_d, _ = oracle.flat_search(data, q, k, oracle.L2)
        assert np.array_equal(ids, o_ids) and np.array_equal(d, o_d), k
        assert (_rounds(idx) > 0) == collected, k


@pytest.mark.parametrize("dim,k,collected", [(64, 17, False), (64, 33, False), (64, 34, True),
                                             (64, 48, True), (200, 17, False), (200, 48, False)])
def test_routing_by_rows_and_chunks(gpu, dim, k, collected):
    # 40,000 rows: with one query chunk the lists keep k' while 40,000 (k' - 16) < 1,040,000
    # (k' <= 41), with two chunks up to k' = 56
    data = datagen.sift_like(40_000, dim, 61)
    q = datagen.sift_like(300, dim, 62)
    idx, ids, d = _search(data, q, k, oracle.L2)
    o_ids, o_d, _ = oracle.flat_search(data, q, k, oracle.L2)
    assert np.array_equal(ids, o_ids) and np.array_equal(d, o_d)
    assert (_rounds(idx) > 0) == collected


@pytest.mark.parametrize("metric", [oracle.L2, oracle.IP])
@pytest.mark.parametrize("k", [16, 37, 100])
def test_collect_moderate_k(gpu, metric, k):
    data = datagen.gaussian(25_000, 72, 53)
    q = datagen.gaussian(260, 72, 54)
    _check(data, q, k, metric)


def test_collect_filtered_two_chunks_config5_shape(gpu):
    # the 10M x 384 unit-Gaussian IP workload's shape on 60,000 rows, 10% mask, k = 100
    data = datagen.unit_gaussian(60_000, 384, 55)
    q = datagen.unit_gaussian(300, 384, 56)
    mask = datagen.mask(60_000, 0.1, 57)
    _check(data, q, 100, oracle.IP, mask=mask)


def test_ip_filtered_two_chunks(gpu):
    # dim 200: two 128-dim query chunks; 30% of the rows kept
    data = datagen.gaussian(40_000, 200, 35)
    q = datagen.gaussian(32, 200, 36)
    mask = datagen.mask(40_000, 0.3, 37)
    _check(data, q, 500, oracle.IP, mask=mask)


def test_l2_gaussian_unfiltered_odd_dim(gpu):
    data = datagen.gaussian(30_000, 61, 38)
    q = datagen.gaussian(300, 61, 39)
    _check(data, q, 256, oracle.L2)


def test_k_above_rows_pads(gpu):
    # every row is a candidate: all 900 rows in order, then padding
    data = datagen.sift_like(900, 32, 40)
    q = datagen.sift_like(20, 32, 41)
    _check(data, q, 2000, oracle.L2, exact=True)
    mask = datagen.mask(900, 0.5, 42)
    _check(data, q, 700, oracle.L2, mask=mask, exact=True)


def test_exact_ties_lower_row_wins(gpu):
    # 25 distinct rows repeated: thousands of exactly equal keys; ties go to the lower row
    base = datagen.sift_like(25, 64, 43)
    data = np.tile(base, (1200, 1))
    q = datagen.sift_like(16, 64, 44)
    _check(data, q, 700, oracle.L2, exact=True)


def test_sample_far_overflow_round(gpu):
    # The sampled rows are far from every query and the rest are near: the sample's
    # threshold lets nearly every row through, the select overflows, and later rounds
    # tighten the threshold from the candidates.
    n, k = 40_000, 992
    sampled = sample_positions(n, k + 8)
    rng = np.random.default_rng(45)
    data = rng.integers(0, 4, size=(n, 48)).astype(np.float32)
    data[sampled] = 255.0
    q = rng.integers(0, 3, size=(12, 48)).astype(np.float32)
    rounds = _check(data, q, k, oracle.L2, exact=True)
    assert rounds >= 2


@pytest.mark.parametrize("dim", [200, 384])
def test_resident_query_collect_overflow_rounds(gpu, dim):
    # the far-overflow layout on rows of 129-384 padded dims, whose collect scan holds the
    # queries in registers (four lanes a query, a pair of them sharing each region): every
    # region overflows in the first round and the retry rounds list their queries; dim 200
    # ends on a partial 128-dim chunk, 384 is three full ones
    n, k = 40_000, 992
    sampled = sample_positions(n, k + 8)
    rng = np.random.default_rng(47)
    data = rng.integers(0, 4, size=(n, dim)).astype(np.float32)
    data[sampled] = 255.0
    q = rng.integers(0, 3, size=(40, dim)).astype(np.float32)
    idx, ids, d = _search(data, q, k, oracle.L2)
    o_ids, o_d, _ = oracle.flat_search(data, q, k, oracle.L2)
    assert np.array_equal(ids, o_ids) and np.array_equal(d, o_d)
    assert idx._last_timing()["path"] == "collect-sampled"
    assert _rounds(idx) >= 2


def test_sample_near_underflow_rounds(gpu):
    # The sampled rows are the near ones: the sample's thresholds admit too few rows, the
    # ladder runs out, and the query finishes from an unbounded round.
    n, k = 40_000, 992
    sampled = sample_positions(n, k + 8)
    rng = np.random.default_rng(46)
    data = rng.integers(200, 256, size=(n, 48)).astype(np.float32)
    data[sampled] = rng.integers(0, 4, size=(sampled.size, 48))
    q = rng.integers(0, 3, size=(12, 48)).astype(np.float32)
    rounds = _check(data, q, k, oracle.L2, exact=True)
    assert rounds >= 3


def _overflow_rows(n, kk, key_index):
    """Rows of 128 dims whose L2 key from the origin is key_index(p) + 1 (one nonzero
    coordinate, its square root), the threshold sample's rows far away: the sample lets
    every other row through and every region of the first round overflows."""
    data = np.zeros((n, 128), np.float32)
    data[:, 0] = np.sqrt(key_index(np.arange(n)) + 1.0).astype(np.float32)
    data[sample_positions(n, kk), 0] = 1000.0
    return data


def test_overflow_with_near_rows_dropped_goes_round_again(gpu):
    # keys grow with the position: each region keeps its first rows, and the rows it drops
    # in the first splits are nearer than the k'-th kept row of the later splits, so the
    # query tightens and goes round again
    n, k, nq = 40_000, 992, 64
    data = _overflow_rows(n, k + 8, lambda p: p.astype(np.float64))
    q = np.zeros((nq, 128), np.float32)
    rounds = _check(data, q, k, oracle.L2, exact=True)
    assert rounds >= 2


def test_overflow_with_far_rows_dropped_finishes(gpu):
    # keys grow with the position within each split of the first round's scan (a sawtooth
    # of the split's length): each region keeps its own nearest rows and drops only rows
    # beyond the k'-th smallest kept one, so the query finishes in the first round
    n, k, nq = 40_000, 992, 64
    q = np.zeros((nq, 128), np.float32)
    # the scan's split length, from a search of the same shape
    idx, _, _ = _search(_overflow_rows(n, k + 8, lambda p: p.astype(np.float64)), q, k,
                        oracle.L2)
    t = idx._last_timing()
    assert t["path"] == "collect-sampled"
    splits = t["splits"]
    rps = [r for r in range(64, n + 64, 64) if -(-n // r) == splits]
    assert len(rps) == 1, rps
    rps = rps[0]
    data = _overflow_rows(n, k + 8, lambda p: (p % rps) + 1e-3 * (p // rps))
    rounds = _check(data, q, k, oracle.L2, exact=True)
    assert rounds == 1


def test_sample_short_of_its_last_split(gpu):
    # 10,000 rows at k = 100 sample 7,407 rows, which leave the sample scan's last split
    # four 64-row tiles short of its layout. Those key blocks are never written and must
    # not count as sampled keys: zeros or an earlier search's candidate keys there make
    # every threshold too tight and cost extra rounds. Two searches in a row on one
    # handle, each exact and finished in one round.
    data = datagen.gaussian(10_000, 128, 61)
    q = datagen.gaussian(300, 128, 62)
    k = 100
    print(f"case n=10000 dim=128 nq=300 k={k} L2, twice", flush=True)
    idx = FlatIndex(128, Metric.L2)
    idx.add(data)
    o_ids, o_d, _ = oracle.flat_search(data, q, k, oracle.L2)
    for _ in range(2):
        ids, d = idx.search_batch(q, k=k)
        assert_parity(ids, d, o_ids, o_d, _key_of(data, q, oracle.L2))
        assert _rounds(idx) == 1


def test_sift_1m_subset(gpu):
    # the 1M x 128 SIFT-like corpus, 16 of its queries, k = 1000
    data = datagen.corpus(3)
    q = datagen.queries(3)[:16]
    _check(data, q, 1000, oracle.L2, exact=True)


def test_knn_seam_raw_keys(gpu):
    lib = _lib.load()
    data = datagen.sift_like(5000, 40, 47)
    q = datagen.sift_like(9, 40, 48)
    k = 300
    g = lib.knn_gpu_create(_lib.f32p(data), 5000, 40)
    assert g
    try:
        ids = np.zeros((9, k), dtype=np.int64)
        keys = np.zeros((9, k), dtype=np.float32)
        rc = lib.knn_gpu_search(g, _lib.f32p(q), 9, k, 0, _lib.i64p(ids), _lib.f32p(keys))
        assert rc == 0, _lib.last_error()
    finally:
        lib.knn_gpu_free(g)
    o_ids, _, o_keys = oracle.flat_search(data, q, k, oracle.L2)
    assert np.array_equal(ids, o_ids)
    assert np.array_equal(keys, o_keys)


def test_k_limit(gpu):
    # k = PX_MAX_K is the last k of the threshold-collect path; past it, every key is
    # computed in the reference's arithmetic and sorted
    idx = FlatIndex(8, Metric.L2)
    idx.add(np.zeros((10, 8), dtype=np.float32))
    for k in (_lib.PX_MAX_K, _lib.PX_MAX_K + 1):
        ids, d = idx.search(np.zeros(8, dtype=np.float32), k=k)
        assert ids.shape == (k,)
        assert np.array_equal(ids[:10], np.arange(10)) and (ids[10:] == -1).all()
        # (one query: the vector-ALU collect scan up to PX_MAX_K)
        assert _path(idx) == ("vector" if k == _lib.PX_MAX_K else "full-sort")


@pytest.mark.parametrize("metric", [oracle.L2, oracle.IP])
def test_full_sort_past_max_k(gpu, metric):
    # k past PX_MAX_K: the keys are the reference's own arithmetic, so ids and distances
    # equal the oracle's bit for bit (ties to the lower row), filtered or not, k above the
    # rows padded
    data = datagen.gaussian(12_000, 40, 73)
    q = datagen.gaussian(20, 40, 74)
    mask = datagen.mask(12_000, 0.5, 75)
    for k, m in ((5000, None), (5000, mask), (13_000, None)):
        print(f"case full sort n=12000 k={k} metric={metric} mask={m is not None}", flush=True)
        idx, ids, d = _search(data, q, k, metric, m)
        assert _path(idx) == "full-sort"
        o_ids, o_d, _ = oracle.flat_search(data, q, k, metric, mask=m)
        assert np.array_equal(ids, o_ids)
        assert np.array_equal(d.view(np.uint32), o_d.view(np.uint32))


def test_full_sort_ties_and_chunks(gpu, tmp_path):
    # 25 distinct rows repeated (exactly equal keys: the lower row first) with a 4 MB budget,
    # so the queries are sorted in several chunks
    import os
    import subprocess
    import sys
    script = tmp_path / "run.py"
    script.write_text(f"""
import sys
sys.path.insert(0, {repr(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))})
import numpy as np
import oracle
from proxima_amd import FlatIndex, Metric, datagen
base = datagen.sift_like(25, 32, 76)
data = np.tile(base, (800, 1))
q = datagen.sift_like(40, 32, 77)
idx = FlatIndex(32, Metric.L2)
idx.add(data)
ids, d = idx.search_batch(q, k=6000)
assert idx._last_timing()["path"] == "full-sort"
o_ids, o_d, _ = oracle.flat_search(data, q, 6000, oracle.L2)
assert np.array_equal(ids, o_ids) and np.array_equal(d, o_d)
print("ok")
""")
    env = dict(os.environ, PX_COLLECT_BYTES=str(4 << 20))
    out = subprocess.run([sys.executable, str(script)], capture_output=True, text=True,
                         timeout=240, env=env)
    assert out.returncode == 0, out.stdout[-2000:] + out.stderr[-2000:]
    assert out.stdout.strip().endswith("ok")


def test_more_queries_than_one_collect_batch(gpu):
    # 17,000 queries: two collect batches of at most 16,384 (k' = 68 > 56: collected on
    # 2,000 rows)
    data = datagen.sift_like(2000, 16, 58)
    q = datagen.sift_like(17_000, 16, 59)
    rounds = _check(data, q, 60, oracle.L2, exact=True)
    assert rounds >= 1


@pytest.mark.parametrize("dim", [48, 384])
def test_retry_rounds_in_memory_bounded_chunks(gpu, tmp_path, dim):
    # The overflow layout of test_sample_far_overflow_round with 300 queries and a 1 MB
    # budget for the candidate regions: each retry round runs in several chunks of queries
    # (dim 384: the collect scan with the queries resident in registers).
    import os
    import subprocess
    import sys
    script = tmp_path / "run.py"
    script.write_text(f"""
import sys
sys.path.insert(0, {repr(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))})
sys.path.insert(0, {repr(os.path.dirname(os.path.abspath(__file__)))})
import numpy as np
import oracle
from proxima_amd import FlatIndex, Metric, datagen
n, k = 40_000, 992
s = max(1, min(n, 16384, 80 * n // (k + 8)))
rng = np.random.default_rng(45)
data = rng.integers(0, 4, size=(n, {dim})).astype(np.float32)
data[np.arange(s) * n // s] = 255.0  # the sampled positions, floor(i * n / s)
q = rng.integers(0, 3, size=(300, {dim})).astype(np.float32)
idx = FlatIndex({dim}, Metric.L2)
idx.add(data)
ids, d = idx.search_batch(q, k=k)
o_ids, o_d, _ = oracle.flat_search(data, q, k, oracle.L2)
assert np.array_equal(ids, o_ids) and np.array_equal(d, o_d)
import ctypes
r = ctypes.c_int(-1)
assert idx._lib.px_flat_last_rounds(idx._h, ctypes.byref(r)) == 0 and r.value >= 2, r.value
print("ok", r.value)
""")
    env = dict(os.environ, PX_COLLECT_BYTES=str(1 << 20))
    out = subprocess.run([sys.executable, str(script)], capture_output=True, text=True,
                         timeout=240, env=env)
    assert out.returncode == 0, out.stdout[-2000:] + out.stderr[-2000:]
    assert out.stdout.strip().startswith("ok")



def _path(idx) -> str:
    return idx._last_timing()["path"]


def test_bound_only_first_round(gpu):
    # k' <= 24 on batches of 256+ queries of at most 128 dims over at most 48 splits (here
    # 40,000 rows and 2,048 queries: 32 splits): the first round takes no sample; each
    # split's first tile and the splits' shared bound decide what is collected
    data = datagen.sift_like(40_000, 64, 63)
    q = datagen.sift_like(2048, 64, 64)
    mask = datagen.mask(40_000, 0.5, 65)
    for k in (1, 10, 16):
        for m in (None, mask):
            idx, ids, d = _search(data, q, k, oracle.L2, m)
            # filtered rows of 64 dims keep the lists at these k (the shared bound of a
            # filtered scan is compiled into the 128-dim collect scan only)
            assert _path(idx) == ("collect-bounded" if m is None else "lists"), k
            o_ids, o_d, _ = oracle.flat_search(data, q, k, oracle.L2, mask=m)
            assert np.array_equal(ids, o_ids) and np.array_equal(d, o_d), k
    # k' = 25 is past the rule, and 40,000 rows are too few for a threshold sample to pay:
    # the per-split lists
    idx, ids, d = _search(data, q, 17, oracle.L2)
    assert _path(idx) == "lists"
    o_ids, o_d, _ = oracle.flat_search(data, q, 17, oracle.L2)
    assert np.array_equal(ids, o_ids) and np.array_equal(d, o_d)
    gd = datagen.unit_gaussian(40_000, 96, 66)
    gq = datagen.unit_gaussian(2048, 96, 67)
    _check(gd, gq, 12, oracle.IP)


@pytest.mark.parametrize("rows,density", [(80_000, 0.5), (400_000, 0.1)])
def test_bound_only_filtered_128_dims(gpu, rows, density):
    # filtered rows of exactly 128 padded dims take the bounded first round too (the shared
    # bound over the kept rows' positions): about 40,000 kept rows and 2,048 queries, the
    # 32 splits of the unfiltered case above
    data = datagen.sift_like(rows, 128, 91)
    q = datagen.sift_like(2048, 128, 92)
    mask = datagen.mask(rows, density, 93)
    for k in (1, 10, 16):
        print(f"case bounded filtered rows={rows} density={density} k={k}", flush=True)
        idx, ids, d = _search(data, q, k, oracle.L2, mask)
        assert _path(idx) == "collect-bounded", k
        o_ids, o_d, _ = oracle.flat_search(data, q, k, oracle.L2, mask=mask)
        assert np.array_equal(ids, o_ids) and np.array_equal(d, o_d), k
    gd = datagen.unit_gaussian(rows, 128, 94)
    gq = datagen.unit_gaussian(2048, 128, 95)
    idx, ids, d = _search(gd, gq, 10, oracle.IP, mask)
    assert _path(idx) == "collect-bounded"
    o_ids, o_d, _ = oracle.flat_search(gd, gq, 10, oracle.IP, mask=mask)
    assert_parity(ids, d, o_ids, o_d, _key_of(gd, gq, oracle.IP))


def test_bound_only_overflow_and_ties(gpu):
    # Keys fall along the rows (each tile nearer than the last), so the shared bound
    # prunes little in the last splits, their regions overflow and retry rounds tighten the
    # threshold from the candidates; only 512 distinct keys, so ties at the bound decide
    # by row.
    n = 40_000
    data = np.zeros((n, 16), dtype=np.float32)
    data[:, 0] = 255 - (np.arange(n) * 255) // n
    data[:, 3] = np.arange(n) % 2
    rng = np.random.default_rng(69)
    q = np.zeros((2048, 16), dtype=np.float32)
    q[:, 0] = rng.integers(0, 4, size=2048)
    idx, ids, d = _search(data, q, 16, oracle.L2)
    assert _path(idx) == "collect-bounded"
    o_ids, o_d, _ = oracle.flat_search(data, q, 16, oracle.L2)
    assert np.array_equal(ids, o_ids) and np.array_equal(d, o_d)
    assert _rounds(idx) >= 2


def test_bound_only_consecutive_searches(gpu):
    # The shared-bound slots are refilled with +inf before every launch, which no longer
    # waits for the stream to drain. Five searches in a row on one handle, the query sets
    # alternating (a stale slot of the other set would drop true neighbours), each exact.
    data = datagen.sift_like(40_000, 64, 70)
    qa = datagen.sift_like(2048, 64, 71)
    qb = datagen.sift_like(2048, 64, 72) // 4
    idx = FlatIndex(64, Metric.L2)
    idx.add(data)
    ref = {}
    for name, q in (("a", qa), ("b", qb)):
        ref[name] = oracle.flat_search(data, q, 10, oracle.L2)[:2]
    for name in "abbab":
        q = qa if name == "a" else qb
        print(f"case consecutive search {name}", flush=True)
        ids, d = idx.search_batch(q, k=10)
        assert _path(idx) == "collect-bounded"
        assert np.array_equal(ids, ref[name][0]) and np.array_equal(d, ref[name][1]), name


@pytest.mark.parametrize("n,nq,dim,k,metric,dist", [
    (40_000, 2048, 96, 16, oracle.IP, "unit"),
    (25_000, 4096, 24, 5, oracle.L2, "gauss"),
    (33_000, 1500, 128, 12, oracle.L2, "sift"),
    (40_000, 2048, 8, 1, oracle.L2, "gauss"),
    (33_000, 1500, 61, 10, oracle.IP, "gauss"),
])
def test_bound_only_shapes(gpu, n, nq, dim, k, metric, dist):
    # shapes that take the bounded first round: 16-40 splits, odd and padded dims, k = 1-16
    gen = {"unit": datagen.unit_gaussian, "gauss": datagen.gaussian, "sift": datagen.sift_like}[dist]
    data = gen(n, dim, 80 + dim)
    q = gen(nq, dim, 81 + dim)
    idx, ids, d = _search(data, q, k, metric)
    print(f"case bounded n={n} nq={nq} dim={dim} k={k} metric={metric} {dist}", flush=True)
    assert _path(idx) == "collect-bounded"
    o_ids, o_d, _ = oracle.flat_search(data, q, k, metric)
    if dist == "sift":
        assert np.array_equal(ids, o_ids) and np.array_equal(d, o_d)
    else:
        assert_parity(ids, d, o_ids, o_d, _key_of(data, q, metric))


def test_bound_only_batch_then_sampled_batch(gpu):
    # 17,000 queries run as two collect batches: 16,384 over 16 splits take the bounded first
    # round (k' = 16), the last 616 over 85 splits a sampled one; exact either way
    data = datagen.sift_like(200_000, 16, 90)
    q = datagen.sift_like(17_000, 16, 91)
    print("case two batches, bounded then sampled", flush=True)
    rounds = _check(data, q, 8, oracle.L2, exact=True)
    assert rounds >= 1


def test_bound_only_ip_ties(gpu):
    # inner product on 40 distinct unit rows repeated: exactly equal keys across every split;
    # ties at the bound and in the result go to the lower row
    base = datagen.unit_gaussian(40, 32, 92)
    data = np.tile(base, (1000, 1))
    q = datagen.unit_gaussian(2048, 32, 93)
    idx, ids, d = _search(data, q, 12, oracle.IP)
    print("case bounded IP ties", flush=True)
    assert _path(idx) == "collect-bounded"
    o_ids, o_d, _ = oracle.flat_search(data, q, 12, oracle.IP)
    assert np.array_equal(ids, o_ids) and np.array_equal(d, o_d)
