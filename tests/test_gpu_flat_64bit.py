"""GPU parity past 2^31 corpus elements: the inner-product workload of 10,000,000 x 384
unit-normalised Gaussian rows (16,384 queries, k = 100, 10%-density filter) on its first
5,600,000 rows, 2,150,400,000 floats, so that every row past 5,592,405 (= 2^31 / 384)
starts beyond a 32-bit element offset. The reference indexes rows with usize
(flat.rs:124-137, every row scanned) and knn.cu:48,117,134 with size_t offsets; here the
tile loads, the row ids of a filter and the exact re-rank must all address past 2^31
elements. Each path that a search can take on these rows runs once: the MFMA collect scan
with several query chunks, unfiltered and filtered (k = 100, 300 queries), the per-split
lists (k = 10, 64 queries) and the vector-ALU scan (k = 10, 8 queries). Queries 0-19 are
copies of rows past the boundary, so that their nearest rows lie there; a sample of the
queries (the oracle scans 8.6 GB per query) is checked against the oracle at the parity
rule.
"""
import numpy as np
import pytest

import oracle
from conftest import assert_parity
from proxima_amd import FlatIndex, Metric, datagen

pytestmark = [pytest.mark.gpu, pytest.mark.timeout(300)]

ROWS, DIM = 5_600_000, 384
BOUNDARY = (1 << 31) // DIM   # rows at or past this index start beyond 2^31 elements
PLANTED = 20


@pytest.fixture(scope="module")
def big(gpu):
    print(f"generating {ROWS} x {DIM} unit-Gaussian rows ({ROWS * DIM} floats)", flush=True)
    data = datagen.corpus(5, rows=ROWS)
    assert data.size > (1 << 31) and BOUNDARY < ROWS - 1000
    q = datagen.queries(5, rows=300)
    planted_rows = ROWS - 1 - np.arange(PLANTED) * 317   # all past the boundary
    q[:PLANTED] = data[planted_rows]
    idx = FlatIndex(DIM, Metric.InnerProduct)
    idx.add(data)
    print("corpus added", flush=True)
    return data, q, planted_rows, idx


def _key_of(data, queries):
    return lambda qi, row: -float(oracle.inner_product(queries[qi], data[row]))


def _check(data, q, ids, d, sample, k, mask=None):
    o_ids, o_d, _ = oracle.flat_search(data, q[sample], k, oracle.IP, mask=mask)
    assert_parity(ids[sample], d[sample], o_ids, o_d, _key_of(data, q[sample]))


def test_collect_scan_past_2_31_elements(big):
    data, q, planted_rows, idx = big
    print("case: 300 queries, k=100, unfiltered (collect scan, 3 query chunks)", flush=True)
    ids, d = idx.search_batch(q, k=100)
    assert idx._last_timing()["path"] in ("collect-sampled", "collect-bounded")
    assert np.array_equal(ids[:PLANTED, 0], planted_rows)
    assert (ids >= BOUNDARY).sum() > PLANTED
    _check(data, q, ids, d, np.r_[0:8, 23:300:12], 100)


def test_filtered_collect_scan_past_2_31_elements(big):
    data, q, planted_rows, idx = big
    mask = datagen.config_mask(5, n=ROWS)
    mask[planted_rows] = True
    print("case: 300 queries, k=100, 10% filter (filtered collect scan)", flush=True)
    ids, d = idx.search_batch_filtered(q, mask, k=100)
    assert idx._last_timing()["path"] in ("collect-sampled", "collect-bounded")
    assert np.array_equal(ids[:PLANTED, 0], planted_rows)
    assert mask[ids[ids >= 0]].all()
    _check(data, q, ids, d, np.r_[0:8, 29:300:12], 100, mask=mask)


def test_lists_past_2_31_elements(big):
    data, q, planted_rows, idx = big
    print("case: 64 queries, k=10 (per-split lists)", flush=True)
    ids, d = idx.search_batch(q[:64], k=10)
    assert idx._last_timing()["path"] == "lists"
    assert np.array_equal(ids[:PLANTED, 0], planted_rows)
    _check(data, q[:64], ids, d, np.r_[0:64:2], 10)


def test_vector_scan_past_2_31_elements(big):
    data, q, planted_rows, idx = big
    print("case: 8 queries, k=10 (vector-ALU scan)", flush=True)
    ids, d = idx.search_batch(q[:8], k=10)
    assert idx._last_timing()["path"] == "vector"
    assert np.array_equal(ids[:, 0], planted_rows[:8])
    _check(data, q[:8], ids, d, np.arange(8), 10)
