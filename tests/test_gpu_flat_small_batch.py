"""GPU parity of few-query FlatIndex searches (the vector-ALU collect scan).

A batch of at most 16 queries over rows of at most 1,024 padded dims runs the collect path
with the corpus streamed on the vector ALUs (8 lanes per row, partial dot products summed
across the lanes) instead of the MFMA tiles, whose 32-query tiles would be nearly all
padding; the threshold sample runs the same way. These tests compare it with the oracle
(flat.rs:106-148 restated) at the parity rule and bit for bit on integer-valued data, and
check which path served the batch through the rounds diagnostic (0: per-split lists).
"""
import ctypes

import numpy as np
import pytest

import oracle
from conftest import assert_parity, sample_positions
from proxima_amd import FlatIndex, Metric, datagen

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


def _check(data, queries, k, metric, mask=None, exact=False, searches=1):
    print(f"case n={data.shape[0]} dim={data.shape[1]} nq={queries.shape[0]} k={k} "
          f"metric={metric} mask={'yes' if mask is not None else 'no'}", flush=True)
    idx = FlatIndex(data.shape[1], Metric.L2 if metric == oracle.L2 else Metric.InnerProduct)
    idx.add(data)
    o_ids, o_d, _ = oracle.flat_search(data, queries, k, metric, mask=mask)
    for _ in range(searches):
        if mask is None:
            ids, d = idx.search_batch(queries, k=k)
        else:
            ids, d = idx.search_batch_filtered(queries, mask, k=k)
        assert_parity(ids, d, o_ids, o_d, _key_of(data, queries, metric),
                      allow_exempt=not exact)
        if exact:
            assert np.array_equal(ids, o_ids)
            assert np.array_equal(d.view(np.uint32), o_d.view(np.uint32))
    return _rounds(idx)


@pytest.mark.parametrize("nq", [1, 2, 3, 5, 8])
@pytest.mark.parametrize("metric", [oracle.L2, oracle.IP])
def test_few_queries_gaussian(gpu, nq, metric):
    data = datagen.gaussian(30_000, 128, 71)
    q = datagen.gaussian(nq, 128, 72)
    assert _check(data, q, 10, metric) >= 1  # served by the collect path


@pytest.mark.parametrize("dim", [8, 40, 100, 384, 1000, 1024])
def test_dims(gpu, dim):
    # dims below one 32-float column group, not a multiple of 32, and up to the 1,024 limit
    data = datagen.gaussian(12_000, dim, 73)
    q = datagen.gaussian(4, dim, 74)
    assert _check(data, q, 10, oracle.L2) >= 1


@pytest.mark.parametrize("k", [1, 16, 100, 1000])
def test_k_range_sift_like_exact(gpu, k):
    # integer-valued rows: every key is exact in fp32, so the result is bit for bit
    data = datagen.sift_like(40_000, 128, 75)
    q = datagen.sift_like(3, 128, 76)
    assert _check(data, q, k, oracle.L2, exact=True) >= 1


def test_filtered(gpu):
    data = datagen.gaussian(50_000, 96, 77)
    q = datagen.gaussian(6, 96, 78)
    mask = datagen.mask(50_000, 0.1, 79)
    assert _check(data, q, 20, oracle.IP, mask=mask) >= 1


def test_sparse_filter_fewer_rows_than_k(gpu):
    data = datagen.gaussian(20_000, 64, 80)
    q = datagen.gaussian(2, 64, 81)
    mask = np.zeros(20_000, dtype=bool)
    mask[[5, 17, 19_999]] = True
    _check(data, q, 10, oracle.L2, mask=mask)


def test_tiny_corpus_pads(gpu):
    data = datagen.gaussian(5, 16, 82)
    q = datagen.gaussian(3, 16, 83)
    _check(data, q, 10, oracle.L2)


def test_exact_ties_lower_row_wins(gpu):
    # many rows at the same distance: the lower ids must come first, across splits
    rng = np.random.default_rng(84)
    data = rng.integers(0, 2, size=(20_000, 16)).astype(np.float32)
    q = np.zeros((2, 16), dtype=np.float32)
    _check(data, q, 50, oracle.L2, exact=True)


def test_repeated_searches_one_handle(gpu):
    # the workspace (sample keys, regions) is reused between searches
    data = datagen.gaussian(25_000, 128, 85)
    q = datagen.gaussian(7, 128, 86)
    assert _check(data, q, 10, oracle.IP, searches=3) >= 1


@pytest.mark.parametrize("nq", [9, 12, 16])
def test_up_to_16_queries(gpu, nq):
    data = datagen.gaussian(20_000, 128, 87)
    q = datagen.gaussian(nq, 128, 88)
    assert _check(data, q, 10, oracle.IP) >= 1


def test_16_queries_1024_dims(gpu):
    # the largest query block: 16 x 1,024 floats, the 64 KB of LDS
    data = datagen.gaussian(6_000, 1024, 94)
    q = datagen.gaussian(16, 1024, 95)
    assert _check(data, q, 10, oracle.L2) >= 1


def test_17_queries_use_the_lists(gpu):
    data = datagen.gaussian(20_000, 128, 92)
    q = datagen.gaussian(17, 128, 93)
    assert _check(data, q, 10, oracle.L2) == 0


def test_more_than_1024_dims_use_the_lists(gpu):
    data = datagen.gaussian(4_000, 1032, 89)
    q = datagen.gaussian(2, 1032, 90)
    assert _check(data, q, 10, oracle.L2) == 0


def test_sample_far_retry_rounds(gpu):
    # the sampled rows are far from every query and the rest are near: the first round's
    # threshold lets too many rows through and later rounds tighten it; exact on integers
    n, k = 40_000, 300
    rng = np.random.default_rng(91)
    data = rng.integers(0, 4, size=(n, 48)).astype(np.float32)
    data[sample_positions(n, k + 8)] = 255.0
    q = rng.integers(0, 3, size=(4, 48)).astype(np.float32)
    assert _check(data, q, k, oracle.L2, exact=True) >= 2
