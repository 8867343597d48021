"""GPU parity of the PqIndex ADC scan against the CPU oracle.

ADC keys are sums of LUT entries in subspace order from +0.0 (pq.rs:320-323); the GPU
builds the LUT and sums in the same order, so keys -- and therefore ids and distances --
must be bit-identical to the oracle's.
"""
import numpy as np
import pytest

import oracle
from proxima_amd import Metric, PqIndex, datagen

pytestmark = pytest.mark.gpu


def _index(data, m, nbits, metric, iters=8, sample=0, seed=24301):
    pq = PqIndex(data.shape[1], Metric.L2 if metric == oracle.L2 else Metric.InnerProduct,
                 m=m, nbits=nbits, train_iters=iters, train_sample=sample, seed=seed)
    pq.train(data)
    pq.add(data)
    return pq


@pytest.mark.parametrize("m,nbits", [(16, 8), (8, 8), (4, 6), (6, 4), (12, 3)])
@pytest.mark.parametrize("metric", [oracle.L2, oracle.IP])
def test_pq_bit_exact(gpu, m, nbits, metric):
    dim = 48
    data = datagen.gaussian(6000, dim, 100 + m)
    q = datagen.gaussian(60, dim, 200 + m)
    pq = _index(data, m, nbits, metric)
    books = pq.codebooks()
    codes = pq.codes()
    assert np.array_equal(books, oracle.pq_train(data, m, nbits, 8, 0, 24301))
    assert np.array_equal(codes, oracle.pq_encode(books, data))
    for k in (1, 10, 64):
        ids, d = pq.search_batch(q, k=k)
        o_ids, o_d, _ = oracle.pq_search(books, codes, q, k, metric)
        print(f"pq m={m} nbits={nbits} metric={metric} k={k}", flush=True)
        assert np.array_equal(ids, o_ids)
        assert np.array_equal(d, o_d)


@pytest.mark.parametrize("p", [0.0, 0.01, 0.5])
def test_pq_filtered_bit_exact(gpu, p):
    data = datagen.gaussian(20_000, 64, 5)
    q = datagen.gaussian(40, 64, 6)
    mask = datagen.mask(20_000, p, 7)
    pq = _index(data, 16, 8, oracle.L2, iters=4, sample=5000)
    ids, d = pq.search_batch_filtered(q, mask, k=10)
    o_ids, o_d, _ = oracle.pq_search(pq.codebooks(), pq.codes(), q, 10, oracle.L2, mask=mask)
    assert np.array_equal(ids, o_ids)
    assert np.array_equal(d, o_d)
    assert mask[ids[ids >= 0]].all()


def test_pq_config4_reduced(gpu):
    # the 1M x 128 N(0,1), m=16 workload on its first 200,000 rows, 100 queries, 50% mask
    data = datagen.corpus(4, rows=200_000)
    q = datagen.queries(4, rows=100)
    mask = datagen.config_mask(4, n=200_000)
    pq = PqIndex(128, Metric.L2, m=16, nbits=8, train_iters=25, train_sample=50_000)
    pq.train(data)
    pq.add(data)
    books, codes = pq.codebooks(), pq.codes()
    for msk in (None, mask):
        ids, d = (pq.search_batch(q, k=10) if msk is None else
                  pq.search_batch_filtered(q, msk, k=10))
        o_ids, o_d, _ = oracle.pq_search(books, codes, q, 10, oracle.L2, mask=msk)
        assert np.array_equal(ids, o_ids)
        assert np.array_equal(d, o_d)


def test_pq_recall_reference_thresholds(gpu):
    # tests/test_pq.py:29-43 and :46-54 of the reference (recall@10 > 0.25 for m=8,
    # recall@100 > 0.55 for m=16 on 4000 x 64 Gaussian)
    from proxima_amd import FlatIndex

    rng = np.random.default_rng(0)
    data = rng.standard_normal((4000, 64)).astype(np.float32)
    queries = np.random.default_rng(9).standard_normal((200, 64)).astype(np.float32)
    flat = FlatIndex(64, Metric.L2)
    flat.add(data)

    def recall(approx, gt, k):
        hits = sum(len(set(int(x) for x in a if x >= 0) & set(int(x) for x in g))
                   for a, g in zip(approx, gt))
        return hits / (len(approx) * k)

    gt, _ = flat.search_batch(queries, k=10)
    pq = PqIndex(64, Metric.L2, m=8)
    pq.train(data)
    pq.add(data)
    approx, _ = pq.search_batch(queries, k=10)
    assert recall(approx, gt, 10) > 0.25

    gt100, _ = flat.search_batch(queries, k=100)
    pq16 = PqIndex(64, Metric.L2, m=16)
    pq16.train(data)
    pq16.add(data)
    approx100, _ = pq16.search_batch(queries, k=100)
    assert recall(approx100, gt100, 100) > 0.55


def test_pq_padding_and_empty(gpu):
    data = datagen.gaussian(100, 16, 1)
    pq = _index(data, 4, 6, oracle.IP, iters=2)
    ids, d = pq.search_filtered(data[0], np.zeros(100, dtype=bool), k=5)
    assert (ids == -1).all() and (d == np.float32(-3.4028235e38)).all()
    ids, d = pq.search(data[0], k=120)
    o_ids, o_d, _ = oracle.pq_search(pq.codebooks(), pq.codes(), data[:1], 120, oracle.IP)
    assert np.array_equal(ids, o_ids[0]) and np.array_equal(d, o_d[0])
    assert (ids[100:] == -1).all() and sorted(ids[:100].tolist()) == list(range(100))


@pytest.mark.parametrize("nq", [1, 3])
def test_pq_few_queries_many_lists_exact(gpu, nq):
    # a few queries spread over hundreds of splits x 4 wave lists: the merge sorts only the
    # candidates at or below the k'-th smallest list head
    data = datagen.gaussian(200_000, 32, 301)
    q = datagen.gaussian(nq, 32, 302)
    pq = _index(data, 8, 8, oracle.L2, iters=4, sample=5000)
    for k in (1, 10, 50):
        ids, d = pq.search_batch(q, k=k)
        o_ids, o_d, _ = oracle.pq_search(pq.codebooks(), pq.codes(), q, k, oracle.L2)
        assert np.array_equal(ids, o_ids), k
        assert np.array_equal(d, o_d), k


def test_pq_few_queries_heavy_ties(gpu):
    # 2-bit codebooks over 2 subspaces: 16 distinct codes, so thousands of rows share each
    # key and more than 256 candidates sit at the list-head bound (the merge sorts all)
    data = datagen.gaussian(100_000, 8, 303)
    q = datagen.gaussian(2, 8, 304)
    pq = _index(data, 2, 2, oracle.IP, iters=3, sample=2000)
    ids, d = pq.search_batch(q, k=20)
    o_ids, o_d, _ = oracle.pq_search(pq.codebooks(), pq.codes(), q, 20, oracle.IP)
    assert np.array_equal(ids, o_ids)
    assert np.array_equal(d, o_d)
