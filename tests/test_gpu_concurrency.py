"""Concurrent searches: the reference's search methods take &self (flat.rs:150-230,
pq.rs:349-396), so callers may search one index from several threads. ctypes releases the
GIL around every library call, so these threads really overlap in the library: searches on
one handle are serialised by its lock (they share its workspace and stream), searches on
different handles run on their own streams. Every result must equal the single-threaded one.
"""
import threading

import numpy as np
import pytest

from proxima_amd import FlatIndex, Metric, PqIndex, datagen

pytestmark = pytest.mark.gpu


def test_threads_share_and_split_handles(gpu):
    data = datagen.sift_like(30_000, 64, 401)
    qs = [datagen.sift_like(300, 64, 402 + i) for i in range(6)]
    a = FlatIndex(64, Metric.L2)
    a.add(data)
    b = FlatIndex(64, Metric.InnerProduct)
    b.add(data)
    pq = PqIndex(64, Metric.L2, m=8, nbits=8, train_iters=3, train_sample=5000)
    pq.train(data)
    pq.add(data)
    # (index, queries, k): list and collect paths on the same handle, PQ lists and collect
    jobs = [(a, qs[0], 10), (a, qs[1], 100), (a, qs[2], 700), (b, qs[3], 10), (b, qs[4], 50),
            (pq, qs[5], 10), (pq, qs[0], 300)]
    expected = [idx.search_batch(q, k=k) for idx, q, k in jobs]
    got = [None] * len(jobs)
    errors = []

    def run(i):
        try:
            idx, q, k = jobs[i]
            for _ in range(3):
                got[i] = idx.search_batch(q, k=k)
        except Exception as exc:  # surfaced below
            errors.append(exc)

    threads = [threading.Thread(target=run, args=(i,)) for i in range(len(jobs))]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    assert not errors, errors
    for (ids_e, d_e), res in zip(expected, got):
        assert res is not None
        ids, d = res
        assert np.array_equal(ids, ids_e) and np.array_equal(d, d_e)
