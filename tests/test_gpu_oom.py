"""Out-of-device-memory paths on the GPU, simulated with PX_DEVICE_BUDGET.

PX_DEVICE_BUDGET (bytes, read at every device allocation of the library) caps the library's
own device memory; an allocation past it fails with hipErrorOutOfMemory as on a full device
(the reference returns NULL from gpu_knn_create on a failed cudaMalloc, gpu.rs:31-33, and its
Python surface raises). Each failure must leave the index as it was -- rows counted, results
unchanged -- and the same index must work again once memory is there.
"""
import contextlib
import os

import numpy as np
import pytest

import oracle
from proxima_amd import FlatIndex, Metric, PqIndex, datagen

pytestmark = pytest.mark.gpu


@contextlib.contextmanager
def device_budget(nbytes):
    os.environ["PX_DEVICE_BUDGET"] = str(nbytes)
    try:
        yield
    finally:
        del os.environ["PX_DEVICE_BUDGET"]


def test_flat_add_and_search_out_of_memory(gpu):
    data = datagen.sift_like(30_000, 48, 301)
    more = datagen.sift_like(40_000, 48, 302)
    q = datagen.sift_like(40, 48, 303)
    big_q = datagen.sift_like(3000, 48, 304)
    idx = FlatIndex(48, Metric.L2)
    idx.add(data)
    ids0, d0 = idx.search_batch(q, k=10)
    print("case flat add past the budget", flush=True)
    with device_budget(1):  # nothing more can be allocated
        with pytest.raises(RuntimeError, match="out of memory"):
            idx.add(more)  # the corpus mirror must grow
        assert len(idx) == 30_000
        ids, d = idx.search_batch(q, k=10)  # its workspace is already there
        assert np.array_equal(ids, ids0) and np.array_equal(d, d0)
        print("case flat search past the budget", flush=True)
        with pytest.raises(RuntimeError, match="out of memory"):
            idx.search_batch(big_q, k=10)  # a larger batch needs a larger workspace
        with pytest.raises(RuntimeError, match="out of memory"):
            idx.search_batch(q, k=500)  # the collect path's buffers
    print("case flat after the budget", flush=True)
    idx.add(more)
    both = np.concatenate([data, more])
    assert len(idx) == 70_000
    for qq, k in ((q, 10), (big_q, 10), (q, 500)):
        ids, d = idx.search_batch(qq, k=k)
        o_ids, o_d, _ = oracle.flat_search(both, qq, k, oracle.L2)
        assert np.array_equal(ids, o_ids) and np.array_equal(d, o_d), k


def test_pq_train_and_add_out_of_memory(gpu):
    data = datagen.gaussian(6000, 32, 311)
    q = datagen.gaussian(20, 32, 312)
    pq = PqIndex(32, Metric.L2, m=8, nbits=6, train_iters=5, train_sample=4000)
    print("case pq train past the budget", flush=True)
    with device_budget(1):
        with pytest.raises(RuntimeError, match="out of memory"):
            pq.train(data)
    pq.train(data)
    pq.add(data[:2000])
    ids0, d0 = pq.search_batch(q, k=10)
    print("case pq add past the budget", flush=True)
    with device_budget(1):
        with pytest.raises(RuntimeError, match="out of memory"):
            pq.add(data[2000:])  # 6,000 codes pass the first code buffer's 4,096 rows
        assert len(pq) == 2000
        ids, d = pq.search_batch(q, k=10)
        assert np.array_equal(ids, ids0) and np.array_equal(d, d0)
    pq.add(data[2000:])
    assert len(pq) == 6000
    ids, d = pq.search_batch(q, k=10)
    o_ids, o_d, _ = oracle.pq_search(pq.codebooks(), pq.codes(), q, 10, oracle.L2)
    assert np.array_equal(ids, o_ids) and np.array_equal(d, o_d)
