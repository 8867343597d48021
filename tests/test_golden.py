"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py).

CPU: the generators reproduce the recorded input SHA-256s on this host, and the oracle
reproduces the recorded ids and keys exactly. GPU: the HIP path meets the parity rule
against the same fixtures (integer-valued workloads bit-exact).
"""
import os
import sys

import numpy as np
import pytest

import oracle
from conftest import assert_parity

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import make_golden as mg  # noqa: E402


def _load(name):
    with np.load(os.path.join(HERE, "golden", name + ".npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.mark.parametrize("name", sorted(mg.FLAT_CASES))
def test_flat_fixture_oracle(name):
    c, rows, nq, ks, metric, p = mg.FLAT_CASES[name]
    fx = _load(name)
    data, q, mask = mg.flat_inputs(c, rows, nq, p)
    assert mg.sha(data) == str(fx["corpus_sha256"])
    assert mg.sha(q) == str(fx["queries_sha256"])
    assert (mg.sha(mask) if mask is not None else "") == str(fx["mask_sha256"])
    for k in ks:
        ids, _, keys = oracle.flat_search(data, q, k, metric, mask=mask)
        assert np.array_equal(ids, fx[f"ids_k{k}"])
        assert np.array_equal(keys, fx[f"keys_k{k}"])


def test_pq_fixture_oracle():
    fx = _load(mg.PQ_CASE)
    data, q, mask = mg.pq_inputs()
    assert mg.sha(data) == str(fx["corpus_sha256"])
    assert mg.sha(q) == str(fx["queries_sha256"])
    assert mg.sha(mask) == str(fx["mask_sha256"])
    books, codes = mg.pq_model(data)
    assert mg.sha(books) == str(fx["books_sha256"])
    assert mg.sha(codes) == str(fx["codes_sha256"])
    for tag, mk in (("", None), ("_mask50", mask)):
        ids, _, keys = oracle.pq_search(books, codes, q, 10, oracle.L2, mask=mk)
        assert np.array_equal(ids, fx[f"ids_k10{tag}"])
        assert np.array_equal(keys, fx[f"keys_k10{tag}"])


def _finish(keys, metric):
    pad = ~np.isfinite(keys)
    d = np.sqrt(np.where(pad, 0, keys)) if metric == oracle.L2 else -keys
    d = d.astype(np.float32)
    d[pad] = np.float32(3.4028235e38) if metric == oracle.L2 else np.float32(-3.4028235e38)
    return d


@pytest.mark.gpu
@pytest.mark.parametrize("name", sorted(mg.FLAT_CASES))
def test_flat_fixture_gpu(gpu, name):
    from proxima_amd import FlatIndex, Metric

    c, rows, nq, ks, metric, p = mg.FLAT_CASES[name]
    fx = _load(name)
    data, q, mask = mg.flat_inputs(c, rows, nq, p)
    idx = FlatIndex(data.shape[1], Metric.L2 if metric == oracle.L2 else Metric.InnerProduct)
    idx.add(data)
    for k in ks:
        print(f"golden {name} k={k}", flush=True)
        if mask is None:
            ids, d = idx.search_batch(q, k=k)
        else:
            ids, d = idx.search_batch_filtered(q, mask, k=k)
        o_ids = fx[f"ids_k{k}"].astype(np.int64)
        o_d = _finish(fx[f"keys_k{k}"], metric)

        def key_of(qi, row):
            if metric == oracle.L2:
                return float(oracle.l2_sqr(q[qi], data[row]))
            return float(-oracle.inner_product(q[qi], data[row]))

        exact = c == 3  # integer-valued workload: keys exact, no exemption needed
        assert_parity(ids, d, o_ids, o_d, key_of, allow_exempt=not exact)
        if exact:
            assert np.array_equal(d, o_d)


@pytest.mark.gpu
def test_pq_fixture_gpu(gpu):
    from proxima_amd import Metric, PqIndex

    fx = _load(mg.PQ_CASE)
    data, q, mask = mg.pq_inputs()
    pq = PqIndex(128, Metric.L2, m=mg.PQ_M, nbits=mg.PQ_NBITS, train_iters=mg.PQ_ITERS,
                 train_sample=0, seed=mg.PQ_SEED)
    pq.train(data[:mg.PQ_TRAIN_ROWS])
    pq.add(data)
    assert mg.sha(pq.codebooks()) == str(fx["books_sha256"])
    assert mg.sha(pq.codes()) == str(fx["codes_sha256"])
    for tag, mk in (("", None), ("_mask50", mask)):
        print(f"golden pq{tag}", flush=True)
        if mk is None:
            ids, d = pq.search_batch(q, k=10)
        else:
            ids, d = pq.search_batch_filtered(q, mk, k=10)
        assert np.array_equal(ids, fx[f"ids_k10{tag}"].astype(np.int64))
        assert np.array_equal(d, _finish(fx[f"keys_k10{tag}"], oracle.L2))
