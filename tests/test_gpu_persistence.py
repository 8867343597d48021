"""Persistence through the HIP path: indexes saved and loaded in the reference's `.sfidx`
format (bincode 1.x fixint, crates/py/src/lib.rs:19-30 over flat.rs:34-40 and
pq.rs:39-46, 217-223) search on the GPU exactly as the index they were saved from, and as
the oracle does on the loaded data. Mirrors the round trips of the reference's
tests/test_persistence.py:14-57 (search before save == search after load, size, metric,
m, trained), and adds a search of indexes built from hand-written reference-layout bytes.
Imports go through ``proxima``, the reference's own package name.
"""
import struct

import numpy as np
import pytest

import oracle
from conftest import assert_parity
from proxima import FlatIndex, Metric, PqIndex
from proxima_amd import datagen

pytestmark = pytest.mark.gpu


def _unit(rows, dim, seed):
    x = datagen.gaussian(rows, dim, seed)
    return (x / np.linalg.norm(x, axis=1, keepdims=True)).astype(np.float32)


def _key_of(data, queries, metric):
    def key_of(qi, row):
        if metric == oracle.L2:
            return float(oracle.l2_sqr(queries[qi], data[row]))
        return -float(oracle.inner_product(queries[qi], data[row]))
    return key_of


@pytest.mark.parametrize("metric", [Metric.L2, Metric.InnerProduct])
def test_flat_roundtrip_searches_on_gpu(gpu, tmp_path, metric):
    data = _unit(3000, 64, 700)
    q = _unit(300, 64, 701)
    idx = FlatIndex(dim=64, metric=metric)
    idx.add(data)
    before_ids, before_d = idx.search_batch(q, k=10)
    one_ids, one_d = idx.search(data[5].copy(), k=10)
    path = str(tmp_path / "flat.sfidx")
    idx.save(path)
    loaded = FlatIndex.load(path)
    print(f"flat round trip metric={metric!r}", flush=True)
    assert loaded.size == idx.size == 3000 and len(loaded) == 3000
    assert loaded.metric == metric and loaded.dim == 64
    assert np.array_equal(loaded.vectors(), data)
    after_ids, after_d = loaded.search_batch(q, k=10)
    assert np.array_equal(after_ids, before_ids)
    assert np.array_equal(after_d, before_d)
    ids1, d1 = loaded.search(data[5].copy(), k=10)
    assert ids1.tolist() == one_ids.tolist() and np.array_equal(d1, one_d)
    om = oracle.L2 if metric == Metric.L2 else oracle.IP
    o_ids, o_d, _ = oracle.flat_search(data, q, 10, om)
    assert_parity(after_ids, after_d, o_ids, o_d, _key_of(data, q, om))


@pytest.mark.parametrize("metric", [Metric.L2, Metric.InnerProduct])
def test_pq_roundtrip_searches_on_gpu(gpu, tmp_path, metric):
    data = _unit(3000, 64, 710)
    q = _unit(200, 64, 711)
    idx = PqIndex(dim=64, metric=metric, m=4)
    idx.train(data)
    idx.add(data)
    before_ids, before_d = idx.search_batch(q, k=10)
    path = str(tmp_path / "pq.sfidx")
    idx.save(path)
    loaded = PqIndex.load(path)
    print(f"pq round trip metric={metric!r}", flush=True)
    assert loaded.is_trained and loaded.size == idx.size and loaded.m == 4
    assert loaded.metric == metric
    after_ids, after_d = loaded.search_batch(q, k=10)
    assert np.array_equal(after_ids, before_ids)
    assert np.array_equal(after_d, before_d)
    om = oracle.L2 if metric == Metric.L2 else oracle.IP
    o_ids, o_d, _ = oracle.pq_search(loaded.codebooks(), loaded.codes(), q, 10, om)
    assert np.array_equal(after_ids, o_ids)
    assert np.array_equal(after_d, o_d)
    # filtered search on the loaded index, bit for bit
    mask = datagen.mask(3000, 0.3, 712)
    f_ids, f_d = loaded.search_batch_filtered(q, mask, k=10)
    o_ids, o_d, _ = oracle.pq_search(loaded.codebooks(), loaded.codes(), q, 10, om, mask=mask)
    assert np.array_equal(f_ids, o_ids) and np.array_equal(f_d, o_d)


def test_flat_from_reference_bytes(gpu, tmp_path):
    # FlatIndex {dim: u64, metric: u32 variant, n: u64, data: (u64 len, f32...)}, written by
    # hand: 5 rows of 4 dims, inner product
    rows = np.array([[1, 0, 0, 0], [0, 2, 0, 0], [0, 0, 3, 0], [1, 1, 1, 1], [-1, 0, 0, 0]],
                    dtype=np.float32)
    blob = (struct.pack("<Q", 4) + struct.pack("<I", 1) + struct.pack("<Q", 5) +
            struct.pack("<Q", 20) + rows.astype("<f4").tobytes())
    path = tmp_path / "ref_flat.sfidx"
    path.write_bytes(blob)
    idx = FlatIndex.load(str(path))
    assert idx.metric == Metric.InnerProduct and idx.size == 5 and idx.dim == 4
    q = np.array([[1, 1, 1, 1], [0, 0, 1, 0]], dtype=np.float32)
    ids, d = idx.search_batch(q, k=3)
    # dot products by hand: q0 -> [1, 2, 3, 4, -1]; q1 -> [0, 0, 3, 1, 0]
    assert ids.tolist() == [[3, 2, 1], [2, 3, 0]]
    assert d.tolist() == [[4.0, 3.0, 2.0], [3.0, 1.0, 0.0]]
    o_ids, o_d, _ = oracle.flat_search(rows, q, 3, oracle.IP)
    assert np.array_equal(ids, o_ids) and np.array_equal(d, o_d)
    # the known answer of flat.rs:323-338 in file form: corpus {0^4, 1^4}, L2, k = 5
    blob = (struct.pack("<Q", 4) + struct.pack("<I", 0) + struct.pack("<Q", 2) +
            struct.pack("<Q", 8) + struct.pack("<8f", 0, 0, 0, 0, 1, 1, 1, 1))
    path.write_bytes(blob)
    idx = FlatIndex.load(str(path))
    ids, d = idx.search(np.zeros(4, dtype=np.float32), k=5)
    assert ids.tolist() == [0, 1, -1, -1, -1]
    assert d.tolist() == [0.0, 2.0] + [float(np.finfo(np.float32).max)] * 3


def test_pq_from_reference_bytes(gpu, tmp_path):
    # PqIndex {metric: u32, pq: {dim, m, dsub, k: u64, codebooks: (u64, f32...)},
    # codes: (u64, u8...), n: u64}: dim 4, m 2, dsub 2, 2 centroids per subspace, L2
    books = np.array([[[0, 0], [10, 10]], [[1, 1], [5, 5]]], dtype=np.float32)  # [m][k][dsub]
    codes = np.array([[0, 0], [1, 1], [0, 1], [1, 0]], dtype=np.uint8)
    blob = (struct.pack("<I", 0) + struct.pack("<4Q", 4, 2, 2, 2) + struct.pack("<Q", 8) +
            books.astype("<f4").tobytes() + struct.pack("<Q", 8) + codes.tobytes() +
            struct.pack("<Q", 4))
    path = tmp_path / "ref_pq.sfidx"
    path.write_bytes(blob)
    pq = PqIndex.load(str(path))
    assert pq.is_trained and pq.size == 4 and pq.m == 2 and pq.metric == Metric.L2
    q = np.array([[0, 0, 1, 1], [10, 10, 5, 5]], dtype=np.float32)
    ids, d = pq.search_batch(q, k=4)
    # ADC keys by hand, LUT[sub][c] = |q_sub - c|^2 summed in subspace order:
    # q0: rows (0,0)->0+0, (1,1)->200+32, (0,1)->0+32, (1,0)->200+0
    # q1: rows (0,0)->200+32, (1,1)->0+0, (0,1)->200+0, (1,0)->0+32
    assert ids.tolist() == [[0, 2, 3, 1], [1, 3, 2, 0]]
    expect = np.sqrt(np.array([[0, 32, 200, 232], [0, 32, 200, 232]], dtype=np.float32))
    assert np.array_equal(d, expect)
    o_ids, o_d, _ = oracle.pq_search(books, codes, q, 4, oracle.L2)
    assert np.array_equal(ids, o_ids) and np.array_equal(d, o_d)
