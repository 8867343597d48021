"""CPU oracle for Proxima's exact-search path -- TEST INFRASTRUCTURE ONLY.

The checker, never the product: only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg import this package. It wraps oracle/libpx_oracle.so, a C restatement of
crates/core/src/distance.rs:3-39, flat.rs:106-230 and pq.rs:25-396 (see px_oracle.h for
the line-by-line map and the canonical (key, id) tie order).

Parity status of every function: pinned (tests/test_oracle.py) by the reference's known
answers and structural tests, numpy float64 brute force, integer-exact closed forms
(sums below 2^24 are exact in any order), hand-computed lane orders, and for PQ training
by hand-derived known answers (the reciprocal-multiply mean of pq.rs:185-188 and the
empty-cluster re-seed of pq.rs:180-183 from published SplitMix64 draws), the Lloyd-step
invariant, distinct-row initialisation and bit equality with the product's own trainer
(tests/test_oracle.py). The one detail no check can pin
-- which of several exactly equal keys Rust's BinaryHeap keeps at the k-boundary -- is
exempt under the parity rule (exact ties differ by 0 < 1e-5 relative).
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_float, c_int, c_int64, c_uint8, c_uint64

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libpx_oracle.so")
_lib = None

L2 = 0
IP = 1


def load():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} missing: run `make -C oracle`")
        lib = ctypes.CDLL(LIB_PATH)
        f32p, i64p, u8p = POINTER(c_float), POINTER(c_int64), POINTER(c_uint8)
        lib.px_or_l2_sqr.restype = c_float
        lib.px_or_l2_sqr.argtypes = [f32p, f32p, c_int64]
        lib.px_or_inner_product.restype = c_float
        lib.px_or_inner_product.argtypes = [f32p, f32p, c_int64]
        lib.px_or_splitmix_next.restype = c_uint64
        lib.px_or_splitmix_next.argtypes = [POINTER(c_uint64)]
        lib.px_or_flat_search.restype = c_int
        lib.px_or_flat_search.argtypes = [f32p, c_int64, c_int64, c_int, f32p, c_int64, c_int64,
                                          u8p, i64p, f32p, f32p, c_int]
        lib.px_or_pq_train.restype = c_int
        lib.px_or_pq_train.argtypes = [f32p, c_int64, c_int64, c_int64, c_int64, c_int64,
                                       c_int64, c_uint64, f32p, c_int]
        lib.px_or_pq_encode.restype = c_int
        lib.px_or_pq_encode.argtypes = [f32p, c_int64, c_int64, c_int64, f32p, c_int64, u8p,
                                        c_int]
        lib.px_or_pq_adc_table.restype = None
        lib.px_or_pq_adc_table.argtypes = [f32p, c_int64, c_int64, c_int64, c_int, f32p, f32p]
        lib.px_or_pq_search.restype = c_int
        lib.px_or_pq_search.argtypes = [f32p, c_int64, c_int64, c_int64, c_int, u8p, c_int64,
                                        f32p, c_int64, c_int64, u8p, i64p, f32p, f32p, c_int]
        lib.px_or_max_threads.restype = c_int
        lib.px_or_max_threads.argtypes = []
        _lib = lib
    return _lib


def _f(a):
    return a.ctypes.data_as(POINTER(c_float))


def _c32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def max_threads() -> int:
    return int(load().px_or_max_threads())


def l2_sqr(a, b) -> np.float32:
    a, b = _c32(a), _c32(b)
    assert a.shape == b.shape
    return np.float32(load().px_or_l2_sqr(_f(a), _f(b), a.size))


def inner_product(a, b) -> np.float32:
    a, b = _c32(a), _c32(b)
    assert a.shape == b.shape
    return np.float32(load().px_or_inner_product(_f(a), _f(b), a.size))


def splitmix(seed: int, count: int) -> list[int]:
    st = c_uint64(seed)
    return [int(load().px_or_splitmix_next(ctypes.byref(st))) for _ in range(count)]


def flat_search(data, queries, k: int, metric: int, mask=None, nthreads: int = 0):
    """Returns (ids int64[nq,k], dists float32[nq,k], keys float32[nq,k]) in canonical order."""
    data, queries = _c32(data), _c32(queries)
    n, dim = data.shape
    nq = queries.shape[0]
    ids = np.empty((nq, k), dtype=np.int64)
    dists = np.empty((nq, k), dtype=np.float32)
    keys = np.empty((nq, k), dtype=np.float32)
    mp = None
    if mask is not None:
        m = np.ascontiguousarray(mask, dtype=np.bool_).view(np.uint8)
        assert m.size == n
        mp = m.ctypes.data_as(POINTER(c_uint8))
    rc = load().px_or_flat_search(_f(data), n, dim, metric, _f(queries), nq, k, mp,
                                  ids.ctypes.data_as(POINTER(c_int64)), _f(dists), _f(keys),
                                  nthreads)
    if rc != 0:
        raise ValueError("oracle rejected the arguments")
    return ids, dists, keys


def pq_train(training, m: int, nbits: int, train_iters: int, train_sample: int, seed: int,
             nthreads: int = 0) -> np.ndarray:
    t = _c32(training)
    n, dim = t.shape
    ks = 1 << nbits
    books = np.empty((m, ks, dim // m), dtype=np.float32)
    rc = load().px_or_pq_train(_f(t), n, dim, m, nbits, train_iters, train_sample, seed,
                               _f(books), nthreads)
    if rc != 0:
        raise ValueError("oracle rejected the training arguments")
    return books


def pq_encode(books, vectors, nthreads: int = 0) -> np.ndarray:
    books, v = _c32(books), _c32(vectors)
    m, ks, dsub = books.shape
    n, dim = v.shape
    codes = np.empty((n, m), dtype=np.uint8)
    rc = load().px_or_pq_encode(_f(books), dim, m, ks.bit_length() - 1, _f(v), n,
                                codes.ctypes.data_as(POINTER(c_uint8)), nthreads)
    if rc != 0:
        raise ValueError("oracle rejected the encode arguments")
    return codes


def pq_adc_table(books, query, metric: int) -> np.ndarray:
    books, q = _c32(books), _c32(query)
    m, ks, dsub = books.shape
    table = np.empty((m, ks), dtype=np.float32)
    load().px_or_pq_adc_table(_f(books), q.size, m, ks.bit_length() - 1, metric, _f(q),
                              _f(table))
    return table


def pq_search(books, codes, queries, k: int, metric: int, mask=None, nthreads: int = 0):
    books, q = _c32(books), _c32(queries)
    codes = np.ascontiguousarray(codes, dtype=np.uint8)
    m, ks, dsub = books.shape
    n = codes.shape[0]
    nq, dim = q.shape
    ids = np.empty((nq, k), dtype=np.int64)
    dists = np.empty((nq, k), dtype=np.float32)
    keys = np.empty((nq, k), dtype=np.float32)
    mp = None
    if mask is not None:
        mm = np.ascontiguousarray(mask, dtype=np.bool_).view(np.uint8)
        assert mm.size == n
        mp = mm.ctypes.data_as(POINTER(c_uint8))
    rc = load().px_or_pq_search(_f(books), dim, m, ks.bit_length() - 1, metric,
                                codes.ctypes.data_as(POINTER(c_uint8)), n, _f(q), nq, k, mp,
                                ids.ctypes.data_as(POINTER(c_int64)), _f(dists), _f(keys),
                                nthreads)
    if rc != 0:
        raise ValueError("oracle rejected the search arguments")
    return ids, dists, keys
