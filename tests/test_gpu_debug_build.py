"""The debug build on the GPU: every search path with the kernels' index checks compiled in.

proxima_amd/libproxima_px_debug.so is the library built with -DPX_DEBUG: its scan, select,
merge and PQ kernels check the positions, row ids, region slots, dense offsets and list
entries they touch against the launch's bounds and record the first failure, which fails
the search with PX_ERR_ARG naming the file and line (the kernels never trap). Each case
runs once through the product library and once through the debug build, loaded side by
side in this process: the debug build must report no failed check and return the product's
results bit for bit.
"""
import ctypes

import numpy as np
import pytest

from proxima_amd import _lib, datagen

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def libs(gpu):
    return _lib.load(), _lib.load_path(_lib.DEBUG_LIB_PATH)


def _ptr(a, t):
    return a.ctypes.data_as(ctypes.POINTER(t))


def _flat(lib, data, q, k, metric, mask=None):
    h = ctypes.c_void_p()
    assert lib.px_flat_create(metric, data.shape[1], ctypes.byref(h)) == 0
    try:
        assert lib.px_flat_add(h, _ptr(data, ctypes.c_float), data.shape[0]) == 0
        ids = np.empty((q.shape[0], k), np.int64)
        d = np.empty((q.shape[0], k), np.float32)
        m = None if mask is None else _ptr(mask.view(np.uint8), ctypes.c_uint8)
        rc = lib.px_flat_search(h, _ptr(q, ctypes.c_float), q.shape[0], k, m,
                                _ptr(ids, ctypes.c_int64), _ptr(d, ctypes.c_float))
        path = ctypes.c_int()
        lib.px_flat_last_path(h, ctypes.byref(path))
        return rc, ids, d, path.value, lib.px_last_error()
    finally:
        lib.px_flat_destroy(h)


def _pq(lib, data, q, k, mask=None):
    h = ctypes.c_void_p()
    assert lib.px_pq_create(0, data.shape[1], 8, 8, ctypes.byref(h)) == 0
    try:
        assert lib.px_pq_train(h, _ptr(data, ctypes.c_float), data.shape[0], 4, 4000, 5) == 0
        assert lib.px_pq_add(h, _ptr(data, ctypes.c_float), data.shape[0]) == 0
        ids = np.empty((q.shape[0], k), np.int64)
        d = np.empty((q.shape[0], k), np.float32)
        m = None if mask is None else _ptr(mask.view(np.uint8), ctypes.c_uint8)
        rc = lib.px_pq_search(h, _ptr(q, ctypes.c_float), q.shape[0], k, m,
                              _ptr(ids, ctypes.c_int64), _ptr(d, ctypes.c_float))
        return rc, ids, d, -1, lib.px_last_error()
    finally:
        lib.px_pq_destroy(h)


# name -> (run(lib) -> (rc, ids, dists, path, error), expected path: 0 lists, 1 sampled
# collect, 2 bounded collect, 3 vector-ALU collect, 4 full sort, -1 PQ); data made on demand
def _case(name):
    g = datagen
    if name.startswith("lists") or name == "vector-ALU collect":
        d, q = g.gaussian(30_000, 64, 901), g.gaussian(100, 64, 902)
        if name == "lists L2":
            return (lambda lib: _flat(lib, d, q, 10, 0)), 0
        if name == "lists IP":
            return (lambda lib: _flat(lib, d, q, 10, 1)), 0
        if name == "lists filtered":
            m = g.mask(30_000, 0.3, 903)
            return (lambda lib: _flat(lib, d, q, 10, 0, m)), 0
        return (lambda lib: _flat(lib, d, q[:5], 10, 0)), 3
    if name == "bounded collect":
        d, q = g.sift_like(40_000, 64, 904), g.sift_like(2048, 64, 905)
        return (lambda lib: _flat(lib, d, q, 10, 0)), 2
    if name == "sampled collect":
        d, q = g.gaussian(20_000, 100, 906), g.gaussian(300, 100, 907)
        return (lambda lib: _flat(lib, d, q, 200, 1)), 1
    if name == "collect, 3 chunks, filtered":
        d, q = g.unit_gaussian(20_000, 300, 908), g.unit_gaussian(300, 300, 909)
        m = g.mask(20_000, 0.1, 910)
        return (lambda lib: _flat(lib, d, q, 150, 1, m)), 1
    if name == "full sort":
        d, q = g.gaussian(6000, 24, 911), g.gaussian(10, 24, 912)
        return (lambda lib: _flat(lib, d, q, 4100, 0)), 4
    d, q = g.gaussian(6000, 32, 913), g.gaussian(50, 32, 914)
    if name == "pq lists":
        return (lambda lib: _pq(lib, d, q, 10)), -1
    m = g.mask(6000, 0.5, 915)
    return (lambda lib: _pq(lib, d, q, 200, m)), -1


CASES = ["lists L2", "lists IP", "lists filtered", "bounded collect", "sampled collect",
         "collect, 3 chunks, filtered", "vector-ALU collect", "full sort", "pq lists",
         "pq collect filtered"]


@pytest.mark.parametrize("name", CASES)
def test_debug_build_checks_pass_and_match(libs, name):
    run, path = _case(name)
    prod, dbg = libs
    print(f"case debug build {name}", flush=True)
    rc, ids, d, p, err = run(prod)
    assert rc == 0, err
    rc_d, ids_d, d_d, p_d, err_d = run(dbg)
    assert rc_d == 0, err_d
    assert p == p_d == path
    assert np.array_equal(ids, ids_d) and np.array_equal(d, d_d)
