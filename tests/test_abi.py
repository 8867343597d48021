"""The C ABI (include/proxima_px.h) without a GPU: the library loads, exports every
declared entry point, and its argument checks and no-device errors behave as documented.
No compute call is made."""
import ctypes
import os
import re
import subprocess

import numpy as np
import pytest

from proxima_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    names = set()
    for fn in os.listdir(os.path.join(ROOT, "include")):
        if not fn.endswith(".h"):
            continue
        with open(os.path.join(ROOT, "include", fn)) as fh:
            text = re.sub(r"/\*.*?\*/", "", fh.read(), flags=re.S)
        for m in re.finditer(r"^[A-Za-z_][\w \*]*?\b((?:px|knn_gpu)_\w+)\s*\(", text, re.M):
            names.add(m.group(1))
    return names


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    declared = _declared()
    assert len(declared) >= 40
    missing = [n for n in sorted(declared) if not hasattr(lib, n)]
    assert not missing, missing
    # the ctypes binding covers exactly the header
    assert declared == set(_lib.SIGNATURES)


def test_version_and_error_strings():
    lib = _lib.load()
    assert lib.px_version() == b"0.1.0"
    h = ctypes.c_void_p()
    assert lib.px_flat_create(0, 0, ctypes.byref(h)) == _lib.PX_ERR_DIM
    assert b"dim" in lib.px_last_error()
    assert lib.px_flat_create(7, 4, ctypes.byref(h)) == _lib.PX_ERR_ARG
    assert lib.px_flat_create(0, 4, None) == _lib.PX_ERR_ARG
    assert lib.px_pq_create(0, 10, 3, 8, ctypes.byref(h)) == _lib.PX_ERR_DIM
    assert lib.px_pq_create(0, 8, 0, 8, ctypes.byref(h)) == _lib.PX_ERR_ARG
    assert lib.px_pq_create(0, 8, 2, 9, ctypes.byref(h)) == _lib.PX_ERR_ARG


def test_handle_lifecycle_and_argument_checks():
    lib = _lib.load()
    h = ctypes.c_void_p()
    assert lib.px_flat_create(1, 4, ctypes.byref(h)) == 0
    try:
        assert lib.px_flat_dim(h) == 4 and lib.px_flat_metric(h) == 1
        bad = np.array([[0, np.nan, 0, 0]], dtype=np.float32)
        assert lib.px_flat_add(h, _lib.f32p(bad), 1) == _lib.PX_ERR_NONFINITE
        assert lib.px_flat_size(h) == 0
        ok = np.arange(8, dtype=np.float32).reshape(2, 4)
        assert lib.px_flat_add(h, _lib.f32p(ok), 2) == 0
        assert lib.px_flat_size(h) == 2 and lib.px_flat_memory_bytes(h) == 32
        back = np.empty((2, 4), np.float32)
        assert lib.px_flat_get_vectors(h, 0, 2, _lib.f32p(back)) == 0
        assert np.array_equal(back, ok)
        q = np.zeros((1, 4), np.float32)
        ids = np.empty(1, np.int64)
        d = np.empty(1, np.float32)
        assert lib.px_flat_search(h, _lib.f32p(q), 1, -1, None, _lib.i64p(ids),
                                  _lib.f32p(d)) == _lib.PX_ERR_BAD_K
        # any k >= 0 is an argument the search accepts (flat.rs:106-148 keeps a heap of k);
        # with no device it then reports the device
        big_ids = np.empty(_lib.PX_MAX_K + 1, np.int64)
        big_d = np.empty(_lib.PX_MAX_K + 1, np.float32)
        assert lib.px_flat_search(h, _lib.f32p(q), 1, _lib.PX_MAX_K + 1, None,
                                  _lib.i64p(big_ids), _lib.f32p(big_d)) == _lib.PX_ERR_DEVICE
        nanq = np.full((1, 4), np.inf, np.float32)
        assert lib.px_flat_search(h, _lib.f32p(nanq), 1, 1, None, _lib.i64p(ids),
                                  _lib.f32p(d)) == _lib.PX_ERR_NONFINITE
        # k == 0 still validates the queries (the reference checks finiteness first)
        assert lib.px_flat_search(h, _lib.f32p(nanq), 1, 0, None, _lib.i64p(ids),
                                  _lib.f32p(d)) == _lib.PX_ERR_NONFINITE
        assert lib.px_flat_search(None, _lib.f32p(q), 1, 1, None, _lib.i64p(ids),
                                  _lib.f32p(d)) == _lib.PX_ERR_ARG
    finally:
        lib.px_flat_destroy(h)
    lib.px_flat_destroy(None)
    lib.knn_gpu_free(None)
    lib.px_pq_destroy(None)


def test_pq_untrained_errors():
    lib = _lib.load()
    h = ctypes.c_void_p()
    assert lib.px_pq_create(0, 8, 2, 4, ctypes.byref(h)) == 0
    try:
        v = np.zeros((3, 8), np.float32)
        assert lib.px_pq_add(h, _lib.f32p(v), 3) == _lib.PX_ERR_UNTRAINED
        ids = np.empty(3, np.int64)
        d = np.empty(3, np.float32)
        assert lib.px_pq_search(h, _lib.f32p(v), 1, 3, None, _lib.i64p(ids),
                                _lib.f32p(d)) == _lib.PX_ERR_UNTRAINED
        assert lib.px_pq_train(h, _lib.f32p(v), 3, 5, 0, 1) == _lib.PX_ERR_ARG  # < 16 rows
        assert lib.px_pq_is_trained(h) == 0 and lib.px_pq_memory_bytes(h) == 0
    finally:
        lib.px_pq_destroy(h)


@pytest.mark.skipif(_lib.device_count() > 0, reason="checks the no-device path")
def test_no_device_search_fails_loudly():
    # There is no CPU search path: without a gfx950 device a search is an error.
    lib = _lib.load()
    assert lib.px_device_count() == 0
    h = ctypes.c_void_p()
    assert lib.px_flat_create(0, 4, ctypes.byref(h)) == 0
    try:
        data = np.ones((3, 4), np.float32)
        assert lib.px_flat_add(h, _lib.f32p(data), 3) == 0
        ids = np.empty(2, np.int64)
        d = np.empty(2, np.float32)
        rc = lib.px_flat_search(h, _lib.f32p(data), 1, 2, None, _lib.i64p(ids), _lib.f32p(d))
        assert rc == _lib.PX_ERR_DEVICE
        assert b"gfx950" in lib.px_last_error()
    finally:
        lib.px_flat_destroy(h)
    assert lib.knn_gpu_create(_lib.f32p(np.ones((2, 4), np.float32)), 2, 4) is None


def _abi_check_binary():
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "c_abi", "abi_check")
    if not os.path.exists(path):
        pytest.fail(f"{path} is missing: build it with __graft_entry__.build() "
                    "(make -C tests/c_abi)")
    return path


@pytest.mark.skipif(_lib.device_count() > 0, reason="checks the no-device path")
def test_c_program_no_device():
    # the same binary runs the gfx950 known answers on a GPU box (test_gpu_c_abi.py)
    out = subprocess.run([_abi_check_binary()], capture_output=True, text=True, timeout=60)
    assert out.returncode == 0, out.stderr
    assert out.stdout.startswith("abi_check ok (no-device path")
