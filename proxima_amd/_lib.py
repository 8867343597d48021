"""ctypes binding of libproxima_px.so (include/proxima_px.h).

This is the binding a Python caller of the C ABI would write; the reference's own
binding of its GPU seam is the Rust ``extern "C"`` block in crates/core/src/gpu.rs:10-15.
The library is built in-tree by ``__graft_entry__.build()`` (or ``make -C
proxima_amd/csrc``); importing this module does not build anything.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_char, c_char_p, c_float, c_int, c_int64, c_longlong, c_size_t
from ctypes import c_uint8, c_uint64, c_void_p

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libproxima_px.so")
# the same library with the kernels' index checks compiled in (-DPX_DEBUG): a failed check
# fails the search with PX_ERR_ARG naming its file and line
DEBUG_LIB_PATH = os.path.join(_HERE, "libproxima_px_debug.so")

PX_OK = 0
PX_ERR_BAD_K = -1
PX_ERR_SHMEM = -2
PX_ERR_DIM = -3
PX_ERR_NONFINITE = -4
PX_ERR_ARG = -5
PX_ERR_UNTRAINED = -6
PX_ERR_DEVICE = -7
PX_MAX_K = 4096

_f32p = POINTER(c_float)
_i64p = POINTER(c_int64)
_u8p = POINTER(c_uint8)

# name -> (restype, argtypes); mirrors include/proxima_px.h one to one.
SIGNATURES = {
    "px_last_error": (c_char_p, []),
    "px_version": (c_char_p, []),
    "knn_gpu_create": (c_void_p, [_f32p, c_int, c_int]),
    "knn_gpu_search": (c_int, [c_void_p, _f32p, c_int, c_int, c_int, POINTER(c_longlong), _f32p]),
    "knn_gpu_free": (None, [c_void_p]),
    "px_flat_create": (c_int, [c_int, c_int64, POINTER(c_void_p)]),
    "px_flat_destroy": (None, [c_void_p]),
    "px_flat_add": (c_int, [c_void_p, _f32p, c_int64]),
    "px_flat_search": (c_int, [c_void_p, _f32p, c_int64, c_int64, _u8p, _i64p, _f32p]),
    "px_flat_search_device": (c_int, [c_void_p, c_void_p, c_int64, c_int64, c_void_p, c_void_p,
                                      c_void_p]),
    "px_flat_search_device_noalloc": (c_int, [c_void_p, c_void_p, c_int64, c_int64, c_void_p,
                                              c_void_p, c_void_p]),
    "px_flat_get_vectors": (c_int, [c_void_p, c_int64, c_int64, _f32p]),
    "px_flat_size": (c_int64, [c_void_p]),
    "px_flat_dim": (c_int64, [c_void_p]),
    "px_flat_metric": (c_int, [c_void_p]),
    "px_flat_memory_bytes": (c_int64, [c_void_p]),
    "px_pq_create": (c_int, [c_int, c_int64, c_int64, c_int64, POINTER(c_void_p)]),
    "px_pq_destroy": (None, [c_void_p]),
    "px_pq_train": (c_int, [c_void_p, _f32p, c_int64, c_int64, c_int64, c_uint64]),
    "px_pq_set_codebooks": (c_int, [c_void_p, _f32p]),
    "px_pq_get_codebooks": (c_int, [c_void_p, _f32p]),
    "px_pq_add": (c_int, [c_void_p, _f32p, c_int64]),
    "px_pq_add_codes": (c_int, [c_void_p, _u8p, c_int64]),
    "px_pq_get_codes": (c_int, [c_void_p, c_int64, c_int64, _u8p]),
    "px_pq_search": (c_int, [c_void_p, _f32p, c_int64, c_int64, _u8p, _i64p, _f32p]),
    "px_pq_search_device": (c_int, [c_void_p, c_void_p, c_int64, c_int64, c_void_p, c_void_p,
                                    c_void_p]),
    "px_pq_is_trained": (c_int, [c_void_p]),
    "px_pq_size": (c_int64, [c_void_p]),
    "px_pq_dim": (c_int64, [c_void_p]),
    "px_pq_m": (c_int64, [c_void_p]),
    "px_pq_nbits": (c_int64, [c_void_p]),
    "px_pq_metric": (c_int, [c_void_p]),
    "px_pq_memory_bytes": (c_int64, [c_void_p]),
    "px_pq_raw_bytes": (c_int64, [c_void_p]),
    "px_device_count": (c_int, []),
    "px_device_info": (c_int, [c_int, POINTER(c_char), c_size_t, POINTER(c_int), _i64p,
                               POINTER(c_int), POINTER(c_char), c_size_t]),
    "px_flat_set_timing": (c_int, [c_void_p, c_int]),
    "px_flat_last_timing": (c_int, [c_void_p, _f32p, _f32p, POINTER(c_int), POINTER(c_int)]),
    "px_flat_last_rounds": (c_int, [c_void_p, POINTER(c_int)]),
    "px_flat_last_path": (c_int, [c_void_p, POINTER(c_int)]),
    "px_flat_set_scan_f16": (c_int, [c_void_p, c_int]),
    "px_flat_last_scan_f16": (c_int, [c_void_p, POINTER(c_int)]),
    "px_flat_set_spin_limit": (c_int, [c_void_p, c_int]),
    "px_pq_last_rounds": (c_int, [c_void_p, POINTER(c_int)]),
    "px_hip_versions": (c_int, [POINTER(c_int), POINTER(c_int)]),
    "px_pq_set_timing": (c_int, [c_void_p, c_int]),
    "px_pq_last_timing": (c_int, [c_void_p, _f32p, _f32p, POINTER(c_int), POINTER(c_int)]),
    "px_dev_alloc": (c_int, [POINTER(c_void_p), c_size_t]),
    "px_dev_free": (c_int, [c_void_p]),
    "px_dev_upload": (c_int, [c_void_p, c_void_p, c_size_t]),
    "px_dev_download": (c_int, [c_void_p, c_void_p, c_size_t]),
    "px_dev_copy_kernel": (c_int, [c_void_p, c_void_p, c_size_t, _f32p]),
    "px_dev_lds_gather": (c_int, [c_int, c_int, c_int, _f32p, POINTER(ctypes.c_double)]),
}

_lib = None


def load() -> ctypes.CDLL:
    """Load libproxima_px.so once; raise ImportError naming the build step if absent."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; "
            "g.build()'` or `make -C proxima_amd/csrc` (hipcc --offload-arch=gfx950)")
    _lib = load_path(LIB_PATH)
    return _lib


def load_path(path: str) -> ctypes.CDLL:
    """A build of the library at `path` (e.g. DEBUG_LIB_PATH) with the signatures set; a
    separate handle with its own state, loaded beside the default one."""
    lib = ctypes.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


def last_error() -> str:
    msg = load().px_last_error()
    return msg.decode("utf-8", "replace") if msg else ""


def device_count() -> int:
    return int(load().px_device_count())


def device_info(device: int = 0) -> dict:
    lib = load()
    name = ctypes.create_string_buffer(256)
    arch = ctypes.create_string_buffer(64)
    cus = c_int(0)
    hbm = c_int64(0)
    clk = c_int(0)
    rc = lib.px_device_info(device, name, 256, ctypes.byref(cus), ctypes.byref(hbm),
                            ctypes.byref(clk), arch, 64)
    if rc != PX_OK:
        raise RuntimeError(last_error())
    return {"name": name.value.decode(), "arch": arch.value.decode(), "cus": cus.value,
            "hbm_bytes": hbm.value, "clock_khz": clk.value}


def f32p(a):
    return a.ctypes.data_as(_f32p)


def i64p(a):
    return a.ctypes.data_as(_i64p)


def u8p(a):
    return a.ctypes.data_as(_u8p)
