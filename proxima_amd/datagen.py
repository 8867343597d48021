"""Deterministic synthetic workloads (ctypes over libpx_datagen.so).

SplitMix64 in counter form: element i of seed s is mix(s + (i+1) * 0x9E3779B97F4A7C15),
the i-th output of the reference's sequential generator (crates/core/src/pq.rs:27-33).
Every sampler is integer arithmetic up to one final rounding, so the same seed gives the
same bits on every host.

Workloads (seeds: corpus 1000c+1, queries 1000c+2, mask 1000c+3):
  1  FlatIndex L2, 10,000 x 128 N(0,1), 100 queries, k=10
  2  FlatIndex IP, 100,000 x 384 unit Gaussian, 1,000 held-out queries, k=10
  3  FlatIndex L2, 1,000,000 x 128 SIFT-like integers in [0,255], 10,000 queries, k=10/100
  4  PqIndex L2 ADC, 1,000,000 x 128 N(0,1), m=16 x 8 bit, 10,000 queries, k=10, 50% mask
  5  FlatIndex IP, 10,000,000 x 384 unit Gaussian, 16,384 queries, k=100, 10% mask
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_double, c_float, c_int, c_int64, c_uint8, c_uint64

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libpx_datagen.so")
_gen = None


def _load():
    global _gen
    if _gen is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is missing: run __graft_entry__.build()")
        g = ctypes.CDLL(LIB_PATH)
        f32p, u8p = POINTER(c_float), POINTER(c_uint8)
        g.px_gen_stream_at.restype = c_uint64
        g.px_gen_stream_at.argtypes = [c_uint64, c_uint64]
        for name in ("px_gen_uniform_pm1", "px_gen_gaussian", "px_gen_sift"):
            fn = getattr(g, name)
            fn.restype = None
            fn.argtypes = [c_uint64, c_int64, c_int64, f32p]
        g.px_gen_normalize_rows.restype = None
        g.px_gen_normalize_rows.argtypes = [f32p, c_int64, c_int64]
        g.px_gen_mask.restype = None
        g.px_gen_mask.argtypes = [c_uint64, c_int64, c_int64, c_double, u8p]
        g.px_gen_max_threads.restype = c_int
        g.px_gen_max_threads.argtypes = []
        _gen = g
    return _gen


def _f32(n: int) -> np.ndarray:
    return np.empty(n, dtype=np.float32)


def _fp(a: np.ndarray):
    return a.ctypes.data_as(POINTER(c_float))


def stream_at(seed: int, i: int) -> int:
    return int(_load().px_gen_stream_at(seed, i))


def uniform_pm1(rows: int, dim: int, seed: int) -> np.ndarray:
    """The reference tests' generator (flat.rs:238-250): uniform in [-1, 1]."""
    out = _f32(rows * dim)
    _load().px_gen_uniform_pm1(seed, 0, out.size, _fp(out))
    return out.reshape(rows, dim)


def gaussian(rows: int, dim: int, seed: int) -> np.ndarray:
    out = _f32(rows * dim)
    _load().px_gen_gaussian(seed, 0, out.size, _fp(out))
    return out.reshape(rows, dim)


def unit_gaussian(rows: int, dim: int, seed: int) -> np.ndarray:
    out = gaussian(rows, dim, seed)
    _load().px_gen_normalize_rows(_fp(out), rows, dim)
    return out


def sift_like(rows: int, dim: int, seed: int) -> np.ndarray:
    out = _f32(rows * dim)
    _load().px_gen_sift(seed, 0, out.size, _fp(out))
    return out.reshape(rows, dim)


def mask(n: int, p: float, seed: int) -> np.ndarray:
    out = np.empty(n, dtype=np.uint8)
    _load().px_gen_mask(seed, 0, n, float(p), out.ctypes.data_as(POINTER(c_uint8)))
    return out.view(np.bool_)


CONFIGS = {
    1: dict(kind="flat", metric="L2", n=10_000, dim=128, nq=100, k=(10,), dist="gaussian",
            mask=None),
    2: dict(kind="flat", metric="IP", n=100_000, dim=384, nq=1_000, k=(10,), dist="unit",
            mask=None),
    3: dict(kind="flat", metric="L2", n=1_000_000, dim=128, nq=10_000, k=(10, 100),
            dist="sift", mask=None),
    4: dict(kind="pq", metric="L2", n=1_000_000, dim=128, nq=10_000, k=(10,), dist="gaussian",
            mask=0.5, m=16, nbits=8, train_sample=50_000, train_iters=25, seed=24301),
    5: dict(kind="flat", metric="IP", n=10_000_000, dim=384, nq=16_384, k=(100,), dist="unit",
            mask=0.1),
}


def _draw(dist: str, rows: int, dim: int, seed: int) -> np.ndarray:
    if dist == "gaussian":
        return gaussian(rows, dim, seed)
    if dist == "unit":
        return unit_gaussian(rows, dim, seed)
    if dist == "sift":
        return sift_like(rows, dim, seed)
    raise ValueError(dist)


def corpus(c: int, rows: int | None = None) -> np.ndarray:
    cfg = CONFIGS[c]
    return _draw(cfg["dist"], cfg["n"] if rows is None else rows, cfg["dim"], 1000 * c + 1)


def queries(c: int, rows: int | None = None) -> np.ndarray:
    cfg = CONFIGS[c]
    return _draw(cfg["dist"], cfg["nq"] if rows is None else rows, cfg["dim"], 1000 * c + 2)


def config_mask(c: int, n: int | None = None) -> np.ndarray | None:
    cfg = CONFIGS[c]
    if cfg["mask"] is None:
        return None
    return mask(cfg["n"] if n is None else n, cfg["mask"], 1000 * c + 3)
