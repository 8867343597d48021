"""Python surface of the MI355X backend, mirroring the reference's ``proxima._core``.

Same class names, constructor defaults, keyword names, return dtypes and shapes, and
exception types as the PyO3 module in crates/py/src/lib.rs (Metric 49-54, FlatIndex
65-230, PqIndex 440-683). Validation happens before any compute, in the reference's
order. Every search runs in libproxima_px.so on the GPU; there is no CPU search path,
so on a machine without a gfx950 device a search raises RuntimeError.

``HnswIndex`` (the reference's graph ANN index) is not part of this backend.
"""
from __future__ import annotations

import ctypes
import enum
import operator
import os
import struct

import numpy as np

from . import _lib
from ._lib import (PX_ERR_ARG, PX_ERR_BAD_K, PX_ERR_DIM, PX_ERR_NONFINITE, PX_ERR_UNTRAINED,
                   PX_OK)

__version__ = "0.1.0"


class Metric(enum.IntEnum):
    """crates/core/src/metric.rs:3-7; compares equal to its variant index (PyO3 eq_int)."""

    L2 = 0
    InnerProduct = 1

    def __repr__(self) -> str:
        return f"Metric.{self.name}"

    __str__ = __repr__


def _usize(value, name: str) -> int:
    """PyO3 usize extraction: any __index__ integer, OverflowError when negative."""
    try:
        v = operator.index(value)
    except TypeError:
        raise TypeError(f"argument '{name}': '{type(value).__name__}' object cannot be "
                        "interpreted as an integer") from None
    if v < 0:
        raise OverflowError(f"argument '{name}': can't convert negative int to unsigned")
    return v


def _metric(value) -> Metric:
    if not isinstance(value, Metric):
        raise TypeError(f"argument 'metric': '{type(value).__name__}' object is not a Metric")
    return value


def _f32_array(a, ndim: int, name: str) -> np.ndarray:
    """PyReadonlyArray{1,2}<f32>: float32 ndarray of the given rank, else TypeError.
    Non-contiguous input is copied (crates/py/src/lib.rs:18-31)."""
    if not isinstance(a, np.ndarray) or a.dtype != np.float32 or a.ndim != ndim:
        raise TypeError(f"argument '{name}': expected a {ndim}-D numpy.ndarray of float32")
    return np.ascontiguousarray(a)


def _bool_array(a, name: str) -> np.ndarray:
    """PyReadonlyArray1<bool> (crates/py/src/lib.rs:33-39)."""
    if not isinstance(a, np.ndarray) or a.dtype != np.bool_ or a.ndim != 1:
        raise TypeError(f"argument '{name}': expected a 1-D numpy.ndarray of bool")
    return np.ascontiguousarray(a)


def _raise(rc: int) -> None:
    msg = _lib.last_error()
    if rc == PX_ERR_NONFINITE:
        raise ValueError("input must not contain NaN or infinite values")  # lib.rs:41-47
    if rc in (PX_ERR_DIM, PX_ERR_ARG, PX_ERR_UNTRAINED, PX_ERR_BAD_K):
        raise ValueError(msg)
    raise RuntimeError(f"proxima_amd GPU backend error {rc}: {msg}")


def _check(rc: int) -> None:
    if rc != PX_OK:
        _raise(rc)


# ---- bincode 1.x (little-endian, fixint) persistence, crates/core/src/lib.rs:19-30 ------
def _write(path, payload: bytes) -> None:
    try:
        with open(os.fspath(path), "wb") as fh:
            fh.write(payload)
    except OSError as e:
        raise IOError(str(e)) from e


def _read(path) -> bytes:
    try:
        with open(os.fspath(path), "rb") as fh:
            return fh.read()
    except OSError as e:
        raise IOError(str(e)) from e


class _Reader:
    def __init__(self, buf: bytes):
        self.buf = buf
        self.off = 0

    def take(self, n: int) -> bytes:
        if self.off + n > len(self.buf):
            raise IOError("io error: unexpected end of file")
        b = self.buf[self.off:self.off + n]
        self.off += n
        return b

    def u64(self) -> int:
        return struct.unpack("<Q", self.take(8))[0]

    def u32(self) -> int:
        return struct.unpack("<I", self.take(4))[0]

    def metric(self) -> Metric:
        v = self.u32()
        if v > 1:
            raise IOError(f"invalid value: integer `{v}`, expected variant index 0 <= i < 2")
        return Metric(v)

    def f32_vec(self) -> np.ndarray:
        n = self.u64()
        return np.frombuffer(self.take(4 * n), dtype="<f4").astype(np.float32)

    def u8_vec(self) -> np.ndarray:
        n = self.u64()
        return np.frombuffer(self.take(n), dtype=np.uint8).copy()


class FlatIndex:
    """Exact kNN (crates/py/src/lib.rs:65-230 over crates/core/src/flat.rs)."""

    def __init__(self, dim, metric=Metric.InnerProduct):
        dim = _usize(dim, "dim")
        metric = _metric(metric)
        if dim == 0:
            raise ValueError("dim must be > 0")
        lib = _lib.load()
        h = ctypes.c_void_p()
        _check(lib.px_flat_create(int(metric), dim, ctypes.byref(h)))
        self._lib = lib
        self._h = h
        self._dim = dim
        self._metric = metric

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            self._lib.px_flat_destroy(h)
            self._h = None

    # lib.rs:81-94
    def add(self, vectors):
        v = _f32_array(vectors, 2, "vectors")
        if v.shape[1] != self._dim:
            raise ValueError(f"vector dim {v.shape[1]} does not match index dim {self._dim}")
        _check(self._lib.px_flat_add(self._h, _lib.f32p(v), v.shape[0]))

    def _run(self, q: np.ndarray, k: int, mask):
        nq = q.shape[0]
        ids = np.empty((nq, k), dtype=np.int64)
        dists = np.empty((nq, k), dtype=np.float32)
        mp = _lib.u8p(mask.view(np.uint8)) if mask is not None else None
        rc = self._lib.px_flat_search(self._h, _lib.f32p(q), nq, k, mp, _lib.i64p(ids),
                                      _lib.f32p(dists))
        _check(rc)
        return ids, dists

    def _mask(self, mask):
        m = _bool_array(mask, "mask")
        if m.shape[0] != self.size:
            raise ValueError(f"mask length {m.shape[0]} must equal index size {self.size}")
        return m

    # lib.rs:96-112
    def search(self, query, k=10):
        q = _f32_array(query, 1, "query")
        k = _usize(k, "k")
        if q.shape[0] != self._dim:
            raise ValueError("query dim mismatch")
        ids, dists = self._run(q.reshape(1, -1), k, None)
        return ids[0], dists[0]

    # lib.rs:114-139
    def search_batch(self, queries, k=10, num_threads=0):
        q = _f32_array(queries, 2, "queries")
        k = _usize(k, "k")
        _usize(num_threads, "num_threads")  # accepted; the GPU path has no host pool
        if q.shape[1] != self._dim:
            raise ValueError("query dim mismatch")
        return self._run(q, k, None)

    # lib.rs:141-164
    def search_filtered(self, query, mask, k=10):
        q = _f32_array(query, 1, "query")
        k = _usize(k, "k")
        if q.shape[0] != self._dim:
            raise ValueError("query dim mismatch")
        m = self._mask(mask)
        ids, dists = self._run(q.reshape(1, -1), k, m)
        return ids[0], dists[0]

    # lib.rs:166-198
    def search_batch_filtered(self, queries, mask, k=10, num_threads=0):
        q = _f32_array(queries, 2, "queries")
        k = _usize(k, "k")
        _usize(num_threads, "num_threads")
        if q.shape[1] != self._dim:
            raise ValueError("query dim mismatch")
        m = self._mask(mask)
        return self._run(q, k, m)

    @property
    def size(self) -> int:
        return int(self._lib.px_flat_size(self._h))

    @property
    def dim(self) -> int:
        return self._dim

    @property
    def metric(self) -> Metric:
        return self._metric

    @property
    def memory_bytes(self) -> int:
        return int(self._lib.px_flat_memory_bytes(self._h))

    def __len__(self) -> int:
        return self.size

    def vectors(self) -> np.ndarray:
        """All stored rows as an (n, dim) float32 array (read back from HBM)."""
        n = self.size
        out = np.empty((n, self._dim), dtype=np.float32)
        _check(self._lib.px_flat_get_vectors(self._h, 0, n, _lib.f32p(out)))
        return out

    # lib.rs:219-226 (save, load) over flat.rs:34-40: dim u64, metric u32, n u64, data (u64 len, f32...)
    def save(self, path) -> None:
        data = self.vectors()
        head = struct.pack("<QIQQ", self._dim, int(self._metric), data.shape[0], data.size)
        _write(path, head + data.astype("<f4").tobytes())

    @staticmethod
    def load(path) -> "FlatIndex":
        r = _Reader(_read(path))
        dim = r.u64()
        metric = r.metric()
        n = r.u64()
        data = r.f32_vec()
        if dim == 0 or data.size != n * dim:
            raise IOError("corrupt FlatIndex file: data length does not match n * dim")
        idx = FlatIndex(dim, metric)
        if n:
            idx.add(data.reshape(n, dim))
        return idx

    def _timing(self, enable: bool = True) -> None:
        _check(self._lib.px_flat_set_timing(self._h, 1 if enable else 0))

    def _scan_f16(self, enable: bool = True) -> None:
        """Use the fp16 copy of rows exact in fp16 (default on): the collect scan multiplies
        in fp16 where the queries are exact too, the few-query vector scan reads the copy;
        off keeps both on the fp32 rows. Diagnostic; no counterpart in the reference."""
        _check(self._lib.px_flat_set_scan_f16(self._h, 1 if enable else 0))

    def _spin_limit(self, polls: int = 0) -> None:
        """Polls a stage-sync wait of the barrier-free scans makes before it gives up (0: the
        kernels' own, about 5 ms). A give-up fails the search with RuntimeError and writes no
        outputs. Test hook; no counterpart in the reference."""
        _check(self._lib.px_flat_set_spin_limit(self._h, int(polls)))

    def _last_timing(self) -> dict:
        scan, total = ctypes.c_float(), ctypes.c_float()
        splits, blocks = ctypes.c_int(), ctypes.c_int()
        _check(self._lib.px_flat_last_timing(self._h, ctypes.byref(scan), ctypes.byref(total),
                                             ctypes.byref(splits), ctypes.byref(blocks)))
        rounds, path, f16 = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
        _check(self._lib.px_flat_last_rounds(self._h, ctypes.byref(rounds)))
        _check(self._lib.px_flat_last_path(self._h, ctypes.byref(path)))
        _check(self._lib.px_flat_last_scan_f16(self._h, ctypes.byref(f16)))
        return {"scan_ms": scan.value, "total_ms": total.value, "splits": splits.value,
                "blocks": blocks.value, "collect_rounds": rounds.value,
                "path": ("lists", "collect-sampled", "collect-bounded", "vector",
                         "full-sort")[path.value],
                "scan_f16": bool(f16.value)}


class PqIndex:
    """Product quantization with an ADC scan (crates/py/src/lib.rs:440-683 over pq.rs)."""

    def __init__(self, dim, metric=Metric.InnerProduct, m=8, nbits=8, train_iters=25,
                 train_sample=50000, seed=24301):
        dim = _usize(dim, "dim")
        metric = _metric(metric)
        m = _usize(m, "m")
        nbits = _usize(nbits, "nbits")
        train_iters = _usize(train_iters, "train_iters")
        train_sample = _usize(train_sample, "train_sample")
        seed = _usize(seed, "seed")
        if seed >= 1 << 64:
            raise OverflowError("argument 'seed': int too big to convert")
        if m == 0:
            raise ValueError("m must be >= 1")
        if dim == 0 or dim % m != 0:
            raise ValueError("dim must be > 0 and divisible by m")
        if not 1 <= nbits <= 8:
            raise ValueError("nbits must be in 1..=8")
        lib = _lib.load()
        h = ctypes.c_void_p()
        _check(lib.px_pq_create(int(metric), dim, m, nbits, ctypes.byref(h)))
        self._lib = lib
        self._h = h
        self._dim = dim
        self._metric = metric
        self._m = m
        self._nbits = nbits
        self._train_iters = train_iters
        self._train_sample = train_sample
        self._seed = seed

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            self._lib.px_pq_destroy(h)
            self._h = None

    # lib.rs:472-490
    def train(self, training):
        t = _f32_array(training, 2, "training")
        if t.shape[1] != self._dim:
            raise ValueError("training dim mismatch")
        k = 1 << self._nbits
        if t.shape[0] < k:
            raise ValueError(f"training set too small: need at least {k} rows for "
                             f"nbits={self._nbits}, got {t.shape[0]}")
        _check(self._lib.px_pq_train(self._h, _lib.f32p(t), t.shape[0], self._train_iters,
                                     self._train_sample, self._seed))

    # lib.rs:492-504
    def add(self, vectors):
        if not self.is_trained:
            raise ValueError("index is not trained; call train() first")
        v = _f32_array(vectors, 2, "vectors")
        if v.shape[1] != self._dim:
            raise ValueError("vector dim mismatch")
        _check(self._lib.px_pq_add(self._h, _lib.f32p(v), v.shape[0]))

    def _trained(self):
        if not self.is_trained:
            raise ValueError("index is not trained")

    def _run(self, q: np.ndarray, k: int, mask):
        nq = q.shape[0]
        ids = np.empty((nq, k), dtype=np.int64)
        dists = np.empty((nq, k), dtype=np.float32)
        mp = _lib.u8p(mask.view(np.uint8)) if mask is not None else None
        _check(self._lib.px_pq_search(self._h, _lib.f32p(q), nq, k, mp, _lib.i64p(ids),
                                      _lib.f32p(dists)))
        return ids, dists

    def _mask(self, mask):
        m = _bool_array(mask, "mask")
        if m.shape[0] != self.size:
            raise ValueError(f"mask length {m.shape[0]} must equal index size {self.size}")
        return m

    def search(self, query, k=10):
        q = _f32_array(query, 1, "query")
        k = _usize(k, "k")
        self._trained()
        if q.shape[0] != self._dim:
            raise ValueError("query dim mismatch")
        ids, dists = self._run(q.reshape(1, -1), k, None)
        return ids[0], dists[0]

    def search_batch(self, queries, k=10, num_threads=0):
        q = _f32_array(queries, 2, "queries")
        k = _usize(k, "k")
        _usize(num_threads, "num_threads")
        self._trained()
        if q.shape[1] != self._dim:
            raise ValueError("query dim mismatch")
        return self._run(q, k, None)

    def search_filtered(self, query, mask, k=10):
        q = _f32_array(query, 1, "query")
        k = _usize(k, "k")
        self._trained()
        if q.shape[0] != self._dim:
            raise ValueError("query dim mismatch")
        m = self._mask(mask)
        ids, dists = self._run(q.reshape(1, -1), k, m)
        return ids[0], dists[0]

    def search_batch_filtered(self, queries, mask, k=10, num_threads=0):
        q = _f32_array(queries, 2, "queries")
        k = _usize(k, "k")
        _usize(num_threads, "num_threads")
        self._trained()
        if q.shape[1] != self._dim:
            raise ValueError("query dim mismatch")
        m = self._mask(mask)
        return self._run(q, k, m)

    @property
    def is_trained(self) -> bool:
        return bool(self._lib.px_pq_is_trained(self._h))

    @property
    def size(self) -> int:
        return int(self._lib.px_pq_size(self._h)) if self.is_trained else 0

    @property
    def dim(self) -> int:
        return self._dim

    @property
    def m(self) -> int:
        return self._m

    @property
    def metric(self) -> Metric:
        return self._metric

    @property
    def memory_bytes(self) -> int:
        return int(self._lib.px_pq_memory_bytes(self._h))

    @property
    def raw_bytes(self) -> int:
        return int(self._lib.px_pq_raw_bytes(self._h))

    @property
    def compression_ratio(self) -> float:
        mem = self.memory_bytes
        return self.raw_bytes / mem if self.is_trained and mem > 0 else 0.0

    def __len__(self) -> int:
        return self.size

    def codebooks(self) -> np.ndarray:
        ks = 1 << self._nbits
        out = np.empty((self._m, ks, self._dim // self._m), dtype=np.float32)
        _check(self._lib.px_pq_get_codebooks(self._h, _lib.f32p(out)))
        return out

    def codes(self) -> np.ndarray:
        n = self.size
        out = np.empty((n, self._m), dtype=np.uint8)
        _check(self._lib.px_pq_get_codes(self._h, 0, n, _lib.u8p(out)))
        return out

    def add_codes(self, codes) -> None:
        """Append pre-encoded rows (uint8 [n, m])."""
        self._trained()
        c = np.ascontiguousarray(codes, dtype=np.uint8)
        if c.ndim != 2 or c.shape[1] != self._m:
            raise ValueError("codes must have shape (n, m)")
        _check(self._lib.px_pq_add_codes(self._h, _lib.u8p(c), c.shape[0]))

    # lib.rs:662-678 over pq.rs:217-223 / 39-46: metric u32; pq {dim, m, dsub, k: u64,
    # codebooks (u64 len, f32...)}; codes (u64 len, u8...); n u64
    def save(self, path) -> None:
        self._trained()
        books = self.codebooks()
        codes = self.codes()
        ks = 1 << self._nbits
        out = [struct.pack("<I", int(self._metric)),
               struct.pack("<QQQQ", self._dim, self._m, self._dim // self._m, ks),
               struct.pack("<Q", books.size), books.astype("<f4").tobytes(),
               struct.pack("<Q", codes.size), codes.tobytes(),
               struct.pack("<Q", codes.shape[0])]
        _write(path, b"".join(out))

    @staticmethod
    def load(path) -> "PqIndex":
        r = _Reader(_read(path))
        metric = r.metric()
        dim, m, dsub, ks = r.u64(), r.u64(), r.u64(), r.u64()
        books = r.f32_vec()
        codes = r.u8_vec()
        n = r.u64()
        nbits = ks.bit_length() - 1
        if (m == 0 or dim != m * dsub or ks != 1 << nbits or not 1 <= nbits <= 8
                or books.size != m * ks * dsub or codes.size != n * m):
            raise IOError("corrupt PqIndex file")
        # lib.rs:677: train params reset to the defaults, keeping m and nbits
        idx = PqIndex(dim, metric, m=m, nbits=nbits)
        _check(idx._lib.px_pq_set_codebooks(idx._h, _lib.f32p(books)))
        if n:
            idx.add_codes(codes.reshape(n, m))
        return idx

    def _timing(self, enable: bool = True) -> None:
        _check(self._lib.px_pq_set_timing(self._h, 1 if enable else 0))

    def _last_timing(self) -> dict:
        scan, total = ctypes.c_float(), ctypes.c_float()
        splits, blocks = ctypes.c_int(), ctypes.c_int()
        _check(self._lib.px_pq_last_timing(self._h, ctypes.byref(scan), ctypes.byref(total),
                                           ctypes.byref(splits), ctypes.byref(blocks)))
        return {"scan_ms": scan.value, "total_ms": total.value, "splits": splits.value,
                "blocks": blocks.value}
