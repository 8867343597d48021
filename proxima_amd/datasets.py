"""TEXMEX vector files (.fvecs / .ivecs) and the SIFT1M ground-truth check.

Follows bench/datasets.py:9-40 and the recall/ground-truth helpers of
bench/harness.py:201-218 and bench/bench_sift.py:44-60 in the reference. Each record of an
.fvecs (.ivecs) file is a little-endian int32 dimension d followed by d float32 (int32)
values; every record of a file has the same d. Files are memory-mapped, so SIFT1M's 516 MB
base set is not read twice, and a file whose records do not all carry the first record's
dimension is rejected instead of being reshaped into garbage.
"""
from __future__ import annotations

from dataclasses import dataclass
from pathlib import Path

import numpy as np


def _read_vecs(path, dtype) -> np.ndarray:
    if Path(path).stat().st_size == 0:
        return np.empty((0, 0), dtype=dtype)
    raw = np.memmap(path, dtype="<i4", mode="r")
    dim = int(raw[0])
    if dim <= 0 or raw.size % (dim + 1):
        raise ValueError(f"{path}: not a vecs file (dimension {dim}, {raw.size} words)")
    rows = raw.reshape(-1, dim + 1)
    if not (rows[:, 0] == dim).all():
        raise ValueError(f"{path}: records of different dimensions")
    body = np.array(rows[:, 1:], dtype="<i4")  # copied out of the map
    return body.view(np.float32) if dtype == np.float32 else body.astype(np.int32, copy=False)


def read_fvecs(path) -> np.ndarray:
    """float32 [n, d] from an .fvecs file (bench/datasets.py:9-13)."""
    return _read_vecs(path, np.float32)


def read_ivecs(path) -> np.ndarray:
    """int32 [n, d] from an .ivecs file (bench/datasets.py:16-19)."""
    return _read_vecs(path, np.int32)


def _write_vecs(path, arr: np.ndarray, dtype) -> None:
    a = np.ascontiguousarray(arr, dtype=dtype)
    if a.ndim != 2:
        raise ValueError("expected a 2-D array")
    out = np.empty((a.shape[0], a.shape[1] + 1), dtype="<i4")
    out[:, 0] = a.shape[1]
    out[:, 1:] = a.view("<i4")
    out.tofile(path)


def write_fvecs(path, arr: np.ndarray) -> None:
    _write_vecs(path, arr, np.float32)


def write_ivecs(path, arr: np.ndarray) -> None:
    _write_vecs(path, arr, np.int32)


@dataclass
class AnnDataset:
    """A base set, its queries and their ground-truth neighbour ids (bench/datasets.py:22-29)."""
    base: np.ndarray
    queries: np.ndarray
    ground_truth: np.ndarray
    metric: str
    train: np.ndarray | None = None
    name: str = "dataset"


def load_sift(root="data/sift/sift") -> AnnDataset:
    """SIFT1M from its four TEXMEX files (bench/datasets.py:32-40); the learn set is
    optional."""
    root = Path(root)
    learn = root / "sift_learn.fvecs"
    return AnnDataset(base=read_fvecs(root / "sift_base.fvecs"),
                      queries=read_fvecs(root / "sift_query.fvecs"),
                      ground_truth=read_ivecs(root / "sift_groundtruth.ivecs"),
                      metric="L2", train=read_fvecs(learn) if learn.exists() else None,
                      name="SIFT1M")


def exact_ground_truth(base: np.ndarray, queries: np.ndarray, k: int, metric=None) -> np.ndarray:
    """Exact neighbour ids with this backend's FlatIndex (bench/harness.py:201-207; the
    reference's default metric is InnerProduct)."""
    from ._core import FlatIndex, Metric

    idx = FlatIndex(base.shape[1], Metric.InnerProduct if metric is None else metric)
    idx.add(np.ascontiguousarray(base, dtype=np.float32))
    ids, _ = idx.search_batch(np.ascontiguousarray(queries, dtype=np.float32), k=k)
    return ids


def recall_at_k(approx_ids: np.ndarray, gt_ids: np.ndarray, k: int) -> float:
    """Mean over queries of |approx[:k] & truth[:k]| / |truth[:k]|, padding (-1) ignored and
    queries without truth counted as 0 (bench/harness.py:210-218)."""
    approx = np.asarray(approx_ids)[:, :k]
    truth = np.asarray(gt_ids)[:, :k]
    nq = approx.shape[0]
    if nq == 0:
        return 0.0
    total = 0.0
    for a, t in zip(approx, truth):
        ts = set(int(x) for x in t if x >= 0)
        if ts:
            total += len(ts & set(int(x) for x in a if x >= 0)) / len(ts)
    return total / nq
