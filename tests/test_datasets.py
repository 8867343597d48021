"""TEXMEX .fvecs/.ivecs reading and recall@k (CPU only; bench/datasets.py:9-40,
bench/harness.py:210-218)."""
import numpy as np
import pytest

from proxima_amd import datagen, datasets


def test_fvecs_ivecs_round_trip_and_layout(tmp_path):
    x = datagen.gaussian(37, 13, 1)
    g = np.arange(37 * 5, dtype=np.int32).reshape(37, 5)[::-1]
    datasets.write_fvecs(tmp_path / "a.fvecs", x)
    datasets.write_ivecs(tmp_path / "a.ivecs", g)
    # the byte layout itself: int32 dimension, then the row's values, per record
    raw = np.fromfile(tmp_path / "a.fvecs", dtype="<i4").reshape(37, 14)
    assert (raw[:, 0] == 13).all()
    assert np.array_equal(raw[:, 1:].view("<f4"), x)
    assert np.array_equal(datasets.read_fvecs(tmp_path / "a.fvecs"), x)
    got = datasets.read_ivecs(tmp_path / "a.ivecs")
    assert got.dtype == np.int32 and np.array_equal(got, g)


def test_hand_built_fvecs_record(tmp_path):
    # two records of d = 2: [1.5, -2.0] and [0.25, 8.0]
    words = np.array([2, 0, 0, 2, 0, 0], dtype="<i4")
    words[1:3] = np.array([1.5, -2.0], dtype="<f4").view("<i4")
    words[4:6] = np.array([0.25, 8.0], dtype="<f4").view("<i4")
    words.tofile(tmp_path / "h.fvecs")
    assert datasets.read_fvecs(tmp_path / "h.fvecs").tolist() == [[1.5, -2.0], [0.25, 8.0]]


def test_corrupt_files_rejected(tmp_path):
    np.array([3, 1, 2, 3, 2, 1, 2], dtype="<i4").tofile(tmp_path / "bad.ivecs")
    with pytest.raises(ValueError):
        datasets.read_ivecs(tmp_path / "bad.ivecs")
    np.array([3, 1, 2, 3, 4, 1, 2, 3], dtype="<i4").tofile(tmp_path / "mixed.ivecs")
    with pytest.raises(ValueError):
        datasets.read_ivecs(tmp_path / "mixed.ivecs")


def test_load_sift_layout(tmp_path):
    base = datagen.sift_like(50, 128, 2)
    q = datagen.sift_like(4, 128, 3)
    gt = np.tile(np.arange(100, dtype=np.int32), (4, 1))
    datasets.write_fvecs(tmp_path / "sift_base.fvecs", base)
    datasets.write_fvecs(tmp_path / "sift_query.fvecs", q)
    datasets.write_ivecs(tmp_path / "sift_groundtruth.ivecs", gt)
    ds = datasets.load_sift(tmp_path)
    assert ds.name == "SIFT1M" and ds.metric == "L2" and ds.train is None
    assert np.array_equal(ds.base, base) and np.array_equal(ds.queries, q)
    assert np.array_equal(ds.ground_truth, gt)


def test_recall_at_k_semantics():
    gt = np.array([[1, 2, 3, 4], [5, 6, -1, -1], [-1, -1, -1, -1]])
    approx = np.array([[4, 3, 9, 9], [6, 7, 8, 9], [1, 2, 3, 4]])
    # query 0: {1,2,3} vs {4,3,9} -> 1/3 at k=3; query 1: {5,6} vs {6,7,8} -> 1/2;
    # query 2: no truth -> 0, still counted in the mean
    assert datasets.recall_at_k(approx, gt, 3) == pytest.approx((1 / 3 + 1 / 2 + 0) / 3)
    assert datasets.recall_at_k(approx, gt, 4) == pytest.approx((2 / 4 + 1 / 2) / 3)
    assert datasets.recall_at_k(approx[:0], gt[:0], 3) == 0.0
