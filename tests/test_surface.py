"""The Python surface (proxima_amd mirrors the reference's proxima._core, crates/py/src/lib.rs)
on the CPU: names, defaults, dtypes, validation order and exception types, and the
.sfidx persistence layout. Nothing here searches, so no GPU is needed; searches are
covered by the gpu-marked tests."""
import inspect
import struct

import numpy as np
import pytest

from proxima_amd import FlatIndex, Metric, PqIndex, __version__, datagen


def test_module_surface():
    assert __version__ == "0.1.0"  # crates/py/src/lib.rs:691
    assert Metric.L2 == 0 and Metric.InnerProduct == 1  # eq_int, lib.rs:49-54
    sig = inspect.signature(FlatIndex.__init__)
    assert sig.parameters["metric"].default == Metric.InnerProduct  # lib.rs:73
    assert inspect.signature(FlatIndex.search_batch).parameters["k"].default == 10
    assert inspect.signature(FlatIndex.search_batch).parameters["num_threads"].default == 0
    p = inspect.signature(PqIndex.__init__).parameters  # lib.rs:450-452
    assert (p["metric"].default, p["m"].default, p["nbits"].default, p["train_iters"].default,
            p["train_sample"].default, p["seed"].default) == (
        Metric.InnerProduct, 8, 8, 25, 50000, 24301)
    for name in ("search", "search_batch", "search_filtered", "search_batch_filtered"):
        assert hasattr(FlatIndex, name) and hasattr(PqIndex, name)


def test_flat_validation():
    with pytest.raises(ValueError, match="dim must be > 0"):
        FlatIndex(0)
    with pytest.raises(OverflowError):
        FlatIndex(-3)
    idx = FlatIndex(8, Metric.L2)
    with pytest.raises(ValueError, match="vector dim 9 does not match index dim 8"):
        idx.add(np.zeros((10, 9), dtype=np.float32))
    with pytest.raises(TypeError):
        idx.add(np.zeros((10, 8), dtype=np.float64))  # PyReadonlyArray<f32>: no casting
    with pytest.raises(TypeError):
        idx.add(np.zeros(8, dtype=np.float32))
    with pytest.raises(ValueError, match="NaN or infinite"):
        idx.add(np.full((2, 8), np.nan, dtype=np.float32))
    assert idx.size == 0
    idx.add(np.zeros((10, 8), dtype=np.float32))
    with pytest.raises(ValueError, match="query dim mismatch"):
        idx.search(np.zeros(7, dtype=np.float32), k=3)
    with pytest.raises(ValueError, match="query dim mismatch"):
        idx.search_batch(np.zeros((2, 7), dtype=np.float32))
    with pytest.raises(ValueError, match="mask length 9 must equal index size 10"):
        idx.search_filtered(np.zeros(8, dtype=np.float32), np.ones(9, dtype=bool))
    with pytest.raises(TypeError):
        idx.search_filtered(np.zeros(8, dtype=np.float32), np.ones(10, dtype=np.uint8))
    with pytest.raises(ValueError, match="NaN or infinite"):
        idx.search(np.full(8, np.inf, dtype=np.float32), k=0)
    with pytest.raises(OverflowError):
        idx.search(np.zeros(8, dtype=np.float32), k=-1)


def test_metric_and_metadata():
    # tests/test_engine.py:80-94
    idx = FlatIndex(dim=16, metric=Metric.L2)
    assert idx.metric == Metric.L2 and idx.dim == 16
    idx.add(np.zeros((4, 16), dtype=np.float32))
    assert idx.memory_bytes == 4 * 16 * 4
    idx.add(np.ones((3, 16), dtype=np.float32))
    assert idx.size == len(idx) == 7


def test_non_contiguous_input_is_copied():
    # crates/py/src/lib.rs:18-31; tests/test_engine.py:97-111
    data = datagen.gaussian(50, 12, 3)
    idx = FlatIndex(12, Metric.L2)
    idx.add(np.asfortranarray(data))
    idx.add(data[::2])
    assert np.array_equal(idx.vectors(), np.concatenate([data, data[::2]]))


def test_pq_validation():
    with pytest.raises(ValueError, match="m must be >= 1"):
        PqIndex(dim=8, m=0)
    with pytest.raises(ValueError, match="divisible by m"):
        PqIndex(dim=10, m=3)
    with pytest.raises(ValueError, match="nbits"):
        PqIndex(dim=8, m=2, nbits=9)
    pq = PqIndex(dim=16, metric=Metric.L2, m=4, nbits=4)
    assert not pq.is_trained and pq.size == 0 and pq.memory_bytes == 0
    assert pq.compression_ratio == 0.0
    with pytest.raises(ValueError, match="not trained; call train"):
        pq.add(np.zeros((3, 16), dtype=np.float32))
    with pytest.raises(ValueError, match="index is not trained"):
        pq.search(np.zeros(16, dtype=np.float32))
    with pytest.raises(ValueError, match="index is not trained"):
        pq.search_batch_filtered(np.zeros((1, 16), dtype=np.float32), np.ones(0, dtype=bool))
    with pytest.raises(ValueError, match="training set too small: need at least 16 rows"):
        pq.train(np.zeros((15, 16), dtype=np.float32))
    with pytest.raises(ValueError, match="training dim mismatch"):
        pq.train(np.zeros((20, 8), dtype=np.float32))
    bad = datagen.gaussian(40, 16, 1)
    bad[3, 3] = np.nan
    with pytest.raises(ValueError, match="NaN or infinite"):
        pq.train(bad)
    pq.train(datagen.gaussian(40, 16, 2))
    assert pq.is_trained
    with pytest.raises(ValueError, match="vector dim mismatch"):
        pq.add(np.zeros((3, 8), dtype=np.float32))
    with pytest.raises(ValueError, match="query dim mismatch"):
        pq.search(np.zeros(8, dtype=np.float32))


def test_pq_sizes_and_compression():
    # tests/test_pq.py:59-66 and pq.rs:463-472 (iterations do not change the sizes)
    base = datagen.gaussian(40000, 64, 0)
    pq = PqIndex(dim=64, metric=Metric.L2, m=8, train_iters=2)
    pq.train(base)
    pq.add(base)
    assert pq.size == len(pq) == 40000
    assert pq.raw_bytes == 40000 * 64 * 4
    assert pq.memory_bytes == 40000 * 8 + 8 * 256 * 8 * 4  # pq.rs:250-252
    assert pq.compression_ratio > 20


def test_flat_file_layout_known_answer(tmp_path):
    # bincode 1.x fixint little-endian of FlatIndex {dim: usize, metric: Metric, n: usize,
    # data: Vec<f32>} (flat.rs:34-40, lib.rs:19-30): u64, u32 variant index, u64, u64 len, f32s
    idx = FlatIndex(2, Metric.L2)
    idx.add(np.array([[1, 2], [3, 4]], dtype=np.float32))
    path = tmp_path / "flat.sfidx"
    idx.save(str(path))
    expect = (struct.pack("<Q", 2) + struct.pack("<I", 0) + struct.pack("<Q", 2) +
              struct.pack("<Q", 4) + struct.pack("<4f", 1, 2, 3, 4))
    assert path.read_bytes() == expect
    loaded = FlatIndex.load(str(path))
    assert loaded.metric == Metric.L2 and loaded.dim == 2 and loaded.size == 2
    assert np.array_equal(loaded.vectors(), [[1, 2], [3, 4]])


def test_pq_file_layout_known_answer(tmp_path):
    # PqIndex {metric, pq: {dim, m, dsub, k: usize, codebooks: Vec<f32>}, codes: Vec<u8>,
    # n: usize} (pq.rs:39-46, 217-223)
    pq = PqIndex(4, Metric.InnerProduct, m=2, nbits=1, train_iters=3)
    pq.train(datagen.gaussian(10, 4, 1))
    pq.add(datagen.gaussian(3, 4, 2))
    path = tmp_path / "pq.sfidx"
    pq.save(str(path))
    books, codes = pq.codebooks(), pq.codes()
    expect = (struct.pack("<I", 1) + struct.pack("<4Q", 4, 2, 2, 2) + struct.pack("<Q", 8) +
              books.astype("<f4").tobytes() + struct.pack("<Q", 6) + codes.tobytes() +
              struct.pack("<Q", 3))
    assert path.read_bytes() == expect
    loaded = PqIndex.load(str(path))
    assert loaded.is_trained and loaded.size == 3 and loaded.m == 2
    assert loaded.metric == Metric.InnerProduct
    assert np.array_equal(loaded.codebooks(), books) and np.array_equal(loaded.codes(), codes)
    # crates/py/src/lib.rs:677: loaded indexes get the default training parameters
    assert (loaded._train_iters, loaded._train_sample, loaded._seed) == (25, 50000, 24301)


def test_persistence_errors(tmp_path):
    with pytest.raises(ValueError, match="not trained"):
        PqIndex(dim=64, metric=Metric.L2, m=8).save(str(tmp_path / "x.sfidx"))
    with pytest.raises(IOError):
        FlatIndex.load(str(tmp_path / "missing.sfidx"))
    (tmp_path / "short.sfidx").write_bytes(b"\x02\x00")
    with pytest.raises(IOError):
        FlatIndex.load(str(tmp_path / "short.sfidx"))
    (tmp_path / "badvariant.sfidx").write_bytes(struct.pack("<QI", 2, 7))
    with pytest.raises(IOError):
        FlatIndex.load(str(tmp_path / "badvariant.sfidx"))
