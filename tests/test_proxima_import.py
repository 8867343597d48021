"""The reference's import path (python/proxima/__init__.py:1-4, module proxima._core per
pyproject.toml:21-24) resolves to the MI355X backend's classes, with no caller change."""
import pytest


def test_reference_import_path():
    import proxima
    import proxima_amd
    from proxima import FlatIndex, HnswIndex, Metric, PqIndex  # noqa: F401
    from proxima._core import FlatIndex as CoreFlat
    from proxima._core import __version__

    assert proxima.FlatIndex is proxima_amd.FlatIndex is CoreFlat
    assert proxima.PqIndex is proxima_amd.PqIndex
    assert proxima.Metric is proxima_amd.Metric
    assert __version__ == proxima.__version__ == "0.1.0"
    assert sorted(proxima.__all__) == ["FlatIndex", "HnswIndex", "Metric", "PqIndex"]
    assert Metric.L2 == 0 and Metric.InnerProduct == 1
    idx = FlatIndex(8)  # defaults as lib.rs:72-79: metric InnerProduct
    assert idx.metric == Metric.InnerProduct and idx.dim == 8 and idx.size == 0


def test_hnsw_is_not_provided():
    from proxima import HnswIndex

    with pytest.raises(NotImplementedError, match="HnswIndex"):
        HnswIndex(dim=8)
    with pytest.raises(NotImplementedError):
        HnswIndex.load("x.sfidx")
