"""``proxima._core``: the module name the reference's PyO3 extension has
(crates/py/src/lib.rs:685-692 adds Metric, FlatIndex, HnswIndex, PqIndex and __version__).
FlatIndex, PqIndex, Metric and __version__ are the MI355X backend's (proxima_amd._core)."""
from proxima_amd._core import FlatIndex, Metric, PqIndex, __version__


class HnswIndex:
    """Placeholder for the reference's HNSW graph index (crates/core/src/hnsw.rs), which is
    approximate graph search and not part of this exact-search backend."""

    def __init__(self, *args, **kwargs):
        raise NotImplementedError(
            "HnswIndex is not provided by the MI355X backend: it serves FlatIndex (exact "
            "search) and PqIndex (product-quantization ADC scan) only")

    @staticmethod
    def load(path):
        raise NotImplementedError(
            "HnswIndex is not provided by the MI355X backend: it serves FlatIndex (exact "
            "search) and PqIndex (product-quantization ADC scan) only")


__all__ = ["FlatIndex", "HnswIndex", "Metric", "PqIndex", "__version__"]
