"""proxima_amd -- MI355X-native exact-search backend for Proxima's FlatIndex and PqIndex.

Drop-in for the reference's ``proxima`` surface on this path
(python/proxima/__init__.py:1-4 re-exports ``FlatIndex, HnswIndex, Metric, PqIndex`` from
``proxima._core``). ``HnswIndex`` (approximate graph search) is not part of this backend.
"""
from ._core import FlatIndex, Metric, PqIndex, __version__
from ._lib import device_count, device_info

__all__ = ["FlatIndex", "PqIndex", "Metric", "device_count", "device_info", "__version__"]
