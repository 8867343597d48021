"""proxima -- the reference's import path, served by the MI355X exact-search backend.

``from proxima import FlatIndex, Metric, PqIndex`` works unchanged for callers of the
reference's Python package (python/proxima/__init__.py:1-4, which re-exports its names from
the compiled module ``proxima._core``, pyproject.toml:21-24). The classes are those of
``proxima_amd`` (searches on a gfx950 GPU through libproxima_px.so). ``HnswIndex``, the
reference's approximate graph index, is outside this backend: the name imports, and
constructing one raises NotImplementedError.
"""
from ._core import FlatIndex, HnswIndex, Metric, PqIndex, __version__

__all__ = ["FlatIndex", "HnswIndex", "PqIndex", "Metric"]
