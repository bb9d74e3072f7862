"""flash_kmeans_cuda — batched Euclidean K-Means on AMD Instinct MI355X (gfx950).

Drop-in for the public surface of OpsiClear/flash-kmeans-cuda
(flash_kmeans_cuda/__init__.py:8-18 of the reference): the same names,
signatures and return conventions, backed by hand-written HIP kernels behind
the C ABI of include/fkc.h.  Importing fails if the HIP library is missing.
"""

from ._version import __version__
from .kmeans import batch_kmeans_Euclid
from .ops import centroid_finalize, centroid_update_sorted, euclid_assign, label_sort
from . import quality

__all__ = [
    "__version__",
    "batch_kmeans_Euclid",
    "euclid_assign",
    "centroid_update_sorted",
    "centroid_finalize",
    "label_sort",
    "quality",
]
