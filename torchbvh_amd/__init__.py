"""torchbvh_amd — MI355X-native BVH build and exact k-NN for 2-D/3-D fp32
point clouds, behind the API of torchbvh's build/k-NN path.

Importing the package never compiles anything; the native library
(``libtorchbvh_amd.so``, hand-written HIP for gfx950 behind a C ABI) is loaded
on first use and must have been built (``python -m torchbvh_amd._build``).
"""

import torch  # noqa: F401  (loads torch's HIP runtime before the native library)

from ._bvh_class import BVH
from ._constants import SUPPORTED_DIMS, SUPPORTED_K
from ._geometry import PointGeometry
from ._handles import BVHHandle, BatchedBVHHandle, RaggedBVHHandle, destroy_bvh
from ._multihead import gather_neighbor_values, interpolate_displaced, query_displaced_knn
from ._native import _C
from ._query import build_bvh, query_knn

__version__ = "0.1.0"

__all__ = [
    "BVH",
    "PointGeometry",
    "BVHHandle",
    "BatchedBVHHandle",
    "RaggedBVHHandle",
    "build_bvh",
    "destroy_bvh",
    "query_knn",
    "query_displaced_knn",
    "gather_neighbor_values",
    "interpolate_displaced",
    "SUPPORTED_K",
    "SUPPORTED_DIMS",
]
