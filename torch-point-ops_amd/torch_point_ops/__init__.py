"""torch_point_ops for MI355X (gfx950).

Drop-in for the reference package's nearest-neighbour path: the same module
layout, functions, nn.Modules and torch.ops registrations
(torch_point_ops/__init__.py:1-30 of the reference), backed by the HIP
kernels of libtpo_hip.so.  Importing fails loudly when the native extension
(_C.so / libtpo_hip.so) is missing; there is no fallback path.
"""
import torch  # noqa: F401  (loads libc10 / libtorch before the extension)

from . import _C  # noqa: F401  (registers the torch.ops schemas and HIP kernels)

from .chamfer import ChamferDistance, chamfer_distance, chamfer_loss
from .emd import EarthMoverDistance, emd, earth_movers_distance
from .knn import KNearestNeighbors, knn_points, knn_gather
from .fps import (
    FarthestPointSampling,
    furthest_point_sampling,
    gather_points,
    farthest_point_sample_and_gather,
    QuickFarthestPointSampling,
    quick_furthest_point_sampling,
    quick_farthest_point_sample_and_gather,
)

__all__ = [
    "ChamferDistance",
    "chamfer_distance",
    "chamfer_loss",
    "EarthMoverDistance",
    "emd",
    "earth_movers_distance",
    "KNearestNeighbors",
    "knn_points",
    "knn_gather",
    "FarthestPointSampling",
    "furthest_point_sampling",
    "gather_points",
    "farthest_point_sample_and_gather",
    "QuickFarthestPointSampling",
    "quick_furthest_point_sampling",
    "quick_farthest_point_sample_and_gather",
]
