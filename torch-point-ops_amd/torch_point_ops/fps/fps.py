"""FPS / gather modules (reference: torch_point_ops/fps/fps.py:5-214)."""
import torch

from . import _gather_xyz, furthest_point_sampling, gather_points, quick_furthest_point_sampling


class FarthestPointSampling(torch.nn.Module):
    """forward(points (N,P,3)) -> indices, or (indices, sampled (N,nsamples,3))."""

    def __init__(self, nsamples, return_gathered=False):
        super().__init__()
        if nsamples <= 0:
            raise ValueError(f"nsamples must be positive, but got {nsamples}")
        self.nsamples = nsamples
        self.return_gathered = return_gathered

    def forward(self, points):
        indices = furthest_point_sampling(points, self.nsamples)
        if self.return_gathered:
            return indices, _gather_xyz(points, indices)
        return indices


class PointGatherer(torch.nn.Module):
    """forward(points (N,C,P), indices (N,M)) -> (N,C,M)."""

    def forward(self, points, indices):
        return gather_points(points, indices)


class FPSFunction(torch.nn.Module):
    """Functional FPS module: forward(points, nsamples, return_gathered=False)."""

    def forward(self, points, nsamples, return_gathered=False):
        indices = furthest_point_sampling(points, nsamples)
        if return_gathered:
            return indices, _gather_xyz(points, indices)
        return indices


class QuickFarthestPointSampling(torch.nn.Module):
    """Quick-FPS module; returns the exact furthest point sampling indices."""

    def __init__(self, nsamples, kd_depth=4, return_gathered=False):
        super().__init__()
        if nsamples <= 0:
            raise ValueError(f"nsamples must be positive, but got {nsamples}")
        if kd_depth <= 0 or kd_depth > 10:
            raise ValueError(f"kd_depth must be between 1 and 10, but got {kd_depth}")
        self.nsamples = nsamples
        self.kd_depth = kd_depth
        self.return_gathered = return_gathered

    def forward(self, points):
        indices = quick_furthest_point_sampling(points, self.nsamples, self.kd_depth)
        if self.return_gathered:
            return indices, _gather_xyz(points, indices)
        return indices


class QuickFPSFunction(torch.nn.Module):
    """Functional quick-FPS module: forward(points, nsamples, kd_depth=4, return_gathered=False)."""

    def forward(self, points, nsamples, kd_depth=4, return_gathered=False):
        indices = quick_furthest_point_sampling(points, nsamples, kd_depth)
        if return_gathered:
            return indices, _gather_xyz(points, indices)
        return indices


fps_function = FPSFunction()
quick_fps_function = QuickFPSFunction()
