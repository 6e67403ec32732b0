"""Furthest point sampling and gather_points
(reference: torch_point_ops/fps/__init__.py:1-329).

torch.ops.torch_point_ops_fps.{fps_forward, gather_points_forward,
gather_points_backward} and torch_point_ops_quick_fps.quick_fps_forward run
the gfx950 kernels of libtpo_hip.so.  quick_fps_forward is served by the
exact FPS kernel (kd_depth is validated only), so the quick variants return
exactly the furthest point sampling indices.
"""
import torch

from .. import _C  # noqa: F401


def _gather_points_backward(ctx, grad_output):
    (idx,) = ctx.saved_tensors
    grad_points = torch.ops.torch_point_ops_fps.gather_points_backward(
        grad_output, idx, ctx.n_points
    )
    return grad_points, None


def _gather_points_setup_context(ctx, inputs, output):
    points, idx = inputs
    ctx.save_for_backward(idx)
    ctx.n_points = points.shape[2]


torch.library.register_autograd(
    "torch_point_ops_fps::gather_points_forward",
    _gather_points_backward,
    setup_context=_gather_points_setup_context,
)


@torch.library.register_fake("torch_point_ops_fps::fps_forward")
def _fps_forward_fake(points, nsamples):
    return torch.empty(points.shape[0], nsamples, device=points.device, dtype=torch.int64)


@torch.library.register_fake("torch_point_ops_fps::gather_points_forward")
def _gather_points_forward_fake(points, idx):
    return torch.empty(points.shape[0], points.shape[1], idx.shape[1], device=points.device,
                       dtype=points.dtype)


@torch.library.register_fake("torch_point_ops_fps::gather_points_backward")
def _gather_points_backward_fake(grad_output, idx, n_points):
    return torch.empty(grad_output.shape[0], grad_output.shape[1], n_points,
                       device=grad_output.device, dtype=grad_output.dtype)


@torch.library.register_fake("torch_point_ops_quick_fps::quick_fps_forward")
def _quick_fps_forward_fake(points, nsamples, kd_depth=4):
    return torch.empty(points.shape[0], nsamples, device=points.device, dtype=torch.int64)


def _check_fps_args(points, nsamples):
    if points.dim() != 3 or points.shape[2] != 3:
        raise ValueError(f"Expected points to have shape (N, P, 3), but got {points.shape}")
    if nsamples <= 0:
        raise ValueError(f"nsamples must be positive, but got {nsamples}")
    if nsamples > points.shape[1]:
        raise ValueError(
            f"nsamples ({nsamples}) cannot exceed number of points ({points.shape[1]})")


def furthest_point_sampling(points, nsamples):
    """Indices (N, nsamples) int64 of iteratively furthest points, starting at index 0.

    Points with |p|^2 <= 1e-3 are never selected (reference fps.cu:142-143).
    """
    _check_fps_args(points, nsamples)
    return torch.ops.torch_point_ops_fps.fps_forward(points.contiguous(), nsamples)


def gather_points(points, idx):
    """out[n, c, m] = points[n, c, idx[n, m]]; differentiable in points.

    Args: points (N, C, P), idx (N, M) int64.  Returns (N, C, M).
    """
    if points.dim() != 3:
        raise ValueError(f"Expected points to have 3 dimensions (N, C, P), but got {points.dim()}")
    if idx.dim() != 2:
        raise ValueError(f"Expected idx to have 2 dimensions (N, M), but got {idx.dim()}")
    if points.shape[0] != idx.shape[0]:
        raise ValueError(
            f"Batch dimensions must match: points {points.shape[0]} vs idx {idx.shape[0]}")
    return torch.ops.torch_point_ops_fps.gather_points_forward(points.contiguous(),
                                                               idx.contiguous())


def _gather_xyz(points, indices):
    # (N, P, 3) -> gather on the (N, 3, P) view -> (N, nsamples, 3)
    return gather_points(points.transpose(1, 2), indices).transpose(1, 2)


def farthest_point_sample_and_gather(points, nsamples):
    """(indices (N, nsamples), sampled points (N, nsamples, 3))."""
    indices = furthest_point_sampling(points, nsamples)
    return indices, _gather_xyz(points, indices)


def quick_furthest_point_sampling(points, nsamples, kd_depth=4):
    """Same indices as furthest_point_sampling; kd_depth must lie in [1, 10]."""
    _check_fps_args(points, nsamples)
    if kd_depth <= 0 or kd_depth > 10:
        raise ValueError(f"kd_depth must be between 1 and 10, but got {kd_depth}")
    return torch.ops.torch_point_ops_quick_fps.quick_fps_forward(points.contiguous(), nsamples,
                                                                 kd_depth)


def quick_farthest_point_sample_and_gather(points, nsamples, kd_depth=4):
    indices = quick_furthest_point_sampling(points, nsamples, kd_depth)
    return indices, _gather_xyz(points, indices)


from .fps import (  # noqa: E402
    FarthestPointSampling,
    PointGatherer,
    FPSFunction,
    QuickFarthestPointSampling,
    QuickFPSFunction,
    fps_function,
    quick_fps_function,
)

__all__ = [
    "furthest_point_sampling",
    "gather_points",
    "farthest_point_sample_and_gather",
    "quick_furthest_point_sampling",
    "quick_farthest_point_sample_and_gather",
    "FarthestPointSampling",
    "PointGatherer",
    "FPSFunction",
    "QuickFarthestPointSampling",
    "QuickFPSFunction",
    "fps_function",
    "quick_fps_function",
]
