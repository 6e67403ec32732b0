"""Chamfer distance (reference: torch_point_ops/chamfer/__init__.py:1-75).

torch.ops.torch_point_ops_chamfer.chamfer_forward / chamfer_backward run the
gfx950 kernels of libtpo_hip.so; this module adds the autograd formula and
the FakeTensor kernels, as the reference does.
"""
import torch

from .. import _C  # noqa: F401


def _chamfer_backward(ctx, grad_dist1, grad_dist2, grad_idx1, grad_idx2):
    # index outputs carry no gradient (reference chamfer/__init__.py:6-11);
    # gradients are not materialised, so an unused distance output arrives
    # as None and counts as zeros
    xyz1, xyz2, idx1, idx2 = ctx.saved_tensors
    if grad_dist1 is None and grad_dist2 is None:
        return None, None
    if grad_dist1 is None:
        grad_dist1 = torch.zeros(idx1.shape, dtype=xyz1.dtype, device=xyz1.device)
    if grad_dist2 is None:
        grad_dist2 = torch.zeros(idx2.shape, dtype=xyz2.dtype, device=xyz2.device)
    return torch.ops.torch_point_ops_chamfer.chamfer_backward(
        xyz1, xyz2, idx1, idx2, grad_dist1, grad_dist2
    )


def _chamfer_setup_context(ctx, inputs, output):
    xyz1, xyz2 = inputs
    _d1, _d2, idx1, idx2 = output
    ctx.save_for_backward(xyz1, xyz2, idx1, idx2)
    ctx.set_materialize_grads(False)  # no zero tensors for the index outputs


torch.library.register_autograd(
    "torch_point_ops_chamfer::chamfer_forward",
    _chamfer_backward,
    setup_context=_chamfer_setup_context,
)


@torch.library.register_fake("torch_point_ops_chamfer::chamfer_forward")
def _chamfer_forward_fake(xyz1, xyz2):
    b, n = xyz1.shape[0], xyz1.shape[1]
    m = xyz2.shape[1]
    like = dict(device=xyz1.device)
    return (
        torch.empty(b, n, dtype=xyz1.dtype, **like),
        torch.empty(b, m, dtype=xyz1.dtype, **like),
        torch.empty(b, n, dtype=torch.int32, **like),
        torch.empty(b, m, dtype=torch.int32, **like),
    )


@torch.library.register_fake("torch_point_ops_chamfer::chamfer_backward")
def _chamfer_backward_fake(xyz1, xyz2, idx1, idx2, grad_dist1, grad_dist2):
    return torch.empty_like(xyz1), torch.empty_like(xyz2)


# chamfer_loss_forward's autograd is registered in C++ (torch_ops.cpp,
# ChamferLossFunction): the training step's backward runs no Python.


@torch.library.register_fake("torch_point_ops_chamfer::chamfer_loss_forward")
def _chamfer_loss_forward_fake(xyz1, xyz2, mean):
    b, n, m = xyz1.shape[0], xyz1.shape[1], xyz2.shape[1]
    return (
        torch.empty((), dtype=xyz1.dtype, device=xyz1.device),
        torch.empty(b, n, dtype=torch.int32, device=xyz1.device),
        torch.empty(b, m, dtype=torch.int32, device=xyz1.device),
    )


@torch.library.register_fake("torch_point_ops_chamfer::chamfer_loss_backward")
def _chamfer_loss_backward_fake(xyz1, xyz2, idx1, idx2, grad_loss, mean):
    return torch.empty_like(xyz1), torch.empty_like(xyz2)


def chamfer_loss(xyz1: torch.Tensor, xyz2: torch.Tensor, mean: bool = True) -> torch.Tensor:
    """mean(dist1) + mean(dist2) (or the sums) of chamfer_distance(xyz1, xyz2),
    reduced inside the forward kernels; the backward spreads the loss gradient
    over the points inside the backward kernel.  Deterministic; equal to the
    unfused reduction up to the order of the float sums."""
    loss, _i1, _i2 = torch.ops.torch_point_ops_chamfer.chamfer_loss_forward(
        xyz1.contiguous(), xyz2.contiguous(), mean
    )
    return loss


def chamfer_distance(xyz1: torch.Tensor, xyz2: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Squared distance from every point to its nearest neighbour in the other cloud.

    Args:
        xyz1: (B, N, 3) point cloud 1.
        xyz2: (B, M, 3) point cloud 2.

    Returns:
        dist1 (B, N) and dist2 (B, M), in the input dtype.  Inputs need not be
        contiguous.
    """
    d1, d2, _i1, _i2 = torch.ops.torch_point_ops_chamfer.chamfer_forward(
        xyz1.contiguous(), xyz2.contiguous()
    )
    return d1, d2


from .chamfer import ChamferDistance  # noqa: E402
