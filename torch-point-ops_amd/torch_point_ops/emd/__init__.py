"""Earth mover's distance (reference: torch_point_ops/emd/__init__.py:1-72).

torch.ops.torch_point_ops_emd.emd_forward / emd_backward run the gfx950
kernels of libtpo_hip.so (approximate matching, its cost and gradients);
this module adds the autograd formula and the FakeTensor kernels, as the
reference does.
"""
import torch

from .. import _C  # noqa: F401


def _emd_backward(ctx, grad_cost, grad_match):
    # match carries no gradient (reference emd/__init__.py:6-11); gradients
    # are not materialised, so an unused cost arrives as None
    xyz1, xyz2, match = ctx.saved_tensors
    if grad_cost is None:
        return None, None
    return torch.ops.torch_point_ops_emd.emd_backward(grad_cost, xyz1, xyz2, match)


def _emd_setup_context(ctx, inputs, output):
    xyz1, xyz2 = inputs
    _, match = output
    ctx.save_for_backward(xyz1, xyz2, match)
    ctx.set_materialize_grads(False)  # no (B, m, n) zero tensor for match's gradient


torch.library.register_autograd(
    "torch_point_ops_emd::emd_forward", _emd_backward, setup_context=_emd_setup_context
)


@torch.library.register_fake("torch_point_ops_emd::emd_forward")
def _(xyz1, xyz2):
    batch_size, n, _ = xyz1.shape
    m = xyz2.shape[1]
    cost = torch.empty(batch_size, device=xyz1.device, dtype=xyz1.dtype)
    match = torch.empty(batch_size, m, n, device=xyz1.device, dtype=xyz1.dtype)
    return cost, match


@torch.library.register_fake("torch_point_ops_emd::emd_backward")
def _(grad_cost, xyz1, xyz2, match):
    return torch.empty_like(xyz1), torch.empty_like(xyz2)


def earth_movers_distance(xyz1: torch.Tensor, xyz2: torch.Tensor) -> torch.Tensor:
    """Earth mover's distance (approximate matching) per cloud.

    Args:
        xyz1: (B, N, 3) point cloud 1.
        xyz2: (B, M, 3) point cloud 2.

    Returns:
        (B,) the matching cost divided by N (0 for an empty xyz1), as the
        reference's emd() (emd/__init__.py:43-65).  Inputs are made
        contiguous here.
    """
    xyz1 = xyz1.contiguous()
    xyz2 = xyz2.contiguous()
    cost, _ = torch.ops.torch_point_ops_emd.emd_forward(xyz1, xyz2)
    if xyz1.size(1) == 0:
        return torch.zeros_like(cost)
    return cost / xyz1.size(1)


emd = earth_movers_distance

from .emd import EarthMoverDistance  # noqa: E402

# Importing the submodule .emd rebinds the package attribute `emd` to it;
# keep the name bound to the function.
emd = earth_movers_distance
