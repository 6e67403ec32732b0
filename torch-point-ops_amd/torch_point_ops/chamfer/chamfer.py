"""ChamferDistance module (reference: torch_point_ops/chamfer/chamfer.py:5-26)."""
import torch

from . import chamfer_distance, chamfer_loss

_REDUCTIONS = ("mean", "sum", None, "none")


class ChamferDistance(torch.nn.Module):
    """Chamfer distance between two point clouds with an optional reduction.

    reduction: "mean" -> mean(dist1) + mean(dist2); "sum" -> sum(dist1) + sum(dist2);
    None / "none" -> the tuple (dist1, dist2).  The two reductions run inside
    the Chamfer kernels (chamfer_loss) instead of as separate torch reductions.
    """

    def __init__(self, reduction="mean"):
        super().__init__()
        if reduction not in _REDUCTIONS:
            raise ValueError(
                f"reduction must be one of ['mean', 'sum', None, 'none'], but got {reduction}"
            )
        self.reduction = reduction

    def forward(self, xyz1, xyz2):
        if self.reduction in ("mean", "sum"):
            return chamfer_loss(xyz1, xyz2, self.reduction == "mean")
        return chamfer_distance(xyz1, xyz2)
