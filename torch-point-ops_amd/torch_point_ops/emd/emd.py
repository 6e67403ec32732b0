"""EarthMoverDistance module (reference: torch_point_ops/emd/emd.py:1-19)."""
import torch

from . import earth_movers_distance


class EarthMoverDistance(torch.nn.Module):
    """Mean over the batch of the earth mover's distance of two point clouds."""

    def forward(self, xyz1, xyz2):
        """
        Args:
            xyz1 (torch.Tensor): (B, N, 3)
            xyz2 (torch.Tensor): (B, M, 3)
        Returns:
            torch.Tensor: () mean EMD distance
        """
        return earth_movers_distance(xyz1, xyz2).mean()
