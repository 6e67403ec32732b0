"""EarthMoverDistance module (reference: torch_point_ops/emd/emd.py:1-19)."""
import torch

from . import earth_movers_distance


class EarthMoverDistance(torch.nn.Module):
    """Mean over the batch of the earth mover's distance of two point clouds."""

    def forward(self, xyz1, xyz2):
        # xyz1 is (B, N, 3) and xyz2 is (B, M, 3), of one floating dtype on
        # one device; the per-cloud distances are averaged to a 0-d tensor
        return earth_movers_distance(xyz1, xyz2).mean()
