"""Placeholders for the reference's EMD API (torch_point_ops/emd/emd.py)."""
import torch

_MSG = ("earth mover's distance is not part of the MI355X build of torch_point_ops "
        "(only chamfer, knn, fps and gather_points are)")


def earth_movers_distance(xyz1, xyz2, *args, **kwargs):
    raise NotImplementedError(_MSG)


emd = earth_movers_distance


class EarthMoverDistance(torch.nn.Module):
    def __init__(self, *args, **kwargs):
        super().__init__()

    def forward(self, xyz1, xyz2):
        raise NotImplementedError(_MSG)
