"""Earth mover's distance: outside the scope of this MI355X build.

The names exist so that `import torch_point_ops` and the reference's
top-level imports keep working; calling them raises NotImplementedError.
"""
from .emd import EarthMoverDistance, emd, earth_movers_distance  # noqa: F401
