from .na1d import NeighborhoodAttention1D
from .na2d import NeighborhoodAttention2D
from .na3d import NeighborhoodAttention3D

__all__ = ["NeighborhoodAttention1D", "NeighborhoodAttention2D", "NeighborhoodAttention3D"]
