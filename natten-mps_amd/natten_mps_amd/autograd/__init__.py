from .na1d import NA1DAVFunction, NA1DQKFunction, NeighborhoodAttention1DFunction, NeighborhoodAttention1DLSEFunction
from .na2d import NA2DAVFunction, NA2DQKFunction, NeighborhoodAttention2DFunction, NeighborhoodAttention2DLSEFunction
from .na3d import NA3DAVFunction, NA3DQKFunction, NeighborhoodAttention3DFunction, NeighborhoodAttention3DLSEFunction

__all__ = [
    "NeighborhoodAttention1DFunction",
    "NeighborhoodAttention2DFunction",
    "NeighborhoodAttention3DFunction",
    "NeighborhoodAttention1DLSEFunction",
    "NeighborhoodAttention2DLSEFunction",
    "NeighborhoodAttention3DLSEFunction",
    "NA1DQKFunction",
    "NA1DAVFunction",
    "NA2DQKFunction",
    "NA2DAVFunction",
    "NA3DQKFunction",
    "NA3DAVFunction",
]
