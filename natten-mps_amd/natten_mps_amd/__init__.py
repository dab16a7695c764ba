"""Neighbourhood attention for AMD Instinct MI355X (gfx950), drop-in for the
public surface of ``natten_mps``.

``import natten_mps_amd`` does not import torch; the first access to a public
attribute loads the torch-dependent modules (PEP 562), registering the
``natten_mps_amd::*`` torch.library ops on the way (as the reference's
``__init__.py:62-73`` does).
"""
from __future__ import annotations

from natten_mps_amd.version import __version__

__all__ = [
    "na1d",
    "na1d_varlen",
    "na2d",
    "na2d_varlen",
    "na3d",
    "na3d_varlen",
    "na1d_qk",
    "na1d_av",
    "na2d_qk",
    "na2d_av",
    "na3d_qk",
    "na3d_av",
    "merge_attentions",
    "NeighborhoodAttention1D",
    "NeighborhoodAttention2D",
    "NeighborhoodAttention3D",
    "has_hip",
    "get_backend",
    "set_backend",
    "register_backend",
    "get_support_matrix",
    "__version__",
]

_LAZY_ATTRS = {
    **{n: "natten_mps_amd.functional" for n in (
        "na1d", "na1d_varlen", "na1d_qk", "na1d_av", "na2d", "na2d_varlen", "na2d_qk", "na2d_av",
        "na3d", "na3d_varlen", "na3d_qk", "na3d_av")},
    "merge_attentions": "natten_mps_amd.merge",
    "NeighborhoodAttention1D": "natten_mps_amd.nn",
    "NeighborhoodAttention2D": "natten_mps_amd.nn",
    "NeighborhoodAttention3D": "natten_mps_amd.nn",
    "get_support_matrix": "natten_mps_amd.support_matrix",
}


def __getattr__(name: str):
    target = _LAZY_ATTRS.get(name)
    if target is None:
        raise AttributeError(f"module {__name__!r} has no attribute {name!r}")
    import importlib

    importlib.import_module("natten_mps_amd._torch_ops")
    return getattr(importlib.import_module(target), name)


def __dir__():
    return sorted(__all__)


def has_hip() -> bool:
    """True when a ROCm GPU and the built libnatten_hip.so are usable."""
    from natten_mps_amd._core import hip as _hip

    return bool(_hip.is_available())


def get_backend() -> str:
    from natten_mps_amd._core import ops

    return ops.get_backend()


def set_backend(name: str) -> None:
    from natten_mps_amd._core import ops

    ops.set_backend(name)


def register_backend(name: str, module) -> None:
    from natten_mps_amd._core import ops

    ops.register_backend(name, module)
