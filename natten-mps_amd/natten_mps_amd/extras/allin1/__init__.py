"""Fused QK + relative position bias and AV for DiNAT-style models
(``extras/allin1/__init__.py`` of /root/reference/src/natten_mps).

Layout: spatial-first ``[B, ..., H, D]``.  Example::

    from natten_mps_amd.extras.allin1 import na1d_qk_rpb, na1d_av_fused

    logits = na1d_qk_rpb(q, k, rpb, kernel_size=5, dilation=2, scale=0.288)
    attn = torch.softmax(logits, dim=-1)
    out = na1d_av_fused(attn, v, kernel_size=5, dilation=2)
"""
from __future__ import annotations

from typing import Optional

import torch

from natten_mps_amd.extras.allin1.functional import natten1dav, natten1dqkrpb, natten2dav, natten2dqkrpb


def na1d_qk_rpb(query: torch.Tensor, key: torch.Tensor, rpb: Optional[torch.Tensor], kernel_size: int,
                dilation: int = 1, *, scale: Optional[float] = None) -> torch.Tensor:
    """Fused 1-D QK + RPB (``__init__.py:32-56``): ``[B, L, H, D]`` ->
    ``[B, L, H, K]`` logits; ``scale`` multiplies the query first; a None rpb
    is a zero bias."""
    if query.ndim != 4:
        raise ValueError(f"query must be 4D [B, L, H, D], got shape {query.shape}")
    if scale is not None:
        query = query * scale
    if rpb is None:
        rpb = torch.zeros(query.shape[2], 2 * kernel_size - 1, device=query.device, dtype=query.dtype)
    return natten1dqkrpb(query, key, rpb, kernel_size, dilation)


def na1d_av_fused(attn: torch.Tensor, value: torch.Tensor, kernel_size: int, dilation: int = 1) -> torch.Tensor:
    """Fused 1-D AV (``__init__.py:59-73``)."""
    if attn.ndim != 4 or value.ndim != 4:
        raise ValueError("attn and value must be 4D for na1d_av_fused")
    return natten1dav(attn, value, kernel_size, dilation)


def na2d_qk_rpb(query: torch.Tensor, key: torch.Tensor, rpb: Optional[torch.Tensor], kernel_size: int,
                dilation: int = 1, *, scale: Optional[float] = None) -> torch.Tensor:
    """Fused 2-D QK + RPB (``__init__.py:76-100``): ``[B, Hh, Hw, H, D]`` ->
    ``[B, Hh, Hw, H, K*K]``."""
    if query.ndim != 5:
        raise ValueError(f"query must be 5D [B, Hh, Hw, H, D], got shape {query.shape}")
    if scale is not None:
        query = query * scale
    if rpb is None:
        rpb = torch.zeros(query.shape[3], 2 * kernel_size - 1, 2 * kernel_size - 1, device=query.device,
                          dtype=query.dtype)
    return natten2dqkrpb(query, key, rpb, kernel_size, dilation)


def na2d_av_fused(attn: torch.Tensor, value: torch.Tensor, kernel_size: int, dilation: int = 1) -> torch.Tensor:
    """Fused 2-D AV (``__init__.py:103-117``)."""
    if attn.ndim != 5 or value.ndim != 5:
        raise ValueError("attn and value must be 5D for na2d_av_fused")
    return natten2dav(attn, value, kernel_size, dilation)


__all__ = ["na1d_qk_rpb", "na1d_av_fused", "na2d_qk_rpb", "na2d_av_fused"]
