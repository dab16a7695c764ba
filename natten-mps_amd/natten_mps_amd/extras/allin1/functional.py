"""QK + relative position bias and AV for DiNAT-style models
(``extras/allin1/functional.py`` of /root/reference/src/natten_mps), on the
'hip' backend's kernels (``natten_hip_rpb_*``).

The ops follow NATTEN 0.17's shifted windows (``reference_impl.py:9-41``):
logits are ``q . k + rpb[h, bias]`` (unscaled) with ``-inf`` at invalid
neighbours, and AV sums ``attn * v`` over valid neighbours.  Tensors stay
spatial-first ``[B, *spatial, heads, dim]``: the kernels read them through
their strides, so there are no heads-first copies.  Gradients (q, k, rpb;
attn, v) come from the backward kernels, not from autograd replay.
"""
from __future__ import annotations

from typing import Optional, Tuple, Union

import torch

from natten_mps_amd._core import hip


def _check_args_against_dim(length: int, kernel_size: int, dilation: int, axis_name: str) -> None:
    """``extras/allin1/functional.py:35-40``."""
    if kernel_size * dilation > length:
        raise ValueError(
            f"Invalid NATTEN args on {axis_name}: kernel_size * dilation must be <= axis length. "
            f"Got kernel_size={kernel_size}, dilation={dilation}, {axis_name}={length}."
        )


def _square(kernel_size, dilation) -> Tuple[int, int]:
    """Kernel and dilation of the 2-D ops: square and uniform only
    (``extras/allin1/functional.py:160-171``)."""
    ks = (kernel_size, kernel_size) if isinstance(kernel_size, int) else tuple(int(x) for x in kernel_size)
    dl = (dilation, dilation) if isinstance(dilation, int) else tuple(int(x) for x in dilation)
    if ks[0] != ks[1] or dl[0] != dl[1]:
        raise ValueError("Only square kernels and uniform dilation are supported for shifted semantics.")
    return int(ks[0]), int(dl[0])


class _QKRPBFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, rank, query, key, rpb, kernel_size, dilation):
        ctx.rank, ctx.ks, ctx.dil = rank, kernel_size, dilation
        ctx.has_rpb = rpb is not None
        ctx.save_for_backward(query, key)
        return hip.rpb_qk_forward(rank, query, key, rpb, kernel_size, dilation)

    @staticmethod
    def backward(ctx, grad):
        q, k = ctx.saved_tensors
        dq, dk, drpb = hip.rpb_qk_backward(ctx.rank, grad.contiguous(), q, k, ctx.has_rpb, ctx.ks, ctx.dil)
        return None, dq, dk, drpb, None, None


class _AVFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, rank, attn, value, kernel_size, dilation):
        ctx.rank, ctx.ks, ctx.dil = rank, kernel_size, dilation
        ctx.save_for_backward(attn, value)
        return hip.rpb_av_forward(rank, attn, value, kernel_size, dilation)

    @staticmethod
    def backward(ctx, grad):
        attn, v = ctx.saved_tensors
        d_attn, dv = hip.rpb_av_backward(ctx.rank, grad.contiguous(), attn, v, ctx.ks, ctx.dil)
        return None, d_attn.to(attn.dtype), dv, None, None


def natten1dqkrpb(query: torch.Tensor, key: torch.Tensor, rpb: Optional[torch.Tensor], kernel_size: int,
                  dilation: int) -> torch.Tensor:
    """1-D QK + RPB logits before softmax (``functional.py:488-503``).
    ``[B, L, H, D]`` -> ``[B, L, H, K]``; rpb ``[H, 2K-1]`` or None."""
    _check_args_against_dim(int(query.shape[1]), int(kernel_size), int(dilation), "length")
    return _QKRPBFunction.apply(1, query, key, rpb, (int(kernel_size),), (int(dilation),))


def natten1dav(attention_probs: torch.Tensor, value: torch.Tensor, kernel_size: int, dilation: int) -> torch.Tensor:
    """1-D AV (``functional.py:506-520``): ``[B, L, H, K]`` x ``[B, L, H, D]``."""
    _check_args_against_dim(int(value.shape[1]), int(kernel_size), int(dilation), "length")
    return _AVFunction.apply(1, attention_probs, value, (int(kernel_size),), (int(dilation),))


def natten2dqkrpb(query: torch.Tensor, key: torch.Tensor, rpb: Optional[torch.Tensor],
                  kernel_size: Union[int, Tuple[int, int]], dilation: Union[int, Tuple[int, int]]) -> torch.Tensor:
    """2-D QK + RPB logits (``functional.py:523-542``): ``[B, Hh, Hw, H, D]``
    -> ``[B, Hh, Hw, H, K*K]``; rpb ``[H, 2K-1, 2K-1]`` or None."""
    k = int(kernel_size[0] if isinstance(kernel_size, tuple) else kernel_size)
    d = int(dilation[0] if isinstance(dilation, tuple) else dilation)
    _check_args_against_dim(int(query.shape[1]), k, d, "height")
    _check_args_against_dim(int(query.shape[2]), k, d, "width")
    k, d = _square(kernel_size, dilation)
    return _QKRPBFunction.apply(2, query, key, rpb, (k, k), (d, d))


def natten2dav(attention_probs: torch.Tensor, value: torch.Tensor, kernel_size: Union[int, Tuple[int, int]],
               dilation: Union[int, Tuple[int, int]]) -> torch.Tensor:
    """2-D AV (``functional.py:545-563``)."""
    k = int(kernel_size[0] if isinstance(kernel_size, tuple) else kernel_size)
    d = int(dilation[0] if isinstance(dilation, tuple) else dilation)
    _check_args_against_dim(int(value.shape[1]), k, d, "height")
    _check_args_against_dim(int(value.shape[2]), k, d, "width")
    k, d = _square(kernel_size, dilation)
    return _AVFunction.apply(2, attention_probs, value, (k, k), (d, d))


__all__ = ["natten1dqkrpb", "natten1dav", "natten2dqkrpb", "natten2dav"]
