"""Oracle: CPU restatement of the reference's extras/allin1 pure ops
(``extras/allin1/functional.py:47-325`` and ``reference_impl.py:9-41`` of
/root/reference/src/natten_mps).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).  Never imported by
the shipped package.

Same semantics as the reference: NATTEN 0.17 shifted windows per axis,
logits ``q . k + rpb[h, bias] + mask`` with the key gathered from a
zero-padded copy (so invalid neighbours read zeros and add nothing to the
q/k gradients, while the bias gradient collects every entry), and AV with
invalid weights replaced by zero.  Gradients come from torch autograd, as in
the reference's pure fallback.  Tensors here are spatial-first
``[B, *spatial, H, D]``; the reference permutes to heads-first and back,
which does not change values.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch


def window_start(index: int, length: int, kernel_size: int, neighborhood: int, dilation: int) -> int:
    """``reference_impl.py:9-22``: start in class coordinates, phase-aligned
    to the query's residue class mod the dilation."""
    phase = index % dilation
    cls_index = index // dilation
    cls_len = -(-length // dilation)
    padded = cls_len * dilation - length
    if phase >= dilation - padded:
        cls_len -= 1
    start = max(cls_index - neighborhood, 0)
    if cls_index + neighborhood >= cls_len:
        start += cls_len - cls_index - neighborhood - 1
    return start * dilation + phase


def window_end(start: int, length: int, kernel_size: int, dilation: int) -> int:
    """``reference_impl.py:25-27`` (half-open)."""
    return min(length, start + kernel_size * dilation)


def bias_start(index: int, length: int, kernel_size: int, neighborhood: int, dilation: int) -> int:
    """``reference_impl.py:30-41``."""
    nh = neighborhood
    if dilation <= 1:
        out = nh
        if index < nh:
            out += nh - index
        if index + nh >= length:
            out += length - index - 1 - nh
        return out
    if index - nh * dilation < 0:
        return kernel_size - 1 - index // dilation
    if index + nh * dilation >= length:
        return (length - index - 1) // dilation
    return nh


def axis_tables(length: int, kernel_size: int, dilation: int) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Per query and neighbour offset: key position ``[L, K]``, validity
    (``0 <= pos < end``) and bias index clamped to ``[0, 2K-2]``."""
    nh = kernel_size // 2
    pos = torch.empty(length, kernel_size, dtype=torch.long)
    valid = torch.empty(length, kernel_size, dtype=torch.bool)
    bias = torch.empty(length, kernel_size, dtype=torch.long)
    for i in range(length):
        s = window_start(i, length, kernel_size, nh, dilation)
        e = window_end(s, length, kernel_size, dilation)
        pb = bias_start(i, length, kernel_size, nh, dilation)
        for off in range(kernel_size):
            p = s + off * dilation
            pos[i, off] = p
            valid[i, off] = 0 <= p < e
            bias[i, off] = min(max(pb + off, 0), 2 * kernel_size - 2)
    return pos, valid, bias


def _gather_keys(x: torch.Tensor, pos: torch.Tensor, axis: int) -> torch.Tensor:
    """x gathered along spatial ``axis`` at ``pos`` ``[n, K]`` (appending a
    neighbour axis after it), zero where pos is outside the axis -- the
    reference's zero-padded key/value."""
    n_axis = x.shape[axis]
    inside = (pos >= 0) & (pos < n_axis)
    g = x.index_select(axis, pos.clamp(0, n_axis - 1).reshape(-1))
    g = g.reshape(*x.shape[:axis], *pos.shape, *x.shape[axis + 1:])
    shape = [1] * g.dim()
    shape[axis], shape[axis + 1] = pos.shape
    return g * inside.reshape(shape).to(g.dtype)


def qkrpb_1d(q: torch.Tensor, k: torch.Tensor, rpb: Optional[torch.Tensor], kernel_size: int,
             dilation: int) -> torch.Tensor:
    """``functional.py:47-100``: ``[B, L, H, D]`` -> logits ``[B, L, H, K]``."""
    L = q.shape[1]
    pos, valid, bias = axis_tables(L, kernel_size, dilation)
    kg = _gather_keys(k, pos, 1)                                  # [B, L, K, H, D]
    score = torch.einsum("blhd,blkhd->blhk", q, kg)
    if rpb is not None:
        score = score + rpb[:, bias].permute(1, 0, 2).unsqueeze(0)  # [1, L, H, K]
    mask = torch.zeros(L, kernel_size, dtype=q.dtype).masked_fill(~valid, float("-inf"))
    return score + mask.reshape(1, L, 1, kernel_size)


def av_1d(attn: torch.Tensor, v: torch.Tensor, kernel_size: int, dilation: int) -> torch.Tensor:
    """``functional.py:103-150``: ``[B, L, H, K]`` x ``[B, L, H, D]``."""
    L = v.shape[1]
    pos, valid, _ = axis_tables(L, kernel_size, dilation)
    vg = _gather_keys(v, pos, 1)                                  # [B, L, K, H, D]
    w = torch.where(valid.reshape(1, L, 1, kernel_size), attn, torch.zeros_like(attn))
    return torch.einsum("blhk,blkhd->blhd", w, vg)


def qkrpb_2d(q: torch.Tensor, k: torch.Tensor, rpb: Optional[torch.Tensor], kernel_size: int,
             dilation: int) -> torch.Tensor:
    """``functional.py:153-250``: ``[B, Hh, Hw, H, D]`` -> ``[B, Hh, Hw, H, K*K]``."""
    B, Hh, Hw, H, D = q.shape
    K = kernel_size
    pi, vi, bi = axis_tables(Hh, K, dilation)
    pj, vj, bj = axis_tables(Hw, K, dilation)
    kg = _gather_keys(_gather_keys(k, pi, 1), pj, 3)              # [B, Hh, K, Hw, K, H, D]
    score = torch.einsum("bxyhd,bxiyjhd->bxyhij", q, kg)
    if rpb is not None:
        rb = rpb[:, bi][:, :, :, bj]                              # [H, Hh, K, Hw, K]
        score = score + rb.permute(1, 3, 0, 2, 4).unsqueeze(0)
    valid = vi.reshape(Hh, 1, K, 1) & vj.reshape(1, Hw, 1, K)
    mask = torch.zeros(Hh, Hw, K, K, dtype=q.dtype).masked_fill(~valid, float("-inf"))
    score = score + mask.reshape(1, Hh, Hw, 1, K, K)
    return score.reshape(B, Hh, Hw, H, K * K)


def av_2d(attn: torch.Tensor, v: torch.Tensor, kernel_size: int, dilation: int) -> torch.Tensor:
    """``functional.py:253-325``."""
    B, Hh, Hw, H, D = v.shape
    K = kernel_size
    pi, vi, _ = axis_tables(Hh, K, dilation)
    pj, vj, _ = axis_tables(Hw, K, dilation)
    vg = _gather_keys(_gather_keys(v, pi, 1), pj, 3)              # [B, Hh, K, Hw, K, H, D]
    valid = (vi.reshape(Hh, 1, K, 1) & vj.reshape(1, Hw, 1, K)).reshape(1, Hh, Hw, 1, K * K)
    w = torch.where(valid, attn, torch.zeros_like(attn)).reshape(B, Hh, Hw, H, K, K)
    return torch.einsum("bxyhij,bxiyjhd->bxyhd", w, vg)


def na1d_qk_rpb(q, k, rpb, kernel_size, dilation=1, scale=None):
    """``__init__.py:32-56``."""
    if scale is not None:
        q = q * scale
    if rpb is None:
        rpb = torch.zeros(q.shape[2], 2 * kernel_size - 1, dtype=q.dtype)
    return qkrpb_1d(q, k, rpb, kernel_size, dilation)


def na2d_qk_rpb(q, k, rpb, kernel_size, dilation=1, scale=None):
    """``__init__.py:76-100``."""
    if scale is not None:
        q = q * scale
    if rpb is None:
        rpb = torch.zeros(q.shape[3], 2 * kernel_size - 1, 2 * kernel_size - 1, dtype=q.dtype)
    return qkrpb_2d(q, k, rpb, kernel_size, dilation)
