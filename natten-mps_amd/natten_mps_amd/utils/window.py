"""Host-side window helpers (the same rule the device kernels use).

Mirrors ``utils/window.py:6-46,91-116`` of /root/reference/src/natten_mps:
the non-causal window of query i on an axis of length L, kernel K and
dilation d is centred on i, shifted inwards at the borders, and for d > 1
stays on the residue class of i.
"""
from __future__ import annotations

import torch


def get_window_start(index: int, length: int, kernel_size: int, dilation: int) -> int:
    half = kernel_size // 2
    if dilation <= 1:
        start = max(index - half, 0)
        if index + half >= length:
            start += length - index - half - 1
        return start
    if index - half * dilation < 0:
        return index % dilation
    if index + half * dilation >= length:
        res = index % dilation
        full = (length // dilation) * dilation
        tail = length - full
        if res < tail:
            return length - tail + res - 2 * half * dilation
        return full + res - kernel_size * dilation
    return index - half * dilation


def get_window_end(index: int, length: int, kernel_size: int, dilation: int) -> int:
    """Inclusive end of the window."""
    return get_window_start(index, length, kernel_size, dilation) + (kernel_size - 1) * dilation


def get_window_start_vectorized(indices: torch.Tensor, length: int, kernel_size: int, dilation: int) -> torch.Tensor:
    half = kernel_size // 2
    idx = indices.to(dtype=torch.long)
    if dilation <= 1:
        start = torch.clamp(idx - half, min=0)
        return start + (idx + half >= length).to(start.dtype) * (length - idx - half - 1)
    res = torch.remainder(idx, dilation)
    full = (length // dilation) * dilation
    tail = length - full
    right = torch.where(res < tail, length - tail + res - 2 * half * dilation, full + res - kernel_size * dilation)
    left = idx - half * dilation < 0
    out = torch.where(left, res, idx - half * dilation)
    return torch.where((~left) & (idx + half * dilation >= length), right, out)
