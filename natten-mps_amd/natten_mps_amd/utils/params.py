"""Argument normalisation and validation (``utils/params.py`` of
/root/reference/src/natten_mps, same rules and messages)."""
from __future__ import annotations

from typing import Sequence


def _as_tuple(param, rank: int, name: str):
    if isinstance(param, (int, bool)):
        vals = (param,) * rank
    elif isinstance(param, Sequence) and not isinstance(param, (str, bytes)):
        vals = tuple(param)
    else:
        raise ValueError(f"{name} must be an int, bool, or tuple/list of length {rank}.")
    if len(vals) != rank:
        raise ValueError(f"{name} must have length {rank}, got {len(vals)}.")
    return vals


def normalize_tuple_param(param, rank, name):
    """int/bool/sequence -> tuple of length ``rank``; all-bool stays bool,
    otherwise positive ints."""
    vals = _as_tuple(param, rank, name)
    if all(isinstance(v, bool) for v in vals):
        return tuple(bool(v) for v in vals)
    for v in vals:
        if isinstance(v, bool):
            raise ValueError(f"{name} cannot mix bool and int values.")
        if not isinstance(v, int):
            raise ValueError(f"{name} values must be int or bool.")
        if v <= 0:
            raise ValueError(f"{name} values must be > 0, got {v}.")
    return tuple(int(v) for v in vals)


def normalize_kernel_size(kernel_size, rank):
    vals = normalize_tuple_param(kernel_size, rank, "kernel_size")
    if any(isinstance(v, bool) for v in vals):
        raise ValueError("kernel_size must contain integers, not bools.")
    return vals


def check_kernel_size_vs_input(kernel_size, input_spatial_shape):
    if len(kernel_size) != len(input_spatial_shape):
        raise ValueError(
            f"kernel_size rank ({len(kernel_size)}) must match input rank ({len(input_spatial_shape)})."
        )
    for i, (k, n) in enumerate(zip(kernel_size, input_spatial_shape)):
        if k > n:
            raise ValueError(f"kernel_size[{i}]={k} cannot exceed input spatial size {n}.")


def check_stride_vs_kernel(stride, kernel_size):
    if len(stride) != len(kernel_size):
        raise ValueError(f"stride rank ({len(stride)}) must match kernel_size rank ({len(kernel_size)}).")
    for i, (s, k) in enumerate(zip(stride, kernel_size)):
        if s > k:
            raise ValueError(f"stride[{i}]={s} must be <= kernel_size[{i}]={k}.")


def check_dilation_kernel_vs_input(dilation, kernel_size, input_spatial_shape):
    if not (len(dilation) == len(kernel_size) == len(input_spatial_shape)):
        raise ValueError("dilation, kernel_size, and input_spatial_shape must share the same rank.")
    for i, (d, k, n) in enumerate(zip(dilation, kernel_size, input_spatial_shape)):
        if d * k > n:
            raise ValueError(
                f"dilation[{i}] * kernel_size[{i}] = {d * k} exceeds input spatial size {n}."
            )
