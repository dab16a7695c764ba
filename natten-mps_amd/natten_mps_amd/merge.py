"""Merging attention outputs that share queries (``merge.py`` of
/root/reference/src/natten_mps).

Given outputs O_i and their log-sum-exps L_i over disjoint key sets, the
result over the union is ``O = sum_i w_i O_i`` with ``w_i = exp(L_i - L)``
and ``L = log sum_i exp(L_i)``.  For two parts this is the sigmoid form used
by ring attention: ``O = O_0 - sigmoid(L_1 - L_0) (O_0 - O_1)``,
``L = L_0 - logsigmoid(L_0 - L_1)``, folded left for more parts.  Arithmetic
is fp32; the output keeps the dtype of ``outputs[0]``.
"""
from __future__ import annotations

from typing import List, Tuple

import torch
from torch import Tensor
from torch.nn import functional as F


def _merge_attentions_fn(outputs: List[Tensor], lse_tensors: List[Tensor]) -> Tuple[Tensor, Tensor]:
    """Forward-only N-way merge (``merge.py:21-49``)."""
    assert len(outputs) >= 2 and len(outputs) == len(lse_tensors)
    dt = outputs[0].dtype
    ls = [l.to(torch.float32).unsqueeze(-1) for l in lse_tensors]
    os_ = [o.to(torch.float32) for o in outputs]
    acc = os_[0] - torch.sigmoid(ls[1] - ls[0]) * (os_[0] - os_[1])
    lse = ls[0] - F.logsigmoid(ls[0] - ls[1])
    for o, l in zip(os_[2:], ls[2:]):
        acc = acc - torch.sigmoid(l - lse) * (acc - o)
        lse = lse - F.logsigmoid(lse - l)
    return acc.to(dt), lse.squeeze(-1)


class _MergeAttentionsAutogradFn(torch.autograd.Function):
    """Two-way merge with the analytic backward (``merge.py:52-102``).

    With ``s = sigmoid(L_1 - L_0)``: ``O = (1-s) O_0 + s O_1`` and
    ``L = L_0 + softplus(L_1 - L_0)``; so ``dO_0 = (1-s) g``, ``dO_1 = s g``,
    and with ``c = <g, O_1 - O_0>``: ``dL_0 = (1-s) gL - c s(1-s)``,
    ``dL_1 = s gL + c s(1-s)``.
    """

    @staticmethod
    def forward(ctx, out_0, out_1, lse_0, lse_1):
        o0, o1 = out_0.to(torch.float32), out_1.to(torch.float32)
        l0, l1 = lse_0.to(torch.float32).unsqueeze(-1), lse_1.to(torch.float32).unsqueeze(-1)
        s = torch.sigmoid(l1 - l0)
        merged = (1 - s) * o0 + s * o1
        lse = l0 + F.softplus(l1 - l0)
        ctx.save_for_backward(o0, o1, s)
        return merged.to(out_0.dtype), lse.squeeze(-1)

    @staticmethod
    def backward(ctx, grad_out, grad_lse):
        o0, o1, s = ctx.saved_tensors
        g = grad_out.to(torch.float32)
        gl = grad_lse.to(torch.float32).unsqueeze(-1)
        c = (g * (o1 - o0)).sum(dim=-1, keepdim=True)
        ds = s * (1 - s)
        d_l0 = (1 - s) * gl - c * ds
        d_l1 = s * gl + c * ds
        return ((1 - s) * g).to(grad_out.dtype), (s * g).to(grad_out.dtype), d_l0.squeeze(-1), d_l1.squeeze(-1)


def merge_attentions(outputs: List[Tensor], lse_tensors: List[Tensor],
                     use_autograd_fix: bool = True) -> Tuple[Tensor, Tensor]:
    """Merge attention outputs ``[B, *spatial, H, D]`` with their LSEs
    ``[B, *spatial, H]`` as if their key/value sets had been concatenated."""
    if len(outputs) < 2:
        raise ValueError("merge_attentions expects at least two outputs.")
    if len(outputs) != len(lse_tensors):
        raise ValueError("Number of outputs and LSE tensors must match.")
    ref = outputs[0].shape
    for i, (o, l) in enumerate(zip(outputs, lse_tensors)):
        if o.shape != ref:
            raise ValueError(f"Output {i} shape {o.shape} does not match output 0 shape {ref}.")
        if l.shape != ref[:-1]:
            raise ValueError(f"LSE {i} shape {l.shape} does not match expected {ref[:-1]}.")
    if use_autograd_fix and outputs[0].requires_grad and len(outputs) == 2:
        return _MergeAttentionsAutogradFn.apply(outputs[0], outputs[1], lse_tensors[0], lse_tensors[1])
    if use_autograd_fix and outputs[0].requires_grad and len(outputs) > 2:
        raise NotImplementedError(
            "merge_attentions backward only supports 2-way merge. "
            "Set use_autograd_fix=False for N-way forward-only merge."
        )
    return _merge_attentions_fn([o.contiguous() for o in outputs], [l.contiguous() for l in lse_tensors])


__all__ = ["merge_attentions"]
