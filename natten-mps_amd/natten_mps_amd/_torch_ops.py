"""torch.library custom ops for torch.compile (``_torch_ops.py`` of
/root/reference/src/natten_mps): ``natten_mps_amd::na{1,2,3}d_qk``,
``na{1,2,3}d_av`` and ``na{1,2,3}d_fwd`` with the reference's schemas, real
implementations for the CUDA dispatch key (ROCm tensors) and CPU (whichever
backend is active), Meta (fake) implementations with
``(S - 1) // stride + 1`` output extents, and autograd formulas.
"""
from __future__ import annotations

import torch

from natten_mps_amd._core import ops
from natten_mps_amd.autograd._factory import _split_backward

LIB = torch.library.Library("natten_mps_amd", "DEF")


def _strided(n: int, s: int) -> int:
    return (n - 1) // s + 1


def _define(rank: int) -> None:
    qk_name, av_name, fwd_name = f"na{rank}d_qk", f"na{rank}d_av", f"na{rank}d_fwd"
    LIB.define(f"{qk_name}(Tensor query, Tensor key, int[] kernel_size, int[] dilation, "
               "int[] stride, bool[] is_causal, float? scale) -> Tensor")
    LIB.define(f"{av_name}(Tensor attn, Tensor value, int[] kernel_size, int[] dilation, "
               "int[] stride, bool[] is_causal) -> Tensor")
    LIB.define(f"{fwd_name}(Tensor query, Tensor key, Tensor value, int[] kernel_size, "
               "int[] stride, int[] dilation, bool[] is_causal, float? scale) -> Tensor")

    qk_fwd = getattr(ops, f"na{rank}d_qk_forward")
    av_fwd = getattr(ops, f"na{rank}d_av_forward")
    na_fwd = getattr(ops, f"na{rank}d_forward")

    def qk_impl(query, key, kernel_size, dilation, stride, is_causal, scale):
        return qk_fwd(query, key, tuple(kernel_size), tuple(dilation), tuple(stride), tuple(is_causal), scale)

    def av_impl(attn, value, kernel_size, dilation, stride, is_causal):
        return av_fwd(attn, value, tuple(kernel_size), tuple(dilation), tuple(stride), tuple(is_causal))

    def fwd_impl(query, key, value, kernel_size, stride, dilation, is_causal, scale):
        sc = float(query.shape[-1] ** -0.5) if scale is None else scale
        return na_fwd(query, key, value, tuple(kernel_size), tuple(stride), tuple(dilation), tuple(is_causal), sc)

    def qk_meta(query, key, kernel_size, dilation, stride, is_causal, scale):
        B, *sp, H, _ = query.shape
        kv = 1
        for k in kernel_size:
            kv *= k
        return query.new_empty(B, *[_strided(n, s) for n, s in zip(sp, stride)], H, kv)

    def av_meta(attn, value, kernel_size, dilation, stride, is_causal):
        return value.new_empty(*attn.shape[:-1], value.shape[-1])

    def fwd_meta(query, key, value, kernel_size, stride, dilation, is_causal, scale):
        B, *sp, H, _ = query.shape
        return query.new_empty(B, *[_strided(n, s) for n, s in zip(sp, stride)], H, value.shape[-1])

    for key in ("CUDA", "CPU"):
        torch.library.impl(LIB, qk_name, key)(qk_impl)
        torch.library.impl(LIB, av_name, key)(av_impl)
        torch.library.impl(LIB, fwd_name, key)(fwd_impl)
    torch.library.impl(LIB, qk_name, "Meta")(qk_meta)
    torch.library.impl(LIB, av_name, "Meta")(av_meta)
    torch.library.impl(LIB, fwd_name, "Meta")(fwd_meta)

    # -- backward ops ---------------------------------------------------------
    # The gradients are ops of their own (with Meta kernels), so that a
    # compiled graph's backward traces them as opaque calls instead of
    # tracing into the library with fake tensors.
    LIB.define(f"{fwd_name}_backward(Tensor grad_out, Tensor query, Tensor key, Tensor value, int[] kernel_size, "
               "int[] stride, int[] dilation, bool[] is_causal, float? scale) -> (Tensor, Tensor, Tensor)")
    LIB.define(f"{qk_name}_backward(Tensor grad_attn, Tensor query, Tensor key, int[] kernel_size, int[] dilation, "
               "int[] stride, bool[] is_causal, float? scale) -> (Tensor, Tensor)")
    LIB.define(f"{av_name}_backward(Tensor grad_out, Tensor attn, Tensor value, int[] kernel_size, int[] dilation, "
               "int[] stride, bool[] is_causal) -> (Tensor, Tensor)")

    def _dense(grads, like):
        return tuple(torch.zeros_like(t) if g is None else g for g, t in zip(grads, like))

    def fwd_bwd_impl(grad_output, q, k, v, kernel_size, stride, dilation, is_causal, scale):
        ks, st, dil, causal = tuple(kernel_size), tuple(stride), tuple(dilation), tuple(is_causal)
        sc = float(q.shape[-1] ** -0.5 if scale is None else scale)
        mod = ops.active_module()
        with_lse = getattr(mod, f"na{rank}d_forward_with_lse", None)
        fused = getattr(mod, f"na{rank}d_fused_backward", None)
        if with_lse is not None and fused is not None:
            out, lse = with_lse(q, k, v, ks, st, dil, causal, sc)
            if lse is not None:
                return tuple(fused(grad_output, q, k, v, out, lse, ks, dil, st, causal, sc))
        res = _split_backward(rank, mod, grad_output, q, k, v, ks, st, dil, causal, sc)
        if res is None:
            with torch.enable_grad():
                leaves = [t.detach().requires_grad_(True) for t in (q, k, v)]
                out = getattr(mod, f"na{rank}d_forward")(*leaves, ks, st, dil, causal, sc)
                res = torch.autograd.grad(out, leaves, grad_output, allow_unused=True)
        return _dense(res[:3], (q, k, v))

    def qk_bwd_impl(grad_output, q, k, kernel_size, dilation, stride, is_causal, scale):
        ks, dil, st, causal = tuple(kernel_size), tuple(dilation), tuple(stride), tuple(is_causal)
        res = getattr(ops, f"na{rank}d_qk_backward")(grad_output, q, k, ks, dil, st, causal, scale=scale)
        if res is None:
            with torch.enable_grad():
                leaves = [t.detach().requires_grad_(True) for t in (q, k)]
                out = qk_fwd(*leaves, ks, dil, st, causal, scale)
                res = torch.autograd.grad(out, leaves, grad_output, allow_unused=True)
        return _dense(res[:2], (q, k))

    def av_bwd_impl(grad_output, attn, v, kernel_size, dilation, stride, is_causal):
        ks, dil, st, causal = tuple(kernel_size), tuple(dilation), tuple(stride), tuple(is_causal)
        res = getattr(ops, f"na{rank}d_av_backward")(grad_output, attn, v, ks, dil, st, causal)
        if res is None:
            with torch.enable_grad():
                leaves = [t.detach().requires_grad_(True) for t in (attn, v)]
                out = av_fwd(*leaves, ks, dil, st, causal)
                res = torch.autograd.grad(out, leaves, grad_output, allow_unused=True)
        return _dense(res[:2], (attn, v))

    for key in ("CUDA", "CPU"):
        torch.library.impl(LIB, f"{fwd_name}_backward", key)(fwd_bwd_impl)
        torch.library.impl(LIB, f"{qk_name}_backward", key)(qk_bwd_impl)
        torch.library.impl(LIB, f"{av_name}_backward", key)(av_bwd_impl)
    torch.library.impl(LIB, f"{fwd_name}_backward", "Meta")(
        lambda g, q, k, v, *a: (torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)))
    torch.library.impl(LIB, f"{qk_name}_backward", "Meta")(
        lambda g, q, k, *a: (torch.empty_like(q), torch.empty_like(k)))
    torch.library.impl(LIB, f"{av_name}_backward", "Meta")(
        lambda g, attn, v, *a: (torch.empty_like(attn), torch.empty_like(v)))

    # -- autograd -------------------------------------------------------------
    this = getattr(torch.ops, LIB.ns)

    def _setup_fwd(ctx, inputs, output):
        q, k, v, kernel_size, stride, dilation, is_causal, scale = inputs
        ctx.params = (list(kernel_size), list(stride), list(dilation), list(is_causal), scale)
        ctx.save_for_backward(q, k, v)

    def _fwd_backward(ctx, grad_output):
        q, k, v = ctx.saved_tensors
        dq, dk, dv = getattr(this, f"{fwd_name}_backward")(grad_output, q, k, v, *ctx.params)
        return dq, dk, dv, None, None, None, None, None

    def _setup_qk(ctx, inputs, output):
        q, k, kernel_size, dilation, stride, is_causal, scale = inputs
        ctx.params = (list(kernel_size), list(dilation), list(stride), list(is_causal), scale)
        ctx.save_for_backward(q, k)

    def _qk_backward(ctx, grad_output):
        q, k = ctx.saved_tensors
        dq, dk = getattr(this, f"{qk_name}_backward")(grad_output, q, k, *ctx.params)
        return dq, dk, None, None, None, None, None

    def _setup_av(ctx, inputs, output):
        attn, v, kernel_size, dilation, stride, is_causal = inputs
        ctx.params = (list(kernel_size), list(dilation), list(stride), list(is_causal))
        ctx.save_for_backward(attn, v)

    def _av_backward(ctx, grad_output):
        attn, v = ctx.saved_tensors
        dattn, dv = getattr(this, f"{av_name}_backward")(grad_output, attn, v, *ctx.params)
        return dattn, dv, None, None, None, None

    torch.library.register_autograd(f"natten_mps_amd::{fwd_name}", _fwd_backward, setup_context=_setup_fwd)
    torch.library.register_autograd(f"natten_mps_amd::{qk_name}", _qk_backward, setup_context=_setup_qk)
    torch.library.register_autograd(f"natten_mps_amd::{av_name}", _av_backward, setup_context=_setup_av)


for _rank in (1, 2, 3):
    _define(_rank)
del _rank

__all__ = ["LIB"]
