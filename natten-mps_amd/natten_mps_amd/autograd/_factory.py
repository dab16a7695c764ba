"""Autograd Functions for neighbourhood attention, generated per rank.

Same classes and call signatures as ``autograd/_factory.py`` of
/root/reference/src/natten_mps, but backend-neutral: the forward-with-LSE and
fused-backward hooks are looked up on the backend that was active at forward
time (the reference hard-codes its Metal module, ``_factory.py:37-38,66-67``).

Backward chain of the fused Function (``_factory.py:55-102``):
1. the backend's fused backward, when the forward produced an LSE;
2. the split path: recompute logits, softmax, AV backward, softmax gradient
   ``dS = P (dA - sum P dA) * scale``, QK backward;
3. re-differentiation of the backend's own forward (works for backends built
   from differentiable torch ops); otherwise an error.

GQA: K/V may carry fewer heads than Q when the backend handles it natively;
the split fallback expands them and sums the gradients over each group.
"""
from __future__ import annotations

import torch

from natten_mps_amd._core import ops


def _kv_repeat(q, k):
    return q.shape[-2] // k.shape[-2]


def _expand(t, n):
    return t if n == 1 else t.repeat_interleave(n, dim=-2)


def _fold(g, n):
    """Sum a gradient of repeat_interleave(n, dim=-2) back to the kv heads."""
    if g is None or n == 1:
        return g
    shp = g.shape
    return g.reshape(*shp[:-2], shp[-2] // n, n, shp[-1]).sum(dim=-2)


def _split_backward(rank, mod, grad_output, q, k, v, ks, st, dil, causal, scale_value):
    qk_fwd = getattr(mod, f"na{rank}d_qk_forward")
    av_bwd = getattr(mod, f"na{rank}d_av_backward", None)
    qk_bwd = getattr(mod, f"na{rank}d_qk_backward", None)
    if av_bwd is None or qk_bwd is None:
        return None
    n = _kv_repeat(q, k)
    ke, ve = _expand(k, n), _expand(v, n)
    logits = qk_fwd(q, ke, ks, dil, st, causal, None)
    attn = torch.softmax(logits * scale_value, dim=-1)
    av = av_bwd(grad_output, attn, ve, ks, dil, st, causal)
    if av is None:
        return None
    d_attn, dv = av
    d_logits = attn * (d_attn - (attn * d_attn).sum(-1, keepdim=True))
    d_logits = d_logits * scale_value
    qk = qk_bwd(d_logits, q, ke, ks, dil, st, causal)
    if qk is None:
        return None
    return qk[0], _fold(qk[1], n), _fold(dv, n)


def _redifferentiate(fn, inputs, needs, grads_out):
    with torch.enable_grad():
        leaves = [t.detach().requires_grad_(bool(r)) if t is not None else None for t, r in zip(inputs, needs)]
        out = fn(*leaves)
        wrt = [t for t in leaves if t is not None and t.requires_grad]
        if not out.requires_grad:
            raise RuntimeError(
                "natten_mps_amd: the active backend provides no backward for this op and its forward is "
                "not differentiable by torch."
            )
        got = torch.autograd.grad(out, wrt, grads_out, allow_unused=True)
    it = iter(got)
    return [next(it) if (t is not None and t.requires_grad) else None for t in leaves]


def create_na_autograd_fn(rank: int) -> type:
    """Fused NA Function: ``apply(q, k, v, kernel_size, stride, dilation,
    is_causal, scale) -> out``."""

    class _Fn(torch.autograd.Function):
        @staticmethod
        def forward(ctx, q, k, v, kernel_size, stride, dilation, is_causal, scale):
            mod = ops.active_module()
            ctx.mod = mod
            ctx.kernel_size, ctx.stride, ctx.dilation = kernel_size, stride, dilation
            ctx.is_causal, ctx.scale = is_causal, scale
            hook = getattr(mod, f"na{rank}d_forward_with_lse", None)
            if hook is not None:
                out, lse = hook(q, k, v, kernel_size, stride, dilation, is_causal, scale)
                if lse is not None:
                    ctx.save_for_backward(q, k, v, lse, out)
                    ctx.has_lse = True
                    return out
            ctx.has_lse = False
            out = getattr(mod, f"na{rank}d_forward")(q, k, v, kernel_size, stride, dilation, is_causal, scale)
            ctx.save_for_backward(q, k, v)
            return out

        @staticmethod
        def backward(ctx, grad_output):
            mod = ctx.mod
            saved = ctx.saved_tensors
            q = saved[0]
            scale_value = float(q.shape[-1] ** -0.5 if ctx.scale is None else ctx.scale)
            tail = (None,) * 5
            if ctx.has_lse:
                q, k, v, lse, out = saved
                fused = getattr(mod, f"na{rank}d_fused_backward", None)
                if fused is not None:
                    dq, dk, dv = fused(grad_output, q, k, v, out, lse, ctx.kernel_size, ctx.dilation,
                                       ctx.stride, ctx.is_causal, scale_value)
                    return (dq, dk, dv) + tail
            else:
                q, k, v = saved
            res = _split_backward(rank, mod, grad_output, q, k, v, ctx.kernel_size, ctx.stride, ctx.dilation,
                                  ctx.is_causal, scale_value)
            if res is not None:
                return tuple(res) + tail
            fwd = getattr(mod, f"na{rank}d_forward")
            g = _redifferentiate(
                lambda a, b, c: fwd(a, b, c, ctx.kernel_size, ctx.stride, ctx.dilation, ctx.is_causal, ctx.scale),
                (q, k, v), ctx.needs_input_grad[:3], grad_output)
            return tuple(g) + tail

    _Fn.__name__ = _Fn.__qualname__ = f"NeighborhoodAttention{rank}DFunction"
    _Fn.__doc__ = f"Fused {rank}D neighborhood attention with autograd support."
    return _Fn


def create_na_lse_autograd_fn(rank: int) -> type:
    """Fused NA returning ``(out, lse)`` with gradients through both outputs.
    Needs a backend with the forward-with-LSE and fused-backward hooks (the
    reference reaches the same result through split QK, logsumexp, softmax and
    AV, ``functional.py:285-290``)."""

    class _Fn(torch.autograd.Function):
        @staticmethod
        def forward(ctx, q, k, v, kernel_size, stride, dilation, is_causal, scale):
            mod = ops.active_module()
            ctx.mod = mod
            ctx.kernel_size, ctx.stride, ctx.dilation = kernel_size, stride, dilation
            ctx.is_causal, ctx.scale = is_causal, scale
            out, lse = getattr(mod, f"na{rank}d_forward_with_lse")(q, k, v, kernel_size, stride, dilation,
                                                                   is_causal, scale)
            ctx.save_for_backward(q, k, v, lse, out)
            return out, lse

        @staticmethod
        def backward(ctx, grad_output, grad_lse):
            q, k, v, lse, out = ctx.saved_tensors
            scale_value = float(q.shape[-1] ** -0.5 if ctx.scale is None else ctx.scale)
            if grad_output is None:
                grad_output = torch.zeros_like(out)
            dq, dk, dv = getattr(ctx.mod, f"na{rank}d_fused_backward")(
                grad_output, q, k, v, out, lse, ctx.kernel_size, ctx.dilation, ctx.stride, ctx.is_causal,
                scale_value, grad_lse)
            return dq, dk, dv, None, None, None, None, None

    _Fn.__name__ = _Fn.__qualname__ = f"NeighborhoodAttention{rank}DLSEFunction"
    _Fn.__doc__ = f"Fused {rank}D neighborhood attention returning (out, lse)."
    return _Fn


def create_na_global_autograd_fn(rank: int) -> type:
    """Fused NA over each query's window plus global keys (the reference's
    ``additional_keys`` / ``additional_values``, ``functional.py:285-299``,
    there a split pass, dense attention and a merge): ``apply(q, k, v, gk, gv,
    kernel_size, stride, dilation, is_causal, scale) -> (out, lse)`` with one
    softmax over both key sets; gradients flow to all five tensors, through
    both outputs.  Needs a backend with the ``na{r}d_forward_with_lse_global``
    and ``na{r}d_fused_backward_global`` hooks."""

    class _Fn(torch.autograd.Function):
        @staticmethod
        def forward(ctx, q, k, v, gk, gv, kernel_size, stride, dilation, is_causal, scale):
            mod = ops.active_module()
            ctx.mod = mod
            ctx.kernel_size, ctx.stride, ctx.dilation = kernel_size, stride, dilation
            ctx.is_causal, ctx.scale = is_causal, scale
            out, lse = getattr(mod, f"na{rank}d_forward_with_lse_global")(q, k, v, gk, gv, kernel_size, stride,
                                                                          dilation, is_causal, scale)
            ctx.save_for_backward(q, k, v, gk, gv, lse, out)
            return out, lse

        @staticmethod
        def backward(ctx, grad_output, grad_lse):
            q, k, v, gk, gv, lse, out = ctx.saved_tensors
            scale_value = float(q.shape[-1] ** -0.5 if ctx.scale is None else ctx.scale)
            if grad_output is None:
                grad_output = torch.zeros_like(out)
            grads = getattr(ctx.mod, f"na{rank}d_fused_backward_global")(
                grad_output, q, k, v, gk, gv, out, lse, ctx.kernel_size, ctx.dilation, ctx.stride, ctx.is_causal,
                scale_value, grad_lse)
            return (*grads, None, None, None, None, None)

    _Fn.__name__ = _Fn.__qualname__ = f"NeighborhoodAttention{rank}DGlobalFunction"
    _Fn.__doc__ = f"Fused {rank}D neighborhood attention plus global keys, returning (out, lse)."
    return _Fn


def create_na_qk_autograd_fn(rank: int) -> type:
    """``apply(q, k, kernel_size, dilation, stride, is_causal, scale) -> logits``."""

    class _Fn(torch.autograd.Function):
        @staticmethod
        def forward(ctx, q, k, kernel_size, dilation, stride, is_causal, scale):
            mod = ops.active_module()
            ctx.mod = mod
            ctx.kernel_size, ctx.dilation, ctx.stride = kernel_size, dilation, stride
            ctx.is_causal, ctx.scale = is_causal, scale
            ctx.save_for_backward(q, k)
            return getattr(mod, f"na{rank}d_qk_forward")(q, k, kernel_size, dilation, stride, is_causal, scale)

        @staticmethod
        def backward(ctx, grad_output):
            q, k = ctx.saved_tensors
            tail = (None,) * 5
            fn = getattr(ctx.mod, f"na{rank}d_qk_backward", None)
            if fn is not None:
                grad = grad_output
                res = (fn(grad, q, k, ctx.kernel_size, ctx.dilation, ctx.stride, ctx.is_causal, scale=ctx.scale)
                       if ctx.scale is not None else
                       fn(grad, q, k, ctx.kernel_size, ctx.dilation, ctx.stride, ctx.is_causal))
                if res is not None:
                    return res[0], res[1], *tail
            fwd = getattr(ctx.mod, f"na{rank}d_qk_forward")
            g = _redifferentiate(
                lambda a, b: fwd(a, b, ctx.kernel_size, ctx.dilation, ctx.stride, ctx.is_causal, ctx.scale),
                (q, k), ctx.needs_input_grad[:2], grad_output)
            return g[0], g[1], *tail

    _Fn.__name__ = _Fn.__qualname__ = f"NA{rank}DQKFunction"
    _Fn.__doc__ = f"Separate {rank}D QK operation with autograd. Returns attention logits."
    return _Fn


def create_na_av_autograd_fn(rank: int) -> type:
    """``apply(attn, v, kernel_size, dilation, stride, is_causal) -> out``."""

    class _Fn(torch.autograd.Function):
        @staticmethod
        def forward(ctx, attn, v, kernel_size, dilation, stride, is_causal):
            mod = ops.active_module()
            ctx.mod = mod
            ctx.kernel_size, ctx.dilation, ctx.stride, ctx.is_causal = kernel_size, dilation, stride, is_causal
            ctx.save_for_backward(attn, v)
            return getattr(mod, f"na{rank}d_av_forward")(attn, v, kernel_size, dilation, stride, is_causal)

        @staticmethod
        def backward(ctx, grad_output):
            attn, v = ctx.saved_tensors
            tail = (None,) * 4
            fn = getattr(ctx.mod, f"na{rank}d_av_backward", None)
            if fn is not None:
                res = fn(grad_output, attn, v, ctx.kernel_size, ctx.dilation, ctx.stride, ctx.is_causal)
                if res is not None:
                    return res[0], res[1], *tail
            fwd = getattr(ctx.mod, f"na{rank}d_av_forward")
            g = _redifferentiate(
                lambda a, b: fwd(a, b, ctx.kernel_size, ctx.dilation, ctx.stride, ctx.is_causal),
                (attn, v), ctx.needs_input_grad[:2], grad_output)
            return g[0], g[1], *tail

    _Fn.__name__ = _Fn.__qualname__ = f"NA{rank}DAVFunction"
    _Fn.__doc__ = f"Separate {rank}D AV operation with autograd. Returns output."
    return _Fn
