"""Functional neighbourhood-attention API (``functional.py:1-675`` of
/root/reference/src/natten_mps): ``na1d/na2d/na3d``, ``na{1,2,3}d_qk`` and
``na{1,2,3}d_av``, with the same arguments, validation, defaults and
composition:

* GQA/MQA: K/V may have fewer heads; query head h uses kv head
  ``h // (Hq/Hkv)`` (the reference's ``repeat_interleave``, ``:27-31``).
  Backends that declare ``NATIVE_GQA`` receive the un-expanded K/V.
* Full-window fast path: kernel >= every spatial dim, stride 1, non-causal ->
  ``F.scaled_dot_product_attention`` (``:148-206``).
* ``return_lse`` / ``additional_keys`` (``:285-299``): NA output and LSE, plus
  dense attention over the extra tokens, merged with ``merge_attentions``.
  Backends that declare ``GLOBAL_KEYS`` take the extra tokens as global keys
  inside their fused kernels (one softmax over each window and the extra
  tokens, the same result) where their ``na{r}d_global_supported`` says so.
  Backends that declare ``FUSED_LSE`` produce the NA output and LSE in one
  fused pass (differentiable through both); others use the reference's
  split QK -> logsumexp/softmax -> AV composition.
* A backend named ``'pure'`` (a differentiable torch backend) is called
  directly, bypassing the autograd Functions (``:301-302``).
"""
from __future__ import annotations

from typing import Optional, Tuple, Union

import torch
import torch.nn.functional as F

from natten_mps_amd._core import ops
from natten_mps_amd.autograd import na1d as _ag1, na2d as _ag2, na3d as _ag3
from natten_mps_amd.utils.params import (
    check_dilation_kernel_vs_input,
    check_kernel_size_vs_input,
    check_stride_vs_kernel,
    normalize_kernel_size,
    normalize_tuple_param,
)

_AG = {1: _ag1, 2: _ag2, 3: _ag3}
_LAYOUTS = {1: "[B, L, H, D]", 2: "[B, H, W, heads, dim]", 3: "[B, D, H, W, heads, dim]"}


def _normalize_is_causal(is_causal, rank: int) -> tuple:
    return tuple(bool(v) for v in normalize_tuple_param(is_causal, rank, "is_causal"))


def _repeat_kv(x: torch.Tensor, n_rep: int) -> torch.Tensor:
    """Expand KV heads to the query heads (GQA/MQA)."""
    return x if n_rep == 1 else x.repeat_interleave(n_rep, dim=-2)


def _validate_qkv(query, key, value, rank: int) -> int:
    """Shape checks with GQA; returns the kv repeat factor (``:34-71``)."""
    nd = rank + 3
    if query.ndim != nd or key.ndim != nd or value.ndim != nd:
        raise ValueError(f"na{rank}d expects query/key/value with shape {_LAYOUTS[rank]}.")
    sq, sk, sv = query.shape[1:-2], key.shape[1:-2], value.shape[1:-2]
    if sq != sk or sq != sv:
        raise ValueError(f"Spatial dimensions must match: Q={sq}, K={sk}, V={sv}.")
    if query.shape[0] != key.shape[0] or query.shape[0] != value.shape[0]:
        raise ValueError("Batch dimensions must match.")
    hq, dq = query.shape[-2], query.shape[-1]
    hkv, dk = key.shape[-2], key.shape[-1]
    if dq != dk:
        raise ValueError(f"Head dim must match between Q and K: Q has {dq}, K has {dk}.")
    if key.shape[-2] != value.shape[-2]:
        raise ValueError(f"K and V must have same number of heads: K={key.shape[-2]}, V={value.shape[-2]}.")
    if hq % hkv != 0:
        raise ValueError(f"heads_q ({hq}) must be divisible by heads_kv ({hkv}) for GQA.")
    return hq // hkv


def _validate_additional_kv(query, additional_keys, additional_values, kv_repeat):
    """Checks and GQA-expands the extra tokens (``:113-145``)."""
    if additional_keys is None and additional_values is None:
        return None, None
    if additional_keys is None or additional_values is None:
        raise ValueError("additional_keys and additional_values must both be provided or both None.")
    ak, av = additional_keys, additional_values
    if ak.ndim != 4 or av.ndim != 4:
        raise ValueError("additional_keys/additional_values must be 4D: [B, N_extra, heads_kv, dim].")
    if ak.shape[0] != query.shape[0]:
        raise ValueError("additional_keys batch must match query batch.")
    if av.shape[0] != query.shape[0]:
        raise ValueError("additional_values batch must match query batch.")
    if ak.shape[-1] != query.shape[-1]:
        raise ValueError("additional_keys head dim must match query head dim.")
    if av.shape[-1] != query.shape[-1]:
        raise ValueError("additional_values head dim must match query head dim.")
    if ak.shape[-2] != av.shape[-2]:
        raise ValueError("additional_keys and additional_values must have same number of heads.")
    if ak.shape[1] != av.shape[1]:
        raise ValueError("additional_keys and additional_values must have same N_extra.")
    return _repeat_kv(ak, kv_repeat), _repeat_kv(av, kv_repeat)


def _full_attn_with_lse(query, key, value, scale: float):
    """Dense attention of every query over ``key/value [B, N, H, D]`` with its
    LSE ``[B, *spatial, H]`` (``:74-110``)."""
    sp = query.shape[1:-2]
    B, H, D = query.shape[0], query.shape[-2], query.shape[-1]
    S = 1
    for s in sp:
        S *= s
    q_t = query.reshape(B, S, H, D).permute(0, 2, 1, 3)
    k_t = key.permute(0, 2, 3, 1).contiguous()          # [B, H, D, N]
    logits = torch.matmul(q_t, k_t) * scale              # [B, H, S, N]
    lse = torch.logsumexp(logits, dim=-1)
    attn = torch.softmax(logits, dim=-1)
    out = torch.matmul(attn, value.permute(0, 2, 1, 3).contiguous())
    out = out.permute(0, 2, 1, 3).reshape(B, *sp, H, value.shape[-1])
    lse = lse.permute(0, 2, 1).reshape(B, *sp, H)
    return out, lse


def _is_full_attention(kernel_size, spatial_shape) -> bool:
    return all(k >= s for k, s in zip(kernel_size, spatial_shape))


def _sdpa_forward(query, key, value, scale, spatial_shape, return_lse=False,
                  additional_keys=None, additional_values=None):
    """Kernel covering the whole input: plain attention (``:148-206``)."""
    B, H, D = query.shape[0], query.shape[-2], query.shape[-1]
    S = 1
    for s in spatial_shape:
        S *= s
    k_all = key.reshape(B, S, H, D)
    v_all = value.reshape(B, S, H, value.shape[-1])
    if additional_keys is not None:
        k_all = torch.cat([k_all, additional_keys], dim=1)
        v_all = torch.cat([v_all, additional_values], dim=1)
    q_t = query.reshape(B, -1, H, D).permute(0, 2, 1, 3)
    k_t = k_all.permute(0, 2, 1, 3)
    v_t = v_all.permute(0, 2, 1, 3)
    out = F.scaled_dot_product_attention(q_t, k_t, v_t, scale=scale)
    out = out.permute(0, 2, 1, 3).reshape(B, *spatial_shape, H, value.shape[-1])
    if return_lse:
        logits = torch.matmul(q_t, k_t.transpose(-2, -1).contiguous()) * scale
        lse = torch.logsumexp(logits, dim=-1).permute(0, 2, 1).reshape(B, *spatial_shape, H)
        return out, lse
    return out


def _using_pure_backend() -> bool:
    return ops.get_backend() == "pure"


# Validated, normalised parameters of recent calls, keyed on the tensor shapes
# and the raw parameters: a repeated call skips the checks (they depend on
# nothing else).  Parameters that are not hashable, or a scale that is not a
# plain number, are validated on every call; a failed check is never cached.
_SETUP_CACHE: dict = {}
_SETUP_CACHE_MAX = 256


def _na_setup(rank, query, key, value, kernel_size, stride, dilation, is_causal, scale, additional_keys,
              additional_values):
    """(kv_repeat, kernel, stride, dilation, causal, spatial, scale, full
    window, extra keys, extra values), checked in the reference's order."""
    ck = None
    plain = additional_keys is None and additional_values is None
    if plain and (scale is None or type(scale) in (float, int)):
        # element types keep bool kernel sizes (rejected) apart from ints
        ktypes = tuple(map(type, kernel_size)) if type(kernel_size) is tuple else type(kernel_size)
        ck = (rank, query.shape, key.shape, value.shape, kernel_size, ktypes, stride, dilation, is_causal, scale)
        try:
            hit = _SETUP_CACHE.get(ck)
        except TypeError:  # unhashable parameters (lists)
            ck, hit = None, None
        if hit is not None:
            return hit
    kv_repeat = _validate_qkv(query, key, value, rank)
    add_k, add_v = _validate_additional_kv(query, additional_keys, additional_values, kv_repeat)
    ks = normalize_kernel_size(kernel_size, rank)
    st = normalize_tuple_param(stride, rank, "stride")
    dil = normalize_tuple_param(dilation, rank, "dilation")
    causal = _normalize_is_causal(is_causal, rank)
    spatial = tuple(query.shape[1:1 + rank])
    check_kernel_size_vs_input(ks, spatial)
    check_stride_vs_kernel(st, ks)
    check_dilation_kernel_vs_input(dil, ks, spatial)
    scale_value = query.shape[-1] ** -0.5 if scale is None else float(scale)
    full = _is_full_attention(ks, spatial) and all(s == 1 for s in st) and not any(causal)
    res = (kv_repeat, ks, st, dil, causal, spatial, scale_value, full, add_k, add_v)
    if ck is not None:
        if len(_SETUP_CACHE) >= _SETUP_CACHE_MAX:
            _SETUP_CACHE.clear()
        _SETUP_CACHE[ck] = res
    return res


def _na(rank, query, key, value, kernel_size, stride, dilation, is_causal, scale, return_lse,
        additional_keys, additional_values):
    kv_repeat, ks, st, dil, causal, spatial, scale_value, full, add_k, add_v = _na_setup(
        rank, query, key, value, kernel_size, stride, dilation, is_causal, scale, additional_keys,
        additional_values)

    if full:
        return _sdpa_forward(query, _repeat_kv(key, kv_repeat), _repeat_kv(value, kv_repeat), scale_value,
                             spatial, return_lse=return_lse, additional_keys=add_k, additional_values=add_v)

    pure = _using_pure_backend()
    mod = ops.active_module()
    native_gqa = bool(getattr(mod, "NATIVE_GQA", False)) and not pure
    if native_gqa:
        k_in, v_in = key, value
    else:
        k_in, v_in = _repeat_kv(key, kv_repeat), _repeat_kv(value, kv_repeat)
    has_additional = add_k is not None
    ag = _AG[rank]

    if has_additional and not pure and getattr(mod, "GLOBAL_KEYS", False):
        # the extra tokens as global keys inside the fused kernels: one
        # softmax over each window and the extra tokens, which is what the
        # composition below computes (split NA + dense attention + merge)
        gk, gv = (additional_keys, additional_values) if native_gqa else (add_k, add_v)
        grads = torch.is_grad_enabled() and any(
            t.requires_grad for t in (query, key, value, additional_keys, additional_values))
        if (gk.dtype == query.dtype and gv.dtype == query.dtype
                and getattr(mod, f"na{rank}d_global_supported")(query, k_in, v_in, gk.shape[1], ks, st, dil, causal,
                                                               grads, gk, gv, scale_value)):
            fn = getattr(ag, f"NeighborhoodAttention{rank}DGlobalFunction")
            try:
                out, lse = fn.apply(query, k_in, v_in, gk, gv, ks, st, dil, causal, scale_value)
                return (out, lse) if return_lse else out
            except NotImplementedError:
                # the backend declined these operands after all (a limit its
                # probe does not see): the composition below computes the same
                pass

    if has_additional or return_lse:
        if getattr(mod, "FUSED_LSE", False) and not pure:
            fn = getattr(ag, f"NeighborhoodAttention{rank}DLSEFunction")
            out, lse = fn.apply(query, k_in, v_in, ks, st, dil, causal, scale_value)
            if not has_additional:
                lse = lse.to(query.dtype)
        else:
            qk = globals()[f"na{rank}d_qk"]
            av = globals()[f"na{rank}d_av"]
            logits = qk(query, k_in, kernel_size=ks, dilation=dil, stride=st, is_causal=causal)
            logits_scaled = logits * scale_value
            lse = torch.logsumexp(logits_scaled, dim=-1)
            attn = torch.softmax(logits_scaled, dim=-1)
            out = av(attn, v_in, kernel_size=ks, dilation=dil, stride=st, is_causal=causal)
        if has_additional:
            from natten_mps_amd.merge import merge_attentions
            out_extra, lse_extra = _full_attn_with_lse(query, add_k, add_v, scale_value)
            out, lse = merge_attentions([out, out_extra], [lse, lse_extra])
        if return_lse:
            return out, lse
        return out

    if pure:
        return getattr(ops, f"na{rank}d_forward")(query, k_in, v_in, ks, st, dil, causal, scale_value)
    fn = getattr(ag, f"NeighborhoodAttention{rank}DFunction")
    return fn.apply(query, k_in, v_in, ks, st, dil, causal, scale_value)


def na1d(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
         kernel_size: Union[int, Tuple[int]], stride: Union[int, Tuple[int]] = 1,
         dilation: Union[int, Tuple[int]] = 1, is_causal: Union[bool, Tuple[bool]] = False,
         scale: Optional[float] = None, return_lse: bool = False,
         additional_keys: Optional[torch.Tensor] = None, additional_values: Optional[torch.Tensor] = None):
    """1-D neighbourhood attention over ``[B, L, H, D]`` (``functional.py:213-303``).

    Returns ``[B, L_out, H_q, D]`` (``L_out = ceil(L/stride)``), or
    ``(out, lse)`` with ``lse`` ``[B, L_out, H_q]`` when ``return_lse``."""
    return _na(1, query, key, value, kernel_size, stride, dilation, is_causal, scale, return_lse,
               additional_keys, additional_values)


def na2d(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
         kernel_size: Union[int, Tuple[int, int]], stride: Union[int, Tuple[int, int]] = 1,
         dilation: Union[int, Tuple[int, int]] = 1, is_causal: Union[bool, Tuple[bool, bool]] = False,
         scale: Optional[float] = None, return_lse: bool = False,
         additional_keys: Optional[torch.Tensor] = None, additional_values: Optional[torch.Tensor] = None):
    """2-D neighbourhood attention over ``[B, H, W, heads, dim]`` (``functional.py:306-394``)."""
    return _na(2, query, key, value, kernel_size, stride, dilation, is_causal, scale, return_lse,
               additional_keys, additional_values)


def na3d(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
         kernel_size: Union[int, Tuple[int, int, int]], stride: Union[int, Tuple[int, int, int]] = 1,
         dilation: Union[int, Tuple[int, int, int]] = 1,
         is_causal: Union[bool, Tuple[bool, bool, bool]] = False,
         scale: Optional[float] = None, return_lse: bool = False,
         additional_keys: Optional[torch.Tensor] = None, additional_values: Optional[torch.Tensor] = None):
    """3-D neighbourhood attention over ``[B, D, H, W, heads, dim]`` (``functional.py:522-611``)."""
    return _na(3, query, key, value, kernel_size, stride, dilation, is_causal, scale, return_lse,
               additional_keys, additional_values)


# ---------------------------------------------------------------------------
# split ops (functional.py:397-519, 614-675)
# ---------------------------------------------------------------------------


def _qk(rank, query, key, kernel_size, dilation, stride, is_causal, scale):
    if query.ndim != rank + 3 or key.ndim != rank + 3:
        raise ValueError(f"na{rank}d_qk expects query/key with shape {_LAYOUTS[rank]}.")
    if query.shape != key.shape:
        raise ValueError(f"query and key must share the same shape in na{rank}d_qk.")
    ks = normalize_kernel_size(kernel_size, rank)
    dil = normalize_tuple_param(dilation, rank, "dilation")
    st = normalize_tuple_param(stride, rank, "stride")
    causal = _normalize_is_causal(is_causal, rank)
    spatial = tuple(query.shape[1:1 + rank])
    check_kernel_size_vs_input(ks, spatial)
    check_dilation_kernel_vs_input(dil, ks, spatial)
    if _using_pure_backend():
        return getattr(ops, f"na{rank}d_qk_forward")(query, key, ks, dil, st, causal, scale)
    return getattr(_AG[rank], f"NA{rank}DQKFunction").apply(query, key, ks, dil, st, causal, scale)


def _av(rank, attn, value, kernel_size, dilation, stride, is_causal):
    if attn.ndim != rank + 3:
        raise ValueError(f"na{rank}d_av expects attn with shape [B, *spatial, heads, K].")
    if value.ndim != rank + 3:
        raise ValueError(f"na{rank}d_av expects value with shape {_LAYOUTS[rank]}.")
    if attn.shape[0] != value.shape[0] or attn.shape[-2] != value.shape[-2]:
        raise ValueError(f"na{rank}d_av requires attn/value to match on batch and heads dimensions.")
    if any(a > v for a, v in zip(attn.shape[1:1 + rank], value.shape[1:1 + rank])):
        raise ValueError(f"na{rank}d_av attn spatial size cannot exceed value spatial size.")
    ks = normalize_kernel_size(kernel_size, rank)
    dil = normalize_tuple_param(dilation, rank, "dilation")
    st = normalize_tuple_param(stride, rank, "stride")
    causal = _normalize_is_causal(is_causal, rank)
    vol = 1
    for k in ks:
        vol *= k
    if attn.shape[-1] != vol:
        raise ValueError(f"na{rank}d_av attn last dim ({attn.shape[-1]}) must match kernel volume ({vol}).")
    spatial = tuple(value.shape[1:1 + rank])
    check_kernel_size_vs_input(ks, spatial)
    check_dilation_kernel_vs_input(dil, ks, spatial)
    if _using_pure_backend():
        return getattr(ops, f"na{rank}d_av_forward")(attn, value, ks, dil, st, causal)
    return getattr(_AG[rank], f"NA{rank}DAVFunction").apply(attn, value, ks, dil, st, causal)


def na1d_qk(query, key, kernel_size, dilation=1, *, stride=1, is_causal=False, scale=None):
    """Unscaled (unless ``scale``) logits ``[B, L_out, H, K]``; causal-invalid entries are -inf."""
    return _qk(1, query, key, kernel_size, dilation, stride, is_causal, scale)


def na2d_qk(query, key, kernel_size, dilation=1, *, stride=1, is_causal=False, scale=None):
    """Logits ``[B, H_out, W_out, heads, kh*kw]``."""
    return _qk(2, query, key, kernel_size, dilation, stride, is_causal, scale)


def na3d_qk(query, key, kernel_size, dilation=1, *, stride=1, is_causal=False, scale=None):
    """Logits ``[B, D_out, H_out, W_out, heads, kd*kh*kw]``."""
    return _qk(3, query, key, kernel_size, dilation, stride, is_causal, scale)


def na1d_av(attn, value, kernel_size, dilation=1, *, stride=1, is_causal=False):
    """``out = sum_k attn_k v_k`` over each neighbourhood."""
    return _av(1, attn, value, kernel_size, dilation, stride, is_causal)


def na2d_av(attn, value, kernel_size, dilation=1, *, stride=1, is_causal=False):
    return _av(2, attn, value, kernel_size, dilation, stride, is_causal)


def na3d_av(attn, value, kernel_size, dilation=1, *, stride=1, is_causal=False):
    return _av(3, attn, value, kernel_size, dilation, stride, is_causal)


# ---------------------------------------------------------------------------
# variable-length attention (functional.py:678-1026)
#
# Tensors are padded to a common extent; sample b attends within its own
# extent only (its windows follow the rule for that extent), and outputs and
# gradients at padding positions are zero.  The 'hip' backend runs all
# samples in one launch per op, each reading its extent from a device array;
# the backward is the fused varlen backward (no per-sample autograd loop).
# ---------------------------------------------------------------------------


def _validate_seq_lens(seq_lens: torch.Tensor, batch_size: int, l_max: int, kernel_size: int,
                       rows=None) -> None:
    """``functional.py:678-700``.  ``rows``: the lengths already on the host
    (``seq_lens.tolist()``), so that a device tensor is read back once."""
    if seq_lens.ndim != 1 or seq_lens.shape[0] != batch_size:
        raise ValueError(
            f"seq_lens must be a 1-D tensor of length B={batch_size}, got shape {tuple(seq_lens.shape)}.")
    if seq_lens.dtype not in (torch.int32, torch.int64):
        raise ValueError(f"seq_lens must be int32 or int64, got {seq_lens.dtype}.")
    if rows is None:
        rows = seq_lens.tolist()
    min_len = int(min(rows))
    max_len = int(max(rows))
    if min_len < kernel_size:
        raise ValueError(
            f"All seq_lens must be >= kernel_size ({kernel_size}), but min(seq_lens)={min_len}.")
    if max_len > l_max:
        raise ValueError(f"All seq_lens must be <= L_max ({l_max}), but max(seq_lens)={max_len}.")


def _validate_spatial_sizes(spatial_sizes: torch.Tensor, batch_size: int, max_spatial: tuple, kernel_size: tuple,
                            rank: int, rows=None) -> None:
    """``functional.py:757-787``.  ``rows``: the sizes already on the host
    (``spatial_sizes.tolist()``), so that a device tensor is read back once."""
    if spatial_sizes.ndim != 2 or spatial_sizes.shape[0] != batch_size or spatial_sizes.shape[1] != rank:
        raise ValueError(f"spatial_sizes must be a [B, {rank}] tensor, got shape {tuple(spatial_sizes.shape)}.")
    if spatial_sizes.dtype not in (torch.int32, torch.int64):
        raise ValueError(f"spatial_sizes must be int32 or int64, got {spatial_sizes.dtype}.")
    if rows is None:
        rows = spatial_sizes.tolist()
    for d in range(rank):
        min_dim = int(min(r[d] for r in rows))
        max_dim = int(max(r[d] for r in rows))
        if min_dim < kernel_size[d]:
            raise ValueError(
                f"All spatial_sizes[:,{d}] must be >= kernel_size[{d}] ({kernel_size[d]}), but min={min_dim}.")
        if max_dim > max_spatial[d]:
            raise ValueError(
                f"All spatial_sizes[:,{d}] must be <= max_spatial[{d}] ({max_spatial[d]}), but max={max_dim}.")


class _NAVarlenFunction(torch.autograd.Function):
    """Fused varlen forward with LSE and the fused varlen backward of the
    active backend (the reference's ``_NA{1,2,3}DVarlenFunction``,
    ``functional.py:703-754``, with the per-sample loop replaced)."""

    @staticmethod
    def forward(ctx, rank, mod, query, key, value, sizes, ks, dil, scale):
        out, lse = getattr(mod, f"na{rank}d_varlen_forward_with_lse")(query, key, value, sizes, ks, dil, scale)
        ctx.rank, ctx.mod, ctx.ks, ctx.dil, ctx.scale = rank, mod, ks, dil, scale
        ctx.save_for_backward(query, key, value, out, lse, sizes)
        return out

    @staticmethod
    def backward(ctx, grad_out):
        q, k, v, out, lse, sizes = ctx.saved_tensors
        dq, dk, dv = getattr(ctx.mod, f"na{ctx.rank}d_varlen_backward")(
            grad_out.contiguous(), q, k, v, out, lse, sizes, ctx.ks, ctx.dil, ctx.scale)
        return None, None, dq, dk, dv, None, None, None, None


def _varlen_per_sample(rank, query, key, value, sizes, ks, dil, scale_value):
    """Per-sample composition through the rank's na*d (``_core/pure.py:573-673``):
    used by backends without fused varlen ops, and for samples whose extent
    equals an even kernel on every axis (the reference's full-window path)."""
    na = {1: na1d, 2: na2d, 3: na3d}[rank]
    out = torch.zeros_like(query)
    for b in range(query.shape[0]):
        ext = [int(x) for x in sizes[b].reshape(-1).tolist()]
        idx = (slice(b, b + 1),) + tuple(slice(0, n) for n in ext)
        out[idx] = na(query[idx], key[idx], value[idx], kernel_size=ks, dilation=dil, scale=scale_value)
    return out


def _varlen(rank, query, key, value, sizes, kernel_size, dilation, scale):
    nd = rank + 3
    if query.ndim != nd or key.ndim != nd or value.ndim != nd:
        raise ValueError(f"na{rank}d_varlen expects query/key/value with shape {_LAYOUTS[rank]}.")
    if query.shape != key.shape or query.shape != value.shape:
        raise ValueError("query, key, and value must have identical shapes.")
    B = query.shape[0]
    ks = normalize_kernel_size(kernel_size, rank)
    dil = normalize_tuple_param(dilation, rank, "dilation")
    max_sp = tuple(query.shape[1:1 + rank])
    # the sizes are read back once (one device synchronisation when they
    # live on the device) and every host-side check works on that copy
    host = sizes.tolist() if sizes.ndim in (1, 2) and sizes.dtype in (torch.int32, torch.int64) else None
    if rank == 1:
        _validate_seq_lens(sizes, B, max_sp[0], ks[0], rows=host)
    else:
        _validate_spatial_sizes(sizes, B, max_sp, ks, rank, rows=host)
    sizes2 = sizes.reshape(B, rank)
    rows = [[int(x)] for x in host] if rank == 1 else [[int(x) for x in r] for r in host]
    # a sample's extent must hold the dilated kernel, as na*d on its slice requires
    for ext in {tuple(row) for row in rows}:
        check_dilation_kernel_vs_input(dil, ks, ext)
    scale_value = query.shape[-1] ** -0.5 if scale is None else float(scale)

    mod = ops.active_module()
    fused = not _using_pure_backend() and hasattr(mod, f"na{rank}d_varlen_forward_with_lse")
    if not fused:
        return _varlen_per_sample(rank, query, key, value, sizes2, ks, dil, scale_value)
    out = _NAVarlenFunction.apply(rank, mod, query, key, value, sizes2, ks, dil, scale_value)
    # samples with every extent equal to its (even) kernel take the full-window
    # path of na*d, whose windows the neighbourhood rule does not describe
    full = [b for b, row in enumerate(rows)
            if all(n == k for n, k in zip(row, ks)) and any(k % 2 == 0 for k in ks)]
    if full:
        out = out.clone()
        sel = torch.tensor(full, dtype=torch.long)
        out[sel] = _varlen_per_sample(rank, query[sel], key[sel], value[sel], sizes2[sel], ks, dil, scale_value)
    return out


def na1d_varlen(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, seq_lens: torch.Tensor,
                kernel_size: Union[int, Tuple[int]], dilation: Union[int, Tuple[int]] = 1,
                scale: Optional[float] = None) -> torch.Tensor:
    """Variable-length 1-D neighbourhood attention (``functional.py:897-933``):
    ``[B, L_max, H, D]`` tensors, ``seq_lens`` ``[B]`` int with
    ``kernel_size <= seq_lens[b] <= L_max``; positions past ``seq_lens[b]``
    are zero in the output."""
    return _varlen(1, query, key, value, seq_lens, kernel_size, dilation, scale)


def na2d_varlen(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, spatial_sizes: torch.Tensor,
                kernel_size: Union[int, Tuple[int, int]], dilation: Union[int, Tuple[int, int]] = 1,
                scale: Optional[float] = None) -> torch.Tensor:
    """Variable-length 2-D neighbourhood attention (``functional.py:936-975``):
    ``[B, H_max, W_max, heads, D]`` tensors and ``spatial_sizes`` ``[B, 2]``."""
    return _varlen(2, query, key, value, spatial_sizes, kernel_size, dilation, scale)


def na3d_varlen(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, spatial_sizes: torch.Tensor,
                kernel_size: Union[int, Tuple[int, int, int]], dilation: Union[int, Tuple[int, int, int]] = 1,
                scale: Optional[float] = None) -> torch.Tensor:
    """Variable-length 3-D neighbourhood attention (``functional.py:978-1019``):
    ``[B, D_max, H_max, W_max, heads, dim]`` tensors and ``spatial_sizes``
    ``[B, 3]``."""
    return _varlen(3, query, key, value, spatial_sizes, kernel_size, dilation, scale)
