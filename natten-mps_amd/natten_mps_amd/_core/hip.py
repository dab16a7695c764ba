"""The ``'hip'`` backend: neighbourhood attention on MI355X (gfx950) through
libnatten_hip.so.

Module contract (same names and argument order as the reference backends,
``_core/ops.py:22-32`` and the hooks the autograd factory looks up,
``autograd/_factory.py:37-38,66-67`` of /root/reference/src/natten_mps):

* ``na{r}d_forward(q, k, v, kernel_size, stride, dilation, is_causal, scale)``
* ``na{r}d_forward_with_lse(...) -> (out, lse)`` -- lse is fp32 ``[B, *sp_out, Hq]``
* ``na{r}d_fused_backward(d_out, q, k, v, out, lse, kernel_size, dilation,
  stride, is_causal, scale, d_lse=None) -> (dq, dk, dv)``
* ``na{r}d_qk_forward(q, k, kernel_size, dilation, stride, is_causal, scale)``
* ``na{r}d_av_forward(attn, v, kernel_size, dilation, stride, is_causal)``
* ``na{r}d_qk_backward(d_attn, q, k, kernel_size, dilation, stride, is_causal,
  scale=None) -> (dq, dk)``
* ``na{r}d_av_backward(d_out, attn, v, kernel_size, dilation, stride,
  is_causal) -> (d_attn, dv)``
* ``na{r}d_varlen_forward(q, k, v, sizes, kernel_size, dilation, scale)``
  (``_core/metal.py:624-811``), plus ``na{r}d_varlen_forward_with_lse`` and
  ``na{r}d_varlen_backward(d_out, q, k, v, out, lse, sizes, kernel_size,
  dilation, scale) -> (dq, dk, dv)`` for the autograd Function

Tensors stay spatial-first ``[B, *sp, H, D]``; the kernels read them through
their strides (only a non-unit innermost stride forces a copy), in their own
dtype (no bf16 upcast copies).  K/V may carry fewer heads than Q (native GQA:
query head h uses kv head ``h // (Hq/Hkv)``).

There is no CPU path: CPU tensors or dtypes other than fp32/fp16/bf16 raise.
"""
from __future__ import annotations

import ctypes
from typing import Optional, Sequence, Tuple

import torch

from . import _lib

# Functional-layer capability flags.
NATIVE_GQA = True
FUSED_LSE = True
GLOBAL_KEYS = True  # additional_keys in the fused kernels (na{r}d_*_global hooks)


_AVAILABLE = False


def is_available() -> bool:
    global _AVAILABLE
    if _AVAILABLE:  # a positive answer cannot change within a process
        return True
    if not _lib.is_built():
        return False
    try:
        if not torch.cuda.is_available():
            return False
        _lib.load()
    except Exception:
        return False
    _AVAILABLE = True
    return True


# ---------------------------------------------------------------------------
# helpers
# ---------------------------------------------------------------------------


def _ceil_div(a: int, b: int) -> int:
    return (a + b - 1) // b


def _on_device(*ts: Optional[torch.Tensor]) -> None:
    dev = None
    for t in ts:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise RuntimeError(
                "natten_mps_amd 'hip' backend: tensors must live on a ROCm GPU "
                f"(got a tensor on {t.device}). Move them with .cuda()."
            )
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError("natten_mps_amd 'hip' backend: all tensors must be on the same GPU.")


def _inner(t: torch.Tensor) -> torch.Tensor:
    """The kernels need a unit stride on the innermost dim only."""
    return t if t.stride(-1) == 1 else t.contiguous()


def _same_dtype(*ts: Optional[torch.Tensor]) -> None:
    dts = {t.dtype for t in ts if t is not None}
    if len(dts) > 1:
        raise TypeError(f"natten_mps_amd 'hip' backend: mixed dtypes {sorted(map(str, dts))}.")


def _byref(x):
    return ctypes.byref(x)


def _fused_problem(rank, q, k, v, kernel_size, stride, dilation, is_causal, scale):
    sp = tuple(q.shape[1:1 + rank])
    return _lib.problem(
        batch=q.shape[0], heads_q=q.shape[-2], heads_kv=k.shape[-2], dim_qk=q.shape[-1], dim_v=v.shape[-1],
        dtype=_lib.dtype_code(q), length=sp, out_length=[_ceil_div(n, s) for n, s in zip(sp, stride)],
        kernel_size=kernel_size, dilation=dilation, stride=stride, is_causal=is_causal, scale=scale,
    )


def _check_qkv(rank, q, k, v):
    nd = rank + 3
    if q.ndim != nd or k.ndim != nd or v.ndim != nd:
        raise ValueError(f"na{rank}d expects query/key/value with {nd} dims [B, *spatial, heads, dim].")
    if q.shape[:1 + rank] != k.shape[:1 + rank] or k.shape[:-1] != v.shape[:-1]:
        raise ValueError("query/key/value batch and spatial dims must match, and key/value heads must match.")
    if q.shape[-1] != k.shape[-1]:
        raise ValueError("query and key head dims must match.")
    if q.shape[-2] % k.shape[-2] != 0:
        raise ValueError(f"heads_q ({q.shape[-2]}) must be divisible by heads_kv ({k.shape[-2]}).")


# ---------------------------------------------------------------------------
# fused forward / backward
#
# The per-call host work (validation, problem descriptor, stride layouts) is
# cached per call signature -- shapes, strides, dtype, device and parameters --
# so a repeated call costs two allocations and one C call.
# ---------------------------------------------------------------------------

_FWD_CACHE: dict = {}
_BWD_CACHE: dict = {}
_CACHE_MAX = 512


class _Sig:
    __slots__ = ("prob", "prob_ref", "refs", "out_shape", "lse_shape", "strided", "device", "fast")


def _fast_call(sig, lays, out_shape, lse_shape, strided):
    """The signature's call object in the C++ host binding (None without it):
    the problem and layouts as raw bytes of their C structs."""
    b = _lib.binding()
    if b is None:
        return None
    blob = b"".join(bytes(x) if x is not None else bytes(_lib.Layout()) for x in lays)
    return b.FusedCall(bytes(sig.prob), blob, list(out_shape), list(lse_shape), bool(strided))


def _register_split(b, op, rank, given, used, outs, prob, kernel_size, dilation, stride, is_causal, scale,
                    zero_dq=False):
    """Register a split-op signature with the binding: ``given`` are the
    hook's input tensors, ``used`` what the C call received (registered only
    when they are the same tensors, i.e. nothing was converted), ``outs`` the
    outputs it allocated (contiguous, as the binding allocates them)."""
    if any(a is not u for a, u in zip(given, used)):
        return
    lays = [_lib.layout(t, rank, 1) for t in (*used, *outs)]
    blob = b"".join(bytes(x) for x in lays)
    out_shape = list(outs[0].shape) if op in (0, 1) else []
    call = b.SplitCall(op, bytes(prob), blob, out_shape, bool(zero_dq))
    b.split_register(rank, list(given), kernel_size, dilation, stride, is_causal, scale, call)


_RAW_STREAM = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _raw_stream(device):
    """hipStream_t of the current stream of `device` (an int)."""
    if _RAW_STREAM is not None:
        return _RAW_STREAM(device.index)
    return torch.cuda.current_stream(device).cuda_stream


def _launch(device, fn, *args):
    """Call a C entry point with the tensors' device current."""
    if torch.cuda.current_device() != device.index:
        with torch.cuda.device(device):
            return fn(*args)
    return fn(*args)


def _fwd_sig(rank, q, k, v, kernel_size, stride, dilation, is_causal, scale_value):
    _check_qkv(rank, q, k, v)
    _on_device(q, k, v)
    _same_dtype(q, k, v)
    sig = _Sig()
    sig.prob = _fused_problem(rank, q, k, v, kernel_size, stride, dilation, is_causal, scale_value)
    sig.prob_ref = ctypes.byref(sig.prob)
    out_sp = tuple(sig.prob.out_length[3 - rank:])
    B, Hq = q.shape[0], q.shape[-2]
    sig.out_shape = (B, *out_sp, Hq, v.shape[-1])
    sig.lse_shape = (B, *out_sp, Hq)
    sig.device = q.device
    out = torch.empty(sig.out_shape, dtype=q.dtype, device="meta")
    lse = torch.empty(sig.lse_shape, dtype=torch.float32, device="meta")
    lays = [_lib.layout(t, rank, 1) for t in (q, k, v, out)] + [_lib.layout(lse, rank, 0)]
    sig.refs = [lays, [ctypes.byref(x) for x in lays]]
    sig.fast = _fast_call(sig, lays, sig.out_shape, sig.lse_shape, False)
    return sig


def forward_with_lse(rank: int, q, k, v, kernel_size, stride, dilation, is_causal, scale):
    b = _lib.binding()
    if b is not None:
        # the binding's own signature cache: the whole call in C++ when this
        # signature was seen before (None otherwise, or when an argument
        # needs the handling below)
        r = b.fwd(rank, q, k, v, kernel_size, stride, dilation, is_causal, scale)
        if r is not None:
            return r
        q0, k0, v0 = q, k, v
    q, k, v = _inner(q), _inner(k), _inner(v)
    scale_value = float(q.shape[-1] ** -0.5 if scale is None else scale)
    key = (rank, q.dtype, k.dtype, v.dtype, q.device, k.device, v.device, q.shape, q.stride(), k.shape,
           k.stride(), v.shape, v.stride(), tuple(kernel_size), tuple(stride), tuple(dilation), tuple(is_causal),
           scale_value)
    sig = _FWD_CACHE.get(key)
    if sig is None:
        sig = _fwd_sig(rank, q, k, v, kernel_size, stride, dilation, is_causal, scale_value)
        if len(_FWD_CACHE) >= _CACHE_MAX:
            _FWD_CACHE.clear()
        _FWD_CACHE[key] = sig
    if sig.fast is not None:
        if b is not None:
            b.fwd_register(rank, q0, k0, v0, kernel_size, stride, dilation, is_causal, scale, sig.fast)
        return sig.fast.forward(q, k, v, _raw_stream(q.device))
    out = torch.empty(sig.out_shape, dtype=q.dtype, device=q.device)
    lse = torch.empty(sig.lse_shape, dtype=torch.float32, device=q.device)
    r = sig.refs[1]
    lib = _lib.load()
    rc = _launch(q.device, lib.natten_hip_forward, sig.prob_ref,
                 q.data_ptr(), r[0], k.data_ptr(), r[1], v.data_ptr(), r[2], out.data_ptr(), r[3],
                 lse.data_ptr(), r[4], _raw_stream(q.device))
    _lib.check(rc, "forward")
    return out, lse


def _bwd_sig(rank, d_out, q, k, v, out, lse, d_lse, kernel_size, stride, dilation, is_causal, scale_value):
    _check_qkv(rank, q, k, v)
    _on_device(d_out, q, k, v, out, lse, d_lse)
    _same_dtype(d_out, q, k, v, out)
    if lse.dtype != torch.float32 or (d_lse is not None and d_lse.dtype != torch.float32):
        raise TypeError("lse and its gradient must be float32")
    sig = _Sig()
    sig.prob = _fused_problem(rank, q, k, v, kernel_size, stride, dilation, is_causal, scale_value)
    sig.prob_ref = ctypes.byref(sig.prob)
    sig.strided = any(s != 1 for s in stride)
    sig.device = q.device
    sig.lse_shape = tuple(lse.shape)
    meta = lambda t: torch.empty(t.shape, dtype=t.dtype, device="meta")  # noqa: E731
    lays = [_lib.layout(t, rank, 1) for t in (q, k, v, out, d_out)]
    lays += [_lib.layout(lse, rank, 0), _lib.layout(d_lse, rank, 0) if d_lse is not None else None]
    lays += [_lib.layout(meta(t), rank, 1) for t in (q, k, v)]
    lays += [_lib.layout(torch.empty(sig.lse_shape, device="meta"), rank, 0)]
    sig.refs = [lays, [ctypes.byref(x) if x is not None else None for x in lays]]
    sig.fast = _fast_call(sig, lays, (), sig.lse_shape, sig.strided)
    return sig


def fused_backward(rank: int, d_out, q, k, v, out, lse, kernel_size, dilation, stride, is_causal, scale,
                   d_lse=None):
    b = _lib.binding()
    if b is not None:
        r = b.bwd(rank, d_out, q, k, v, out, lse, kernel_size, dilation, stride, is_causal, scale, d_lse)
        if r is not None:
            return r
        given = (d_out, q, k, v, out, lse, d_lse)
    q, k, v, out, d_out = _inner(q), _inner(k), _inner(v), _inner(out), _inner(d_out)
    if lse.dtype != torch.float32 or not lse.is_contiguous():
        lse = lse.to(torch.float32).contiguous()
    if d_lse is not None and (d_lse.dtype != torch.float32 or not d_lse.is_contiguous()):
        d_lse = d_lse.to(torch.float32).contiguous()
    scale_value = float(q.shape[-1] ** -0.5 if scale is None else scale)
    key = (rank, q.dtype, k.dtype, v.dtype, out.dtype, d_out.dtype, q.device, k.device, v.device, out.device,
           d_out.device, lse.device, None if d_lse is None else d_lse.device, q.shape, q.stride(), k.shape,
           k.stride(), v.shape, v.stride(), out.shape, out.stride(), d_out.shape, d_out.stride(), lse.shape,
           None if d_lse is None else d_lse.shape, tuple(kernel_size), tuple(stride), tuple(dilation),
           tuple(is_causal), scale_value)
    sig = _BWD_CACHE.get(key)
    if sig is None:
        sig = _bwd_sig(rank, d_out, q, k, v, out, lse, d_lse, kernel_size, stride, dilation, is_causal,
                       scale_value)
        if len(_BWD_CACHE) >= _CACHE_MAX:
            _BWD_CACHE.clear()
        _BWD_CACHE[key] = sig
    if sig.fast is not None:
        if b is not None:
            g_out, g_q, g_k, g_v, g_o, g_lse, g_dlse = given
            b.bwd_register(rank, g_out, g_q, g_k, g_v, g_o, g_lse, kernel_size, dilation, stride, is_causal, scale,
                           g_dlse, sig.fast)
        return sig.fast.backward(q, k, v, out, d_out, lse, d_lse, _raw_stream(q.device))
    dq = (torch.zeros if sig.strided else torch.empty)(q.shape, dtype=q.dtype, device=q.device)
    dk = torch.empty(k.shape, dtype=k.dtype, device=k.device)
    dv = torch.empty(v.shape, dtype=v.dtype, device=v.device)
    delta = torch.empty(sig.lse_shape, dtype=torch.float32, device=q.device)
    r = sig.refs[1]
    lib = _lib.load()
    rc = _launch(q.device, lib.natten_hip_backward, sig.prob_ref,
                 q.data_ptr(), r[0], k.data_ptr(), r[1], v.data_ptr(), r[2], out.data_ptr(), r[3],
                 d_out.data_ptr(), r[4], lse.data_ptr(), r[5],
                 d_lse.data_ptr() if d_lse is not None else None, r[6],
                 dq.data_ptr(), r[7], dk.data_ptr(), r[8], dv.data_ptr(), r[9], delta.data_ptr(), r[10],
                 _raw_stream(q.device))
    _lib.check(rc, "backward")
    return dq, dk, dv


def forward(rank: int, q, k, v, kernel_size, stride, dilation, is_causal, scale):
    return forward_with_lse(rank, q, k, v, kernel_size, stride, dilation, is_causal, scale)[0]


# ---------------------------------------------------------------------------
# split QK / AV and their backward
# ---------------------------------------------------------------------------


def _split_problem(rank, ref, heads, dim_qk, dim_v, sp, out_sp, kernel_size, dilation, stride, is_causal, scale):
    return _lib.problem(
        batch=ref.shape[0], heads_q=heads, heads_kv=heads, dim_qk=dim_qk, dim_v=dim_v,
        dtype=_lib.dtype_code(ref), length=sp, out_length=out_sp, kernel_size=kernel_size,
        dilation=dilation, stride=stride, is_causal=is_causal, scale=scale,
    )


def _attn_extent(rank, attn, sp, stride):
    out_sp = tuple(attn.shape[1:1 + rank])
    for n_out, n, s in zip(out_sp, sp, stride):
        if s != 1 and n_out != _ceil_div(n, s):
            raise ValueError(f"attn spatial extent {out_sp} does not match ceil({tuple(sp)}/{tuple(stride)}).")
        if n_out > n:
            raise ValueError("attn spatial dimensions cannot exceed value spatial dimensions.")
    return out_sp


def qk_forward(rank: int, q, k, kernel_size, dilation, stride, is_causal, scale):
    b = _lib.binding()
    if b is not None:
        r = b.qk(rank, q, k, kernel_size, dilation, stride, is_causal, scale)
        if r is not None:
            return r
    given = (q, k)
    if q.ndim != rank + 3 or q.shape != k.shape:
        raise ValueError(f"na{rank}d_qk expects query/key of identical shape [B, *spatial, heads, dim].")
    _on_device(q, k)
    _same_dtype(q, k)
    q, k = _inner(q), _inner(k)
    sp = tuple(q.shape[1:1 + rank])
    out_sp = tuple(_ceil_div(n, s) for n, s in zip(sp, stride))
    kv = 1
    for x in kernel_size:
        kv *= x
    prob = _split_problem(rank, q, q.shape[-2], q.shape[-1], q.shape[-1], sp, out_sp, kernel_size, dilation,
                          stride, is_causal, scale)
    attn = torch.empty((q.shape[0], *out_sp, q.shape[-2], kv), dtype=q.dtype, device=q.device)
    lib = _lib.load()
    with torch.cuda.device(q.device):
        rc = lib.natten_hip_qk_forward(
            _byref(prob), _lib.ptr(q), _byref(_lib.layout(q, rank, 1)), _lib.ptr(k),
            _byref(_lib.layout(k, rank, 1)), _lib.ptr(attn), _byref(_lib.layout(attn, rank, 1)),
            _lib.stream_of(q))
    _lib.check(rc, "qk_forward")
    if b is not None:
        _register_split(b, 0, rank, given, (q, k), (attn,), prob, kernel_size, dilation, stride, is_causal, scale)
    return attn


def av_forward(rank: int, attn, v, kernel_size, dilation, stride, is_causal):
    b = _lib.binding()
    if b is not None:
        r = b.av(rank, attn, v, kernel_size, dilation, stride, is_causal)
        if r is not None:
            return r
    given = (attn, v)
    if attn.ndim != rank + 3 or v.ndim != rank + 3:
        raise ValueError(f"na{rank}d_av expects attn [B, *spatial, heads, KV] and value [B, *spatial, heads, dim].")
    if attn.shape[0] != v.shape[0] or attn.shape[-2] != v.shape[-2]:
        raise ValueError("Batch and head dimensions of attn/value must match.")
    _on_device(attn, v)
    _same_dtype(attn, v)
    attn, v = _inner(attn), _inner(v)
    sp = tuple(v.shape[1:1 + rank])
    out_sp = _attn_extent(rank, attn, sp, stride)
    prob = _split_problem(rank, v, v.shape[-2], v.shape[-1], v.shape[-1], sp, out_sp, kernel_size, dilation,
                          stride, is_causal, None)
    if attn.shape[-1] != prob.kernel[0] * prob.kernel[1] * prob.kernel[2]:
        raise ValueError("attn last dim must equal the kernel volume.")
    out = torch.empty((v.shape[0], *out_sp, v.shape[-2], v.shape[-1]), dtype=v.dtype, device=v.device)
    lib = _lib.load()
    with torch.cuda.device(v.device):
        rc = lib.natten_hip_av_forward(
            _byref(prob), _lib.ptr(attn), _byref(_lib.layout(attn, rank, 1)), _lib.ptr(v),
            _byref(_lib.layout(v, rank, 1)), _lib.ptr(out), _byref(_lib.layout(out, rank, 1)),
            _lib.stream_of(v))
    _lib.check(rc, "av_forward")
    if b is not None:
        _register_split(b, 1, rank, given, (attn, v), (out,), prob, kernel_size, dilation, stride, is_causal, None)
    return out


def qk_backward(rank: int, d_attn, q, k, kernel_size, dilation, stride, is_causal, scale=None):
    b = _lib.binding()
    if b is not None:
        r = b.qk_bwd(rank, d_attn, q, k, kernel_size, dilation, stride, is_causal, scale)
        if r is not None:
            return r
    given = (d_attn, q, k)
    _on_device(d_attn, q, k)
    d_attn = d_attn.to(q.dtype)
    d_attn, q, k = _inner(d_attn), _inner(q), _inner(k)
    sp = tuple(q.shape[1:1 + rank])
    out_sp = _attn_extent(rank, d_attn, sp, stride)
    prob = _split_problem(rank, q, q.shape[-2], q.shape[-1], q.shape[-1], sp, out_sp, kernel_size, dilation,
                          stride, is_causal, scale)
    strided = any(s != 1 for s in stride) or out_sp != sp
    dq = (torch.zeros if strided else torch.empty)(q.shape, dtype=q.dtype, device=q.device)
    dk = torch.empty(k.shape, dtype=k.dtype, device=k.device)
    lib = _lib.load()
    L = lambda t: _byref(_lib.layout(t, rank, 1))  # noqa: E731
    with torch.cuda.device(q.device):
        rc = lib.natten_hip_qk_backward(
            _byref(prob), _lib.ptr(d_attn), L(d_attn), _lib.ptr(q), L(q), _lib.ptr(k), L(k),
            _lib.ptr(dq), L(dq), _lib.ptr(dk), L(dk), _lib.stream_of(q))
    _lib.check(rc, "qk_backward")
    if b is not None:
        _register_split(b, 2, rank, given, (d_attn, q, k), (dq, dk), prob, kernel_size, dilation, stride,
                        is_causal, scale, zero_dq=strided)
    return dq, dk


def av_backward(rank: int, d_out, attn, v, kernel_size, dilation, stride, is_causal):
    b = _lib.binding()
    if b is not None:
        r = b.av_bwd(rank, d_out, attn, v, kernel_size, dilation, stride, is_causal)
        if r is not None:
            return r
    given = (d_out, attn, v)
    _on_device(d_out, attn, v)
    d_out = d_out.to(v.dtype)
    attn = attn.to(v.dtype)
    d_out, attn, v = _inner(d_out), _inner(attn), _inner(v)
    sp = tuple(v.shape[1:1 + rank])
    out_sp = _attn_extent(rank, attn, sp, stride)
    prob = _split_problem(rank, v, v.shape[-2], v.shape[-1], v.shape[-1], sp, out_sp, kernel_size, dilation,
                          stride, is_causal, None)
    d_attn = torch.empty(attn.shape, dtype=attn.dtype, device=attn.device)
    dv = torch.empty(v.shape, dtype=v.dtype, device=v.device)
    lib = _lib.load()
    L = lambda t: _byref(_lib.layout(t, rank, 1))  # noqa: E731
    with torch.cuda.device(v.device):
        rc = lib.natten_hip_av_backward(
            _byref(prob), _lib.ptr(d_out), L(d_out), _lib.ptr(attn), L(attn), _lib.ptr(v), L(v),
            _lib.ptr(d_attn), L(d_attn), _lib.ptr(dv), L(dv), _lib.stream_of(v))
    _lib.check(rc, "av_backward")
    if b is not None:
        _register_split(b, 3, rank, given, (d_out, attn, v), (d_attn, dv), prob, kernel_size, dilation, stride,
                        is_causal, None)
    return d_attn, dv


def neighborhood_map(rank: int, spatial: Sequence[int], kernel_size, dilation, stride, is_causal,
                     device=None) -> Tuple[torch.Tensor, torch.Tensor]:
    """The fused op's flattened neighbour map ``[*sp_out, KV]`` (int64) and
    validity (bool), computed by the device kernel."""
    device = torch.device("cuda") if device is None else torch.device(device)
    out_sp = [_ceil_div(n, s) for n, s in zip(spatial, stride)]
    kv = 1
    for x in kernel_size:
        kv *= x
    prob = _lib.problem(batch=1, heads_q=1, heads_kv=1, dim_qk=1, dim_v=1, dtype=_lib.F32, length=spatial,
                        out_length=out_sp, kernel_size=kernel_size, dilation=dilation, stride=stride,
                        is_causal=is_causal, scale=None)
    flat = torch.empty((*out_sp, kv), dtype=torch.int64, device=device)
    valid = torch.empty((*out_sp, kv), dtype=torch.uint8, device=device)
    lib = _lib.load()
    with torch.cuda.device(device):
        rc = lib.natten_hip_neighborhood_map(_byref(prob), _lib.ptr(flat), _lib.ptr(valid),
                                             ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream))
    _lib.check(rc, "neighborhood_map")
    return flat, valid.bool()


# ---------------------------------------------------------------------------
# variable-length fused forward / backward (_core/metal.py:624-811 and the
# per-sample backward loops of functional.py:721-754, 804-835, 860-893)
# ---------------------------------------------------------------------------


def _varlen_lens(rank: int, sizes: torch.Tensor, device) -> torch.Tensor:
    """Per-sample extents ``[B, rank]`` -> int32 ``[B, 3]`` on the device,
    padded (leading) axes set to 1."""
    s = sizes.reshape(sizes.shape[0], rank).to(device=device, dtype=torch.int32)
    if rank < 3:
        s = torch.cat([torch.ones((s.shape[0], 3 - rank), dtype=torch.int32, device=device), s], dim=1)
    return s.contiguous()


def _varlen_problem(rank, q, k, v, kernel_size, dilation, scale_value):
    _check_qkv(rank, q, k, v)
    _on_device(q, k, v)
    _same_dtype(q, k, v)
    return _fused_problem(rank, q, k, v, kernel_size, (1,) * rank, dilation, (False,) * rank, scale_value)


def varlen_forward_with_lse(rank: int, q, k, v, sizes, kernel_size, dilation, scale):
    """Fused forward of a padded batch whose sample b has spatial extent
    ``sizes[b]`` (``[B, rank]`` ints): ``(out, lse)``, zero at padding."""
    q, k, v = _inner(q), _inner(k), _inner(v)
    scale_value = float(q.shape[-1] ** -0.5 if scale is None else scale)
    prob = _varlen_problem(rank, q, k, v, kernel_size, dilation, scale_value)
    lens = _varlen_lens(rank, sizes, q.device)
    B, Hq = q.shape[0], q.shape[-2]
    sp = tuple(q.shape[1:1 + rank])
    out = torch.empty((B, *sp, Hq, v.shape[-1]), dtype=q.dtype, device=q.device)
    lse = torch.empty((B, *sp, Hq), dtype=torch.float32, device=q.device)
    L = lambda t, tr=1: _byref(_lib.layout(t, rank, tr))  # noqa: E731
    lib = _lib.load()
    rc = _launch(q.device, lib.natten_hip_varlen_forward, _byref(prob), lens.data_ptr(),
                 q.data_ptr(), L(q), k.data_ptr(), L(k), v.data_ptr(), L(v), out.data_ptr(), L(out),
                 lse.data_ptr(), L(lse, 0), _raw_stream(q.device))
    _lib.check(rc, "varlen_forward")
    return out, lse


def varlen_backward(rank: int, d_out, q, k, v, out, lse, sizes, kernel_size, dilation, scale):
    """``(dq, dk, dv)`` of :func:`varlen_forward_with_lse`, zero at padding."""
    q, k, v, out, d_out = _inner(q), _inner(k), _inner(v), _inner(out), _inner(d_out.to(q.dtype))
    lse = lse.to(torch.float32).contiguous()
    scale_value = float(q.shape[-1] ** -0.5 if scale is None else scale)
    prob = _varlen_problem(rank, q, k, v, kernel_size, dilation, scale_value)
    _on_device(d_out, out, lse)
    lens = _varlen_lens(rank, sizes, q.device)
    dq = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    dk = torch.empty(k.shape, dtype=k.dtype, device=k.device)
    dv = torch.empty(v.shape, dtype=v.dtype, device=v.device)
    delta = torch.empty(lse.shape, dtype=torch.float32, device=q.device)
    L = lambda t, tr=1: _byref(_lib.layout(t, rank, tr))  # noqa: E731
    lib = _lib.load()
    rc = _launch(q.device, lib.natten_hip_varlen_backward, _byref(prob), lens.data_ptr(),
                 q.data_ptr(), L(q), k.data_ptr(), L(k), v.data_ptr(), L(v), out.data_ptr(), L(out),
                 d_out.data_ptr(), L(d_out), lse.data_ptr(), L(lse, 0), dq.data_ptr(), L(dq),
                 dk.data_ptr(), L(dk), dv.data_ptr(), L(dv), delta.data_ptr(), L(delta, 0),
                 _raw_stream(q.device))
    _lib.check(rc, "varlen_backward")
    return dq, dk, dv


# ---------------------------------------------------------------------------
# relative-position-bias split ops (extras/allin1/functional.py:47-485):
# NATTEN 0.17 shifted windows, 1-D and 2-D, spatial-first tensors
# ---------------------------------------------------------------------------


def _rpb_problem(rank, ref, heads, dim_qk, dim_v, kernel_size, dilation):
    sp = tuple(ref.shape[1:1 + rank])
    return _lib.problem(
        batch=ref.shape[0], heads_q=heads, heads_kv=heads, dim_qk=dim_qk, dim_v=dim_v, dtype=_lib.dtype_code(ref),
        length=sp, out_length=sp, kernel_size=kernel_size, dilation=dilation, stride=(1,) * rank,
        is_causal=(False,) * rank, scale=None,
    )


def _rpb_table(rank, rpb, heads, kernel_size, dtype):
    if rpb is None:
        return None
    want = (heads, *[2 * k - 1 for k in kernel_size])
    if tuple(rpb.shape) != want:
        raise ValueError(f"rpb must have shape {want}, got {tuple(rpb.shape)}.")
    return rpb.to(dtype).contiguous()


def _register_rpb(b, op, rank, given, used, flag, outs, prob, kernel_size, dilation, out_shape=(), work_floats=0):
    """Register a relative-position-bias op signature with the binding, as
    _register_split (``used``: the tensors with layouts, the bias table aside)."""
    if any(a is not u for a, u in zip(given, used)):
        return
    lays = [_lib.layout(t, rank, 1) for t in (*used[:5 if op != 4 else 2], *outs)]
    blob = b"".join(bytes(x) for x in lays)
    call = b.SplitCall(op, bytes(prob), blob, list(out_shape), False, int(work_floats))
    b.rpb_register(rank, [t for t in given if t is not None], int(flag), kernel_size, dilation, call)


def rpb_qk_forward(rank: int, q, k, rpb, kernel_size, dilation):
    """Logits ``[B, *sp, H, prod(kernel)]`` = q . k + rpb (unscaled), -inf at
    invalid neighbours."""
    b = _lib.binding()
    if b is not None:
        r = b.rpb_qk(rank, q, k, rpb, kernel_size, dilation)
        if r is not None:
            return r
    given = (q, k, rpb)
    _on_device(q, k, rpb)
    _same_dtype(q, k)
    q, k = _inner(q), _inner(k)
    H = q.shape[-2]
    table = _rpb_table(rank, rpb, H, kernel_size, q.dtype)
    prob = _rpb_problem(rank, q, H, q.shape[-1], q.shape[-1], kernel_size, dilation)
    kv = 1
    for x in kernel_size:
        kv *= x
    attn = torch.empty((*q.shape[:-1], kv), dtype=q.dtype, device=q.device)
    L = lambda t: _byref(_lib.layout(t, rank, 1))  # noqa: E731
    rc = _launch(q.device, _lib.load().natten_hip_rpb_qk_forward, _byref(prob), _lib.ptr(q), L(q), _lib.ptr(k),
                 L(k), _lib.ptr(table), _lib.ptr(attn), L(attn), _raw_stream(q.device))
    _lib.check(rc, "rpb_qk_forward")
    if b is not None:
        _register_rpb(b, 4, rank, given, (q, k, table), rpb is not None, (attn,), prob, kernel_size, dilation,
                      out_shape=attn.shape)
    return attn


def rpb_av_forward(rank: int, attn, v, kernel_size, dilation):
    b = _lib.binding()
    if b is not None:
        r = b.rpb_av(rank, attn, v, kernel_size, dilation)
        if r is not None:
            return r
    given = (attn, v)
    _on_device(attn, v)
    attn = _inner(attn.to(v.dtype))
    v = _inner(v)
    prob = _rpb_problem(rank, v, v.shape[-2], v.shape[-1], v.shape[-1], kernel_size, dilation)
    out = torch.empty(v.shape, dtype=v.dtype, device=v.device)
    L = lambda t: _byref(_lib.layout(t, rank, 1))  # noqa: E731
    rc = _launch(v.device, _lib.load().natten_hip_rpb_av_forward, _byref(prob), _lib.ptr(attn), L(attn),
                 _lib.ptr(v), L(v), _lib.ptr(out), L(out), _raw_stream(v.device))
    _lib.check(rc, "rpb_av_forward")
    if b is not None:
        _register_rpb(b, 5, rank, given, (attn, v), 0, (out,), prob, kernel_size, dilation)
    return out


def rpb_qk_backward(rank: int, d_attn, q, k, with_rpb: bool, kernel_size, dilation):
    """``(dq, dk, drpb)``; drpb is None when the op had no bias."""
    b = _lib.binding()
    if b is not None:
        r = b.rpb_qk_bwd(rank, d_attn, q, k, bool(with_rpb), kernel_size, dilation)
        if r is not None:
            return r
    given = (d_attn, q, k)
    _on_device(d_attn, q, k)
    d_attn = _inner(d_attn.to(q.dtype))
    q, k = _inner(q), _inner(k)
    H = q.shape[-2]
    prob = _rpb_problem(rank, q, H, q.shape[-1], q.shape[-1], kernel_size, dilation)
    dq = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    dk = torch.empty(k.shape, dtype=k.dtype, device=k.device)
    drpb = (torch.empty((H, *[2 * x - 1 for x in kernel_size]), dtype=q.dtype, device=q.device)
            if with_rpb else None)
    L = lambda t: _byref(_lib.layout(t, rank, 1))  # noqa: E731
    lib = _lib.load()
    # The bias gradient's partial sums go to a workspace owned here (the
    # library allocates nothing for them); none when the one pass serves.
    work_floats = int(lib.natten_hip_rpb_dbias_workspace(_byref(prob))) if with_rpb else 0
    work = torch.empty(max(work_floats, 0), dtype=torch.float32, device=q.device) if work_floats > 0 else None
    rc = _launch(q.device, lib.natten_hip_rpb_qk_backward_ws, _byref(prob), _lib.ptr(d_attn), L(d_attn),
                 _lib.ptr(q), L(q), _lib.ptr(k), L(k), _lib.ptr(dq), L(dq), _lib.ptr(dk), L(dk), _lib.ptr(drpb),
                 _lib.ptr(work), max(work_floats, 0), _raw_stream(q.device))
    _lib.check(rc, "rpb_qk_backward")
    if b is not None:
        _register_rpb(b, 6, rank, given, (d_attn, q, k), bool(with_rpb), (dq, dk), prob, kernel_size, dilation,
                      out_shape=drpb.shape if drpb is not None else (), work_floats=max(work_floats, 0))
    return dq, dk, drpb


def rpb_av_backward(rank: int, d_out, attn, v, kernel_size, dilation):
    b = _lib.binding()
    if b is not None:
        r = b.rpb_av_bwd(rank, d_out, attn, v, kernel_size, dilation)
        if r is not None:
            return r
    given = (d_out, attn, v)
    _on_device(d_out, attn, v)
    d_out = _inner(d_out.to(v.dtype))
    attn = _inner(attn.to(v.dtype))
    v = _inner(v)
    prob = _rpb_problem(rank, v, v.shape[-2], v.shape[-1], v.shape[-1], kernel_size, dilation)
    d_attn = torch.empty(attn.shape, dtype=attn.dtype, device=attn.device)
    dv = torch.empty(v.shape, dtype=v.dtype, device=v.device)
    L = lambda t: _byref(_lib.layout(t, rank, 1))  # noqa: E731
    rc = _launch(v.device, _lib.load().natten_hip_rpb_av_backward, _byref(prob), _lib.ptr(d_out), L(d_out),
                 _lib.ptr(attn), L(attn), _lib.ptr(v), L(v), _lib.ptr(d_attn), L(d_attn), _lib.ptr(dv), L(dv),
                 _raw_stream(v.device))
    _lib.check(rc, "rpb_av_backward")
    if b is not None:
        _register_rpb(b, 7, rank, given, (d_out, attn, v), 0, (d_attn, dv), prob, kernel_size, dilation)
    return d_attn, dv


# ---------------------------------------------------------------------------
# global keys (the reference's additional_keys / additional_values): extra
# tokens [B, N, Hkv, D] that every query attends besides its neighbourhood,
# inside the fused kernels (natten_hip_forward_global / _backward_global)
# ---------------------------------------------------------------------------

_GLOBAL_OK: dict = {}


def _aligned_runs(*ts) -> bool:
    """Every tensor 16-byte aligned with its outer strides multiples of 8
    elements and a unit innermost stride (what the tile kernels read)."""
    for t in ts:
        if t.data_ptr() % 16 or t.stride(-1) != 1 or any(s % 8 for s in t.stride()[:-1]):
            return False
    return True


def global_supported(rank: int, q, k, v, n: int, kernel_size, stride, dilation, is_causal, backward: bool,
                     gk=None, gv=None, scale=None) -> bool:
    """True when the fused kernels take these global keys (the MFMA tile path:
    bf16/fp16, head dim 32/64/96/128 for q, k and v, stride 1, GPU tensors,
    aligned operands, a positive scale).  The problem part is asked of the
    library (natten_hip_global_supported, cached per shape); the operands'
    own alignment and the scale are checked here on every call."""
    if (q.device.type != "cuda" or q.dtype not in (torch.float16, torch.bfloat16)
            or not (q.dtype == k.dtype == v.dtype) or q.shape[-1] != v.shape[-1] or n < 1):
        return False
    scale_value = float(q.shape[-1] ** -0.5 if scale is None else scale)
    if not scale_value > 0.0 or not _aligned_runs(*(t for t in (q, k, v, gk, gv) if t is not None)):
        return False
    key = (rank, q.dtype, q.shape, k.shape[-2], n, tuple(kernel_size), tuple(stride), tuple(dilation),
           tuple(is_causal), bool(backward))
    ok = _GLOBAL_OK.get(key)
    if ok is None:
        prob = _fused_problem(rank, q, k, v, kernel_size, stride, dilation, is_causal, 1.0)
        ok = bool(_lib.load().natten_hip_global_supported(_byref(prob), int(n), int(bool(backward))))
        if len(_GLOBAL_OK) >= _CACHE_MAX:
            _GLOBAL_OK.clear()
        _GLOBAL_OK[key] = ok
    return ok


def _check_global(q, k, gk, gv):
    if gk.ndim != 4 or gv.ndim != 4 or gk.shape != gv.shape:
        raise ValueError("global keys / values must both be [B, N, heads_kv, dim] with the same shape.")
    if gk.shape[0] != q.shape[0] or gk.shape[2] != k.shape[-2] or gk.shape[3] != q.shape[-1]:
        raise ValueError("global keys must match the batch, kv heads and head dim of the key tensor.")
    _on_device(q, gk, gv)
    _same_dtype(q, gk, gv)


def forward_with_lse_global(rank: int, q, k, v, gk, gv, kernel_size, stride, dilation, is_causal, scale):
    """(out, lse) of neighbourhood attention plus global keys: one softmax
    over each query's window and the N global keys (lse fp32)."""
    q, k, v, gk, gv = _inner(q), _inner(k), _inner(v), _inner(gk), _inner(gv)
    _check_global(q, k, gk, gv)
    scale_value = float(q.shape[-1] ** -0.5 if scale is None else scale)
    sig = _fwd_sig(rank, q, k, v, kernel_size, stride, dilation, is_causal, scale_value)
    out = torch.empty(sig.out_shape, dtype=q.dtype, device=q.device)
    lse = torch.empty(sig.lse_shape, dtype=torch.float32, device=q.device)
    r = sig.refs[1]
    lgk, lgv = _lib.token_layout(gk), _lib.token_layout(gv)
    rc = _launch(q.device, _lib.load().natten_hip_forward_global, sig.prob_ref,
                 q.data_ptr(), r[0], k.data_ptr(), r[1], v.data_ptr(), r[2], gk.data_ptr(), _byref(lgk),
                 gv.data_ptr(), _byref(lgv), int(gk.shape[1]), out.data_ptr(), r[3], lse.data_ptr(), r[4],
                 _raw_stream(q.device))
    _lib.check(rc, "forward_global")
    return out, lse


def fused_backward_global(rank: int, d_out, q, k, v, gk, gv, out, lse, kernel_size, dilation, stride, is_causal,
                          scale, d_lse=None):
    """(dq, dk, dv, dgk, dgv) of forward_with_lse_global."""
    q, k, v, out, d_out, gk, gv = (_inner(t) for t in (q, k, v, out, d_out, gk, gv))
    _check_global(q, k, gk, gv)
    if lse.dtype != torch.float32 or not lse.is_contiguous():
        lse = lse.to(torch.float32).contiguous()
    if d_lse is not None and (d_lse.dtype != torch.float32 or not d_lse.is_contiguous()):
        d_lse = d_lse.to(torch.float32).contiguous()
    scale_value = float(q.shape[-1] ** -0.5 if scale is None else scale)
    sig = _bwd_sig(rank, d_out, q, k, v, out, lse, d_lse, kernel_size, stride, dilation, is_causal, scale_value)
    lib = _lib.load()
    n = int(gk.shape[1])
    work_floats = int(lib.natten_hip_global_workspace(sig.prob_ref, n))
    if work_floats < 0:
        raise ValueError("natten_mps_amd: invalid problem for global keys.")
    dq = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    dk = torch.empty(k.shape, dtype=k.dtype, device=k.device)
    dv = torch.empty(v.shape, dtype=v.dtype, device=v.device)
    dgk = torch.empty(gk.shape, dtype=gk.dtype, device=gk.device)
    dgv = torch.empty(gv.shape, dtype=gv.dtype, device=gv.device)
    delta = torch.empty(sig.lse_shape, dtype=torch.float32, device=q.device)
    work = torch.empty(max(work_floats, 1), dtype=torch.float32, device=q.device)
    r = sig.refs[1]
    T = lambda t: _byref(_lib.token_layout(t))  # noqa: E731
    rc = _launch(q.device, lib.natten_hip_backward_global, sig.prob_ref,
                 q.data_ptr(), r[0], k.data_ptr(), r[1], v.data_ptr(), r[2], gk.data_ptr(), T(gk),
                 gv.data_ptr(), T(gv), n, out.data_ptr(), r[3], d_out.data_ptr(), r[4], lse.data_ptr(), r[5],
                 d_lse.data_ptr() if d_lse is not None else None, r[6], dq.data_ptr(), r[7], dk.data_ptr(), r[8],
                 dv.data_ptr(), r[9], dgk.data_ptr(), T(dgk), dgv.data_ptr(), T(dgv), delta.data_ptr(), r[10],
                 work.data_ptr(), work_floats, _raw_stream(q.device))
    _lib.check(rc, "backward_global")
    return dq, dk, dv, dgk, dgv


# ---------------------------------------------------------------------------
# rank-specific names (the backend-module contract)
# ---------------------------------------------------------------------------


def _bind(rank: int) -> None:
    g = globals()

    def fwd(q, k, v, kernel_size, stride, dilation, is_causal, scale):
        return forward(rank, q, k, v, kernel_size, stride, dilation, is_causal, scale)

    def fwd_lse(q, k, v, kernel_size, stride, dilation, is_causal, scale):
        return forward_with_lse(rank, q, k, v, kernel_size, stride, dilation, is_causal, scale)

    def fbwd(d_out, q, k, v, out, lse, kernel_size, dilation, stride, is_causal, scale, d_lse=None):
        return fused_backward(rank, d_out, q, k, v, out, lse, kernel_size, dilation, stride, is_causal, scale, d_lse)

    def qk(q, k, kernel_size, dilation, stride=(1,) * rank, is_causal=(False,) * rank, scale=None):
        return qk_forward(rank, q, k, kernel_size, dilation, stride, is_causal, scale)

    def av(attn, v, kernel_size, dilation, stride=(1,) * rank, is_causal=(False,) * rank):
        return av_forward(rank, attn, v, kernel_size, dilation, stride, is_causal)

    def qkb(d_attn, q, k, kernel_size, dilation, stride=(1,) * rank, is_causal=(False,) * rank, scale=None):
        return qk_backward(rank, d_attn, q, k, kernel_size, dilation, stride, is_causal, scale)

    def avb(d_out, attn, v, kernel_size, dilation, stride=(1,) * rank, is_causal=(False,) * rank):
        return av_backward(rank, d_out, attn, v, kernel_size, dilation, stride, is_causal)

    def vfwd(q, k, v, sizes, kernel_size, dilation, scale):
        return varlen_forward_with_lse(rank, q, k, v, sizes, kernel_size, dilation, scale)[0]

    def vfwd_lse(q, k, v, sizes, kernel_size, dilation, scale):
        return varlen_forward_with_lse(rank, q, k, v, sizes, kernel_size, dilation, scale)

    def vbwd(d_out, q, k, v, out, lse, sizes, kernel_size, dilation, scale):
        return varlen_backward(rank, d_out, q, k, v, out, lse, sizes, kernel_size, dilation, scale)

    def gsup(q, k, v, n, kernel_size, stride, dilation, is_causal, backward, gk=None, gv=None, scale=None):
        return global_supported(rank, q, k, v, n, kernel_size, stride, dilation, is_causal, backward, gk, gv,
                                scale)

    def gfwd(q, k, v, gk, gv, kernel_size, stride, dilation, is_causal, scale):
        return forward_with_lse_global(rank, q, k, v, gk, gv, kernel_size, stride, dilation, is_causal, scale)

    def gbwd(d_out, q, k, v, gk, gv, out, lse, kernel_size, dilation, stride, is_causal, scale, d_lse=None):
        return fused_backward_global(rank, d_out, q, k, v, gk, gv, out, lse, kernel_size, dilation, stride,
                                     is_causal, scale, d_lse)

    for suffix, fn in (("forward", fwd), ("forward_with_lse", fwd_lse), ("fused_backward", fbwd),
                       ("global_supported", gsup), ("forward_with_lse_global", gfwd),
                       ("fused_backward_global", gbwd),
                       ("qk_forward", qk), ("av_forward", av), ("qk_backward", qkb), ("av_backward", avb),
                       ("varlen_forward", vfwd), ("varlen_forward_with_lse", vfwd_lse),
                       ("varlen_backward", vbwd)):
        name = f"na{rank}d_{suffix}"
        fn.__name__ = fn.__qualname__ = name
        g[name] = fn


for _r in (1, 2, 3):
    _bind(_r)
del _r
