"""Backend dispatch (mirrors ``_core/ops.py`` of /root/reference/src/natten_mps).

A backend is a module providing the nine forward functions below (checked at
registration, as ``_core/ops.py:38-42`` does); the six ``*_backward``
functions may return ``None`` ("not available").  This build ships one
backend, ``'hip'``; ``'auto'`` resolves to it when a ROCm GPU and the built
library are present.  Other backends (for instance a CPU reference used as a
test oracle) can be added with :func:`register_backend`; ``'auto'`` prefers
``'hip'`` and then any other registered, available backend in registration
order.

Environment: ``NATTEN_BACKEND`` in {auto, hip, <registered name>} sets the
initial choice (read at import, like ``_core/ops.py:34``).
"""
from __future__ import annotations

import os

from . import hip

_REQUIRED_BACKEND_FUNCTIONS = (
    "na1d_forward",
    "na2d_forward",
    "na3d_forward",
    "na1d_qk_forward",
    "na1d_av_forward",
    "na2d_qk_forward",
    "na2d_av_forward",
    "na3d_qk_forward",
    "na3d_av_forward",
)

_ACTIVE_BACKEND = os.environ.get("NATTEN_BACKEND", "auto")
_BACKEND_REGISTRY = {}


def register_backend(name, module):
    for fn_name in _REQUIRED_BACKEND_FUNCTIONS:
        if not hasattr(module, fn_name):
            raise ValueError(f"Backend '{name}' does not define required function '{fn_name}'.")
    _BACKEND_REGISTRY[name] = module


def unregister_backend(name):
    if name == "hip":
        raise ValueError("the 'hip' backend cannot be unregistered.")
    global _ACTIVE_BACKEND
    _BACKEND_REGISTRY.pop(name, None)
    if _ACTIVE_BACKEND == name:
        _ACTIVE_BACKEND = "auto"


def registered_backends():
    return list(_BACKEND_REGISTRY)


def _backend_available(name: str) -> bool:
    module = _BACKEND_REGISTRY[name]
    fn = getattr(module, "is_available", None)
    if callable(fn):
        return bool(fn())
    return True


def set_backend(name):
    global _ACTIVE_BACKEND
    if name == "auto":
        _ACTIVE_BACKEND = "auto"
        return
    if name not in _BACKEND_REGISTRY:
        valid = ["auto", *_BACKEND_REGISTRY.keys()]
        raise ValueError(f"Unknown backend '{name}'. Expected one of: {valid}.")
    if not _backend_available(name):
        raise NotImplementedError(
            f"Backend '{name}' is not available in this build (it needs a ROCm GPU and the built "
            "libnatten_hip.so). Use set_backend('auto') or register another backend."
        )
    _ACTIVE_BACKEND = name


def get_backend():
    if _ACTIVE_BACKEND == "auto":
        return _resolve_backend()
    return _ACTIVE_BACKEND


def _resolve_backend():
    order = ["hip"] + [n for n in _BACKEND_REGISTRY if n != "hip"]
    for name in order:
        if name in _BACKEND_REGISTRY and _backend_available(name):
            return name
    raise RuntimeError(
        "No valid backend for natten_mps_amd: the 'hip' backend needs a ROCm GPU and the built "
        "libnatten_hip.so (python natten-mps_amd/build_lib.py)."
    )


def active_module():
    return _BACKEND_REGISTRY[get_backend()]


_active_module = active_module


def na1d_forward(q, k, v, kernel_size, stride, dilation, is_causal, scale):
    return _active_module().na1d_forward(q, k, v, kernel_size, stride, dilation, is_causal, scale)


def na2d_forward(q, k, v, kernel_size, stride, dilation, is_causal, scale):
    return _active_module().na2d_forward(q, k, v, kernel_size, stride, dilation, is_causal, scale)


def na3d_forward(q, k, v, kernel_size, stride, dilation, is_causal, scale):
    return _active_module().na3d_forward(q, k, v, kernel_size, stride, dilation, is_causal, scale)


def na1d_qk_forward(q, k, kernel_size, dilation, stride=(1,), is_causal=(False,), scale=None):
    return _active_module().na1d_qk_forward(q, k, kernel_size, dilation, stride, is_causal, scale)


def na2d_qk_forward(q, k, kernel_size, dilation, stride=(1, 1), is_causal=(False, False), scale=None):
    return _active_module().na2d_qk_forward(q, k, kernel_size, dilation, stride, is_causal, scale)


def na3d_qk_forward(q, k, kernel_size, dilation, stride=(1, 1, 1), is_causal=(False, False, False), scale=None):
    return _active_module().na3d_qk_forward(q, k, kernel_size, dilation, stride, is_causal, scale)


def na1d_av_forward(attn, v, kernel_size, dilation, stride=(1,), is_causal=(False,)):
    return _active_module().na1d_av_forward(attn, v, kernel_size, dilation, stride, is_causal)


def na2d_av_forward(attn, v, kernel_size, dilation, stride=(1, 1), is_causal=(False, False)):
    return _active_module().na2d_av_forward(attn, v, kernel_size, dilation, stride, is_causal)


def na3d_av_forward(attn, v, kernel_size, dilation, stride=(1, 1, 1), is_causal=(False, False, False)):
    return _active_module().na3d_av_forward(attn, v, kernel_size, dilation, stride, is_causal)


# Backward dispatch -- None means "not available" (re-differentiate instead).
# `scale` is forwarded only when given, so backends with the reference's
# seven-argument signature keep working.


def _qk_bwd(rank, d_attn, q, k, kernel_size, dilation, stride, is_causal, scale):
    fn = getattr(_active_module(), f"na{rank}d_qk_backward", None)
    if fn is None:
        return None
    if scale is None:
        return fn(d_attn, q, k, kernel_size, dilation, stride, is_causal)
    return fn(d_attn, q, k, kernel_size, dilation, stride, is_causal, scale=scale)


def _av_bwd(rank, d_out, attn, v, kernel_size, dilation, stride, is_causal):
    fn = getattr(_active_module(), f"na{rank}d_av_backward", None)
    if fn is None:
        return None
    return fn(d_out, attn, v, kernel_size, dilation, stride, is_causal)


def na1d_qk_backward(d_attn, q, k, kernel_size, dilation, stride=(1,), is_causal=(False,), scale=None):
    return _qk_bwd(1, d_attn, q, k, kernel_size, dilation, stride, is_causal, scale)


def na2d_qk_backward(d_attn, q, k, kernel_size, dilation, stride=(1, 1), is_causal=(False, False), scale=None):
    return _qk_bwd(2, d_attn, q, k, kernel_size, dilation, stride, is_causal, scale)


def na3d_qk_backward(d_attn, q, k, kernel_size, dilation, stride=(1, 1, 1), is_causal=(False, False, False),
                     scale=None):
    return _qk_bwd(3, d_attn, q, k, kernel_size, dilation, stride, is_causal, scale)


def na1d_av_backward(d_out, attn, v, kernel_size, dilation, stride=(1,), is_causal=(False,)):
    return _av_bwd(1, d_out, attn, v, kernel_size, dilation, stride, is_causal)


def na2d_av_backward(d_out, attn, v, kernel_size, dilation, stride=(1, 1), is_causal=(False, False)):
    return _av_bwd(2, d_out, attn, v, kernel_size, dilation, stride, is_causal)


def na3d_av_backward(d_out, attn, v, kernel_size, dilation, stride=(1, 1, 1), is_causal=(False, False, False)):
    return _av_bwd(3, d_out, attn, v, kernel_size, dilation, stride, is_causal)


register_backend("hip", hip)

if _ACTIVE_BACKEND not in {"auto", *_BACKEND_REGISTRY}:
    _ACTIVE_BACKEND = "auto"
