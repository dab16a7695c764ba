"""ctypes binding of libnatten_hip.so (C ABI in include/natten_hip.h).

The library is built in-tree by ``natten-mps_amd/build_lib.py`` and loaded from
this package directory.  No torch types cross the boundary: tensors are passed
as device pointers plus element strides, the stream as a raw ``hipStream_t``.
"""
from __future__ import annotations

import ctypes
import os
import threading
from typing import Optional, Sequence

import torch

LIB_NAME = "libnatten_hip.so"
LIB_PATH = os.environ.get("NATTEN_HIP_LIB") or os.path.join(
    os.path.dirname(os.path.dirname(os.path.abspath(__file__))), LIB_NAME)
ABI_VERSION = 1
# C++ host binding of the fused forward / backward (csrc/na_torch.cpp), built
# beside the library; NATTEN_HIP_BINDING=0 keeps those calls on ctypes.
BIND_PATH = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "_natten_torch.so")

F32, F16, BF16 = 0, 1, 2
_DTYPES = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}

ENTRY_POINTS = (
    "natten_hip_abi_version",
    "natten_hip_last_error",
    "natten_hip_mfma_lds_check",
    "natten_hip_forward",
    "natten_hip_backward",
    "natten_hip_backward_noalloc",
    "natten_hip_global_supported",
    "natten_hip_global_workspace",
    "natten_hip_forward_global",
    "natten_hip_backward_global",
    "natten_hip_qk_forward",
    "natten_hip_av_forward",
    "natten_hip_qk_backward",
    "natten_hip_av_backward",
    "natten_hip_neighborhood_map",
    "natten_hip_varlen_forward",
    "natten_hip_varlen_backward",
    "natten_hip_rpb_qk_forward",
    "natten_hip_rpb_av_forward",
    "natten_hip_rpb_qk_backward",
    "natten_hip_rpb_dbias_workspace",
    "natten_hip_rpb_qk_backward_ws",
    "natten_hip_rpb_av_backward",
    "natten_hip_profile_enable",
    "natten_hip_profile_read",
)


class Problem(ctypes.Structure):
    _fields_ = [
        ("batch", ctypes.c_int32),
        ("heads_q", ctypes.c_int32),
        ("heads_kv", ctypes.c_int32),
        ("dim_qk", ctypes.c_int32),
        ("dim_v", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
        ("has_scale", ctypes.c_int32),
        ("scale", ctypes.c_float),
        ("length", ctypes.c_int32 * 3),
        ("out_length", ctypes.c_int32 * 3),
        ("kernel", ctypes.c_int32 * 3),
        ("dilation", ctypes.c_int32 * 3),
        ("stride", ctypes.c_int32 * 3),
        ("causal", ctypes.c_int32 * 3),
    ]


class KernelStat(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char * 64), ("launches", ctypes.c_int64), ("total_ms", ctypes.c_double),
                ("min_ms", ctypes.c_double), ("max_ms", ctypes.c_double)]


class Layout(ctypes.Structure):
    _fields_ = [("batch", ctypes.c_int64), ("axis", ctypes.c_int64 * 3), ("head", ctypes.c_int64)]


_P = ctypes.POINTER
_VP = ctypes.c_void_p
_LP = _P(Layout)

_SIGNATURES = {
    "natten_hip_abi_version": ([], ctypes.c_int),
    "natten_hip_last_error": ([], ctypes.c_char_p),
    "natten_hip_mfma_lds_check": ([_P(ctypes.c_int32)], ctypes.c_int),
    "natten_hip_forward": ([_P(Problem)] + [_VP, _LP] * 5 + [_VP], ctypes.c_int),
    "natten_hip_backward": ([_P(Problem)] + [_VP, _LP] * 11 + [_VP], ctypes.c_int),
    "natten_hip_backward_noalloc": ([_P(Problem)] + [_VP, _LP] * 10 + [_VP], ctypes.c_int),
    "natten_hip_global_supported": ([_P(Problem), ctypes.c_int32, ctypes.c_int32], ctypes.c_int),
    "natten_hip_global_workspace": ([_P(Problem), ctypes.c_int32], ctypes.c_int64),
    "natten_hip_forward_global": ([_P(Problem)] + [_VP, _LP] * 5 + [ctypes.c_int32] + [_VP, _LP] * 2 + [_VP],
                                  ctypes.c_int),
    "natten_hip_backward_global": ([_P(Problem)] + [_VP, _LP] * 5 + [ctypes.c_int32] + [_VP, _LP] * 10
                                   + [_VP, ctypes.c_int64, _VP], ctypes.c_int),
    "natten_hip_qk_forward": ([_P(Problem)] + [_VP, _LP] * 3 + [_VP], ctypes.c_int),
    "natten_hip_av_forward": ([_P(Problem)] + [_VP, _LP] * 3 + [_VP], ctypes.c_int),
    "natten_hip_qk_backward": ([_P(Problem)] + [_VP, _LP] * 5 + [_VP], ctypes.c_int),
    "natten_hip_av_backward": ([_P(Problem)] + [_VP, _LP] * 5 + [_VP], ctypes.c_int),
    "natten_hip_neighborhood_map": ([_P(Problem), _VP, _VP, _VP], ctypes.c_int),
    "natten_hip_varlen_forward": ([_P(Problem), _VP] + [_VP, _LP] * 5 + [_VP], ctypes.c_int),
    "natten_hip_varlen_backward": ([_P(Problem), _VP] + [_VP, _LP] * 10 + [_VP], ctypes.c_int),
    "natten_hip_rpb_qk_forward": ([_P(Problem)] + [_VP, _LP] * 2 + [_VP] + [_VP, _LP] + [_VP], ctypes.c_int),
    "natten_hip_rpb_av_forward": ([_P(Problem)] + [_VP, _LP] * 3 + [_VP], ctypes.c_int),
    "natten_hip_rpb_qk_backward": ([_P(Problem)] + [_VP, _LP] * 5 + [_VP, _VP], ctypes.c_int),
    "natten_hip_rpb_dbias_workspace": ([_P(Problem)], ctypes.c_int64),
    "natten_hip_rpb_qk_backward_ws": ([_P(Problem)] + [_VP, _LP] * 5 + [_VP, _VP, ctypes.c_int64, _VP],
                                      ctypes.c_int),
    "natten_hip_rpb_av_backward": ([_P(Problem)] + [_VP, _LP] * 5 + [_VP], ctypes.c_int),
    "natten_hip_profile_enable": ([ctypes.c_int], ctypes.c_int),
    "natten_hip_profile_read": ([_P(KernelStat), ctypes.c_int, ctypes.c_int], ctypes.c_int),
}

_lib = None
_lock = threading.Lock()


def is_built() -> bool:
    return os.path.exists(LIB_PATH)


_bind = None
_bind_checked = False


def binding():
    """The C++ host binding module, or None when it is not built or switched
    off.  It links to libnatten_hip.so by its soname, so the library loaded
    here first is the one it calls."""
    global _bind, _bind_checked
    if _bind_checked:
        return _bind
    load()
    mod = None
    if os.environ.get("NATTEN_HIP_BINDING", "1") != "0" and os.path.exists(BIND_PATH):
        import importlib.util

        spec = importlib.util.spec_from_file_location("_natten_torch", BIND_PATH)
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        if mod.abi_version != ABI_VERSION:
            raise RuntimeError("natten_mps_amd: _natten_torch.so ABI version mismatch; rebuild it.")
    _bind, _bind_checked = mod, True
    return _bind


def load() -> ctypes.CDLL:
    """Load the library once; raise a clear error when it is missing."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not is_built():
            raise RuntimeError(
                f"natten_mps_amd: the HIP library {LIB_PATH} is not built. "
                "Run `python natten-mps_amd/build_lib.py` (or __graft_entry__.build())."
            )
        lib = ctypes.CDLL(LIB_PATH)
        for name, (args, res) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = res
        if lib.natten_hip_abi_version() != ABI_VERSION:
            raise RuntimeError("natten_mps_amd: libnatten_hip.so ABI version mismatch; rebuild it.")
        _lib = lib
    return _lib


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = load().natten_hip_last_error().decode(errors="replace")
        if rc == 1:
            raise ValueError(f"natten hip {what}: {msg}")
        if rc == 2:
            raise NotImplementedError(f"natten hip {what}: {msg}")
        raise RuntimeError(f"natten hip {what}: {msg}")


def dtype_code(t: torch.Tensor) -> int:
    try:
        return _DTYPES[t.dtype]
    except KeyError:
        raise TypeError(f"natten hip backend supports float32, float16 and bfloat16, got {t.dtype}") from None


def _pad3(vals: Sequence[int], fill: int) -> list:
    vals = list(vals)
    return [fill] * (3 - len(vals)) + vals


def problem(*, batch: int, heads_q: int, heads_kv: int, dim_qk: int, dim_v: int, dtype: int,
            length: Sequence[int], out_length: Sequence[int], kernel_size: Sequence[int],
            dilation: Sequence[int], stride: Sequence[int], is_causal: Sequence[bool],
            scale: Optional[float]) -> Problem:
    p = Problem()
    p.batch, p.heads_q, p.heads_kv = batch, heads_q, heads_kv
    p.dim_qk, p.dim_v, p.dtype = dim_qk, dim_v, dtype
    p.has_scale = 0 if scale is None else 1
    p.scale = 1.0 if scale is None else float(scale)
    for name, vals, fill in (("length", length, 1), ("out_length", out_length, 1), ("kernel", kernel_size, 1),
                             ("dilation", dilation, 1), ("stride", stride, 1)):
        getattr(p, name)[:] = [int(x) for x in _pad3(vals, fill)]
    p.causal[:] = [int(bool(x)) for x in _pad3(is_causal, False)]
    return p


def layout(t: torch.Tensor, rank: int, trailing: int) -> Layout:
    """Strides of a ``[B, *sp(rank), H, *trailing]`` tensor; ``trailing`` is
    the number of contiguous innermost dims after the head dim (1 for
    q/k/v/out/attn, 0 for lse)."""
    lay = Layout()
    st = t.stride()
    lay.batch = st[0]
    sp = list(st[1:1 + rank])
    lay.axis[:] = [0] * (3 - rank) + sp
    lay.head = st[1 + rank]
    return lay


def token_layout(t: torch.Tensor) -> Layout:
    """Strides of a ``[B, N, H, D]`` tensor of tokens (global keys): the token
    stride goes in axis[2]."""
    lay = Layout()
    st = t.stride()
    lay.batch = st[0]
    lay.axis[:] = [0, 0, st[1]]
    lay.head = st[2]
    return lay


def ptr(t: Optional[torch.Tensor]):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream_of(t: torch.Tensor):
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def profile_enable(on: bool) -> None:
    """Bracket every library launch with HIP events on its stream."""
    load().natten_hip_profile_enable(1 if on else 0)


def profile_read(reset: bool = True) -> dict:
    """Per-kernel {name: (launches, total_ms, min_ms, max_ms)} of the timed launches."""
    lib = load()
    n = lib.natten_hip_profile_read(None, 0, 0)
    buf = (KernelStat * max(n, 1))()
    n = lib.natten_hip_profile_read(buf, n, 1 if reset else 0)
    return {buf[i].name.decode(): (buf[i].launches, buf[i].total_ms, buf[i].min_ms, buf[i].max_ms)
            for i in range(n)}
