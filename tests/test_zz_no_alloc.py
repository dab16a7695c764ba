"""The allocation-free backward (natten_hip_backward_noalloc) against the
ordinary one (natten_hip_backward), through the C ABI.

The no-alloc entry point keeps its delta rows in the library's static device
scratch and builds no geometry table.  Called before any backward table of
the shape exists, it runs the general tile kernels, which compute their
geometry themselves; called again once the ordinary call has built its
tables, it runs the ordinary call's kernels.  Results are bitwise equal to
the ordinary call's, except the first call of a 1-D problem that the
ordinary path runs on the 8x8 tile kernels' 1-D mode (the general tile
kernels sum in another order there): that pair is compared under the parity
bound of tests/_parity.py.  The calls run in a row, each smaller than the one
before, so a later call finds the scratch holding an earlier call's (larger)
contents.
"""
import ctypes

import pytest
import torch

from _parity import assert_parity
from natten_mps_amd._core import _lib, hip

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")

# rank, batch, spatial, heads q / kv, dim, kernel, dilation, causal, dtype,
# with an upstream lse gradient
CALLS = [
    (2, 8, (56, 56), 4, 4, 32, (7, 7), (1, 1), (False, False), torch.bfloat16, False),
    (2, 2, (40, 36), 2, 2, 64, (5, 7), (2, 1), (True, False), torch.float16, True),
    (1, 2, (300,), 4, 2, 64, (9,), (3,), (True,), torch.bfloat16, False),
    (3, 1, (6, 10, 12), 2, 2, 32, (3, 5, 5), (1, 2, 1), (False, False, False), torch.bfloat16, False),
    (2, 1, (17, 23), 2, 2, 16, (5, 3), (1, 1), (False, False), torch.float32, True),
]


def _inputs(seed, B, sp, hq, hkv, dim, dtype):
    g = torch.Generator(device="cpu").manual_seed(seed)
    mk = lambda h: torch.randn(B, *sp, h, dim, generator=g).to(DEV, dtype)  # noqa: E731
    return mk(hq), mk(hkv), mk(hkv), mk(hq)


def _noalloc_backward(rank, do, q, k, v, out, lse, d_lse, ks, dil, causal):
    stride = (1,) * rank
    sig = hip._bwd_sig(rank, do, q, k, v, out, lse, d_lse, ks, stride, dil, causal, float(q.shape[-1] ** -0.5))
    r = sig.refs[1]
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    lib = _lib.load()
    rc = lib.natten_hip_backward_noalloc(
        ctypes.byref(sig.prob), q.data_ptr(), r[0], k.data_ptr(), r[1], v.data_ptr(), r[2], out.data_ptr(), r[3],
        do.data_ptr(), r[4], lse.data_ptr(), r[5], d_lse.data_ptr() if d_lse is not None else None, r[6],
        dq.data_ptr(), r[7], dk.data_ptr(), r[8], dv.data_ptr(), r[9],
        torch.cuda.current_stream(DEV).cuda_stream)
    _lib.check(rc, "backward_noalloc")
    return dq, dk, dv


def test_noalloc_backward_equals_backward():
    for i, (rank, B, sp, hq, hkv, dim, ks, dil, causal, dtype, with_dlse) in enumerate(CALLS):
        print(f"no-alloc call {i}: rank={rank} B={B} sp={sp} heads={hq}/{hkv} dim={dim} kernel={ks} "
              f"dilation={dil} causal={causal} {dtype} dlse={with_dlse}", flush=True)
        q, k, v, do = _inputs(500 + i, B, sp, hq, hkv, dim, dtype)
        stride = (1,) * rank
        out, lse = hip.forward_with_lse(rank, q, k, v, ks, stride, dil, causal, None)
        d_lse = None
        if with_dlse:
            g = torch.Generator(device="cpu").manual_seed(600 + i)
            d_lse = torch.randn(tuple(lse.shape), generator=g).to(DEV)
        # the no-alloc call first: no backward geometry table exists yet for
        # the shape, so its tile kernels compute their geometry themselves
        got = _noalloc_backward(rank, do, q, k, v, out, lse, d_lse, ks, dil, causal)
        ref = hip.fused_backward(rank, do, q, k, v, out, lse, ks, dil, stride, causal, None, d_lse=d_lse)
        torch.cuda.synchronize()
        one_d_tiles = rank == 1 and dim in (32, 64)
        for name, a, b in zip(("dq", "dk", "dv"), got, ref):
            if one_d_tiles:
                assert_parity(a, b, dtype, f"call {i}: {name}")
            else:
                assert torch.equal(a, b), f"call {i}: {name} differs from natten_hip_backward"
        # again, now that the ordinary call's tables exist: its kernels
        again = _noalloc_backward(rank, do, q, k, v, out, lse, d_lse, ks, dil, causal)
        torch.cuda.synchronize()
        for name, a, b in zip(("dq", "dk", "dv"), again, ref):
            assert torch.equal(a, b), f"call {i} (tables built): {name} differs from natten_hip_backward"


def test_noalloc_backward_rejects_problems_past_the_scratch():
    """batch x query positions x heads_q above 4 Mi: a clear error, nothing
    launched (checked on the host before any device work)."""
    B, sp, h, dim = 2, (2 ** 20 + 8,), 2, 32
    prob = _lib.problem(batch=B, heads_q=h, heads_kv=h, dim_qk=dim, dim_v=dim, dtype=_lib.BF16, length=sp,
                        out_length=sp, kernel_size=(3,), dilation=(1,), stride=(1,), is_causal=(False,),
                        scale=dim ** -0.5)
    dummy = torch.empty(16, device=DEV)
    lay = _lib.Layout()
    lib = _lib.load()
    args = [ctypes.byref(prob)] + [dummy.data_ptr(), ctypes.byref(lay)] * 10 + [None]
    rc = lib.natten_hip_backward_noalloc(*args)
    assert rc == 2  # NATTEN_ERR_UNSUPPORTED
    msg = lib.natten_hip_last_error().decode()
    assert "exceed the scratch maximum" in msg and "natten_hip_backward" in msg
