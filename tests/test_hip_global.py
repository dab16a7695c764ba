"""additional_keys / additional_values on the fused kernels (global keys).

The 'hip' backend takes the extra tokens as global keys inside its fused
MFMA kernels: one softmax over each query's window and the extra tokens.  The
reference computes the same thing as a composition (split NA with its LSE,
dense attention over the extra tokens with its LSE, and the sigmoid merge;
``functional.py:74-110,285-299``, ``merge.py:21-156``).  These tests run that
composition through the functional layer over the CPU oracle backend, in
float32 on the same rounded inputs, and compare out, lse and all five
gradients (through both outputs) under the half-precision bound of
``tests/_parity.py``.  Each case also checks that the fused global-key
kernels are the ones that ran.
"""
from __future__ import annotations

import pytest
import torch

from _parity import assert_parity

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0") if torch.cuda.is_available() else None

# rank, spatial, heads q / kv, dim, kernel, dilation, causal, global keys, dtype
CASES = [
    (2, (9, 10), 4, 2, 32, 3, (2, 1), (False, False), 2, torch.bfloat16),
    (2, (14, 13), 4, 4, 64, 5, (1, 1), (True, False), 33, torch.float16),
    (1, (70,), 8, 2, 64, 9, (2,), (True,), 1, torch.bfloat16),
    (3, (5, 6, 7), 2, 2, 32, (3, 3, 5), (1, 2, 1), (False, False, False), 70, torch.bfloat16),
    (2, (16, 16), 2, 2, 128, 3, (1, 1), (False, False), 32, torch.bfloat16),
    (2, (12, 12), 2, 1, 32, 5, (1, 1), (False, False), 5, torch.float16),
    (1, (300,), 4, 4, 32, 33, (1,), (False,), 64, torch.bfloat16),
    (2, (10, 11), 2, 2, 96, 3, (1, 1), (False, False), 7, torch.bfloat16),
]


def _inputs(seed, shapes, dtype):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(s, generator=g, dtype=torch.float32).to(dtype) for s in shapes]


def _run(rank, tensors, do, dl, device, ref_dtype=None, **kw):
    from natten_mps_amd import functional as F

    fn = getattr(F, f"na{rank}d")
    leaves = [(t if ref_dtype is None else t.to(ref_dtype)).to(device).detach().requires_grad_(True)
              for t in tensors]
    out, lse = fn(*leaves[:3], return_lse=True, additional_keys=leaves[3], additional_values=leaves[4], **kw)
    cast = (lambda t: t) if ref_dtype is None else (lambda t: t.to(ref_dtype))
    torch.autograd.backward([out, lse], [cast(do).to(device), cast(dl).to(device)])
    return [out.detach().cpu(), lse.detach().cpu()] + [t.grad.cpu() for t in leaves]


@pytest.mark.parametrize("case", CASES, ids=[f"r{c[0]}-{'x'.join(map(str, c[1]))}-D{c[4]}-n{c[8]}" for c in CASES])
def test_global_keys_match_oracle_composition(case, pure_backend):
    import natten_mps_amd
    from natten_mps_amd._core import _lib

    rank, sp, hq, hkv, dim, ks, dil, causal, n, dtype = case
    B = 2
    q, k, v, gk, gv, do = _inputs(300 + len(sp) + n, [(B, *sp, hq, dim), (B, *sp, hkv, dim), (B, *sp, hkv, dim),
                                                       (B, n, hkv, dim), (B, n, hkv, dim), (B, *sp, hq, dim)], dtype)
    (dl,) = _inputs(400 + n, [(B, *sp, hq)], torch.float32)
    kw = dict(kernel_size=ks, dilation=dil, is_causal=causal)
    # the composition over the oracle backend, float32 on the same rounded inputs
    ref = _run(rank, (q, k, v, gk, gv), do, dl, "cpu", ref_dtype=torch.float32, **kw)
    natten_mps_amd.set_backend("hip")
    _lib.profile_read(reset=True)
    _lib.profile_enable(True)
    try:
        got = _run(rank, (q, k, v, gk, gv), do, dl, DEV, **kw)
        torch.cuda.synchronize()
    finally:
        _lib.profile_enable(False)
    launched = set(_lib.profile_read(reset=True))
    assert {"na_fwd_global_mfma", "na_bwd_q_global_mfma", "na_global_kv_mfma"} <= launched, launched
    assert got[1].dtype == torch.float32  # the merged lse stays fp32, as the composition's
    for name, a, b in zip(("out", "lse", "dq", "dk", "dv", "dgk", "dgv"), got, ref):
        assert_parity(a, b, dtype, name)


def test_global_keys_without_lse_and_without_grad():
    """return_lse=False and an inference call (no autograd) take the same
    kernels and give the same out."""
    from natten_mps_amd import functional as F

    q, k, v, gk, gv = (t.to(DEV) for t in _inputs(7, [(1, 20, 24, 4, 64), (1, 20, 24, 2, 64),
                                                       (1, 20, 24, 2, 64), (1, 3, 2, 64), (1, 3, 2, 64)],
                                                   torch.bfloat16))
    a = F.na2d(q, k, v, kernel_size=7, additional_keys=gk, additional_values=gv)
    with torch.no_grad():
        b, lse = F.na2d(q, k, v, kernel_size=7, return_lse=True, additional_keys=gk, additional_values=gv)
    assert torch.equal(a, b) and lse.shape == (1, 20, 24, 4)


def test_global_keys_backward_is_bitwise_deterministic():
    from natten_mps_amd import functional as F

    q, k, v, gk, gv, do = (t.to(DEV) for t in _inputs(11, [(2, 24, 24, 4, 32), (2, 24, 24, 4, 32),
                                                            (2, 24, 24, 4, 32), (2, 40, 4, 32), (2, 40, 4, 32),
                                                            (2, 24, 24, 4, 32)], torch.bfloat16))

    def grads():
        leaves = [t.detach().requires_grad_(True) for t in (q, k, v, gk, gv)]
        out = F.na2d(*leaves[:3], kernel_size=7, additional_keys=leaves[3], additional_values=leaves[4])
        out.backward(do)
        return [t.grad for t in leaves]

    first = grads()
    for _ in range(3):
        for a, b in zip(first, grads()):
            assert torch.equal(a, b)


def test_global_keys_fall_back_to_the_composition_where_unsupported(pure_backend):
    """fp32 (no MFMA tile) keeps the reference composition on the HIP kernels."""
    import natten_mps_amd
    from natten_mps_amd._core import hip

    q, k, v, gk, gv, do = _inputs(13, [(1, 8, 9, 2, 16), (1, 8, 9, 2, 16), (1, 8, 9, 2, 16), (1, 2, 2, 16),
                                       (1, 2, 2, 16), (1, 8, 9, 2, 16)], torch.float32)
    (dl,) = _inputs(14, [(1, 8, 9, 2)], torch.float32)
    assert not hip.global_supported(2, q.to(DEV), k.to(DEV), v.to(DEV), 2, (3, 3), (1, 1), (1, 1), (False, False),
                                    True)
    ref = _run(2, (q, k, v, gk, gv), do, dl, "cpu", kernel_size=3)
    natten_mps_amd.set_backend("hip")
    got = _run(2, (q, k, v, gk, gv), do, dl, DEV, kernel_size=3)
    for name, a, b in zip(("out", "lse", "dq", "dk", "dv", "dgk", "dgv"), got, ref):
        assert_parity(a, b, torch.float32, name)


def _misaligned(t):
    """The same values at a storage offset of one element: 2-byte aligned,
    so the tile kernels' 16-byte loads cannot read it."""
    buf = torch.empty(t.numel() + 1, dtype=t.dtype, device=t.device)
    view = buf[1:].view(t.shape)
    view.copy_(t)
    return view


@pytest.mark.parametrize("what", ["misaligned_q", "negative_scale"])
def test_global_keys_fall_back_where_operands_decline(what, pure_backend):
    """A problem the library's global-key probe accepts by shape but whose
    operands the tile kernels refuse -- a query view that is not 16-byte
    aligned, or a scale <= 0 -- takes the composition (split NA, dense
    attention, merge) instead of raising, and matches the oracle composition."""
    import natten_mps_amd
    from natten_mps_amd import functional as F
    from natten_mps_amd._core import _lib

    q, k, v, gk, gv, do = _inputs(21, [(2, 10, 12, 2, 32), (2, 10, 12, 2, 32), (2, 10, 12, 2, 32), (2, 3, 2, 32),
                                       (2, 3, 2, 32), (2, 10, 12, 2, 32)], torch.bfloat16)
    (dl,) = _inputs(22, [(2, 10, 12, 2)], torch.float32)
    kw = dict(kernel_size=5)
    if what == "negative_scale":
        kw["scale"] = -0.25
    ref = _run(2, (q, k, v, gk, gv), do, dl, "cpu", ref_dtype=torch.float32, **kw)
    natten_mps_amd.set_backend("hip")
    leaves = [t.to(DEV) for t in (q, k, v, gk, gv)]
    if what == "misaligned_q":
        leaves[0] = _misaligned(leaves[0])
        assert leaves[0].data_ptr() % 16 != 0
    leaves = [t.detach().requires_grad_(True) for t in leaves]
    _lib.profile_read(reset=True)
    _lib.profile_enable(True)
    try:
        out, lse = F.na2d(*leaves[:3], return_lse=True, additional_keys=leaves[3], additional_values=leaves[4], **kw)
        torch.autograd.backward([out, lse], [do.to(DEV), dl.to(DEV)])
        torch.cuda.synchronize()
    finally:
        _lib.profile_enable(False)
    launched = set(_lib.profile_read(reset=True))
    assert not any("global" in n for n in launched), launched
    got = [out.detach().cpu(), lse.detach().cpu()] + [t.grad.cpu() for t in leaves]
    for name, a, b in zip(("out", "lse", "dq", "dk", "dv", "dgk", "dgv"), got, ref):
        assert_parity(a, b, torch.bfloat16, name)
