"""Variable-length attention on the 'hip' backend (natten_hip_varlen_forward /
_backward through na{1,2,3}d_varlen) against the CPU oracle's per-sample
composition (oracle/pure.py, _core/pure.py:573-673), with the cases of the
reference's tests/test_varlen_na{1,2,3}d.py: uniform, mixed, minimum and
asymmetric sizes, dilation, custom scale, padding zero in outputs and
gradients, gradients per sample.

Tolerances: fp32 outputs 1e-5, fp32 gradients 1e-4 (the reference's varlen
gradient tests); bf16 under the half-precision bound of tests/_parity.py,
against the oracle evaluated in fp32 on the same rounded inputs.
"""
from __future__ import annotations

import pytest
import torch

from _parity import assert_parity

import oracle.pure as P

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0") if torch.cuda.is_available() else None
ORACLE = {1: P.na1d_varlen_forward, 2: P.na2d_varlen_forward, 3: P.na3d_varlen_forward}


@pytest.fixture(autouse=True)
def _hip():
    import natten_mps_amd

    natten_mps_amd.set_backend("hip")
    yield


def _fn(rank):
    from natten_mps_amd import functional as F

    return {1: F.na1d_varlen, 2: F.na2d_varlen, 3: F.na3d_varlen}[rank]


def _inputs(seed, shape, dtype, n=4):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(shape, generator=g, dtype=torch.float32).to(dtype) for _ in range(n)]


CASES = [
    # rank, padded shape [B, *sp, H, D], per-sample sizes, kernel, dilation, scale
    (1, (3, 40, 2, 32), [[40], [23], [9]], (5,), (1,), None),
    (1, (2, 64, 4, 16), [[64], [31]], (7,), (3,), 0.3),
    (2, (3, 12, 12, 2, 16), [[12, 12], [8, 10], [6, 6]], (3, 3), (1, 1), None),
    (2, (2, 16, 16, 2, 32), [[16, 16], [10, 12]], (3, 3), (2, 2), None),
    (2, (2, 16, 16, 2, 16), [[16, 8], [6, 14]], (3, 5), (1, 1), 0.1),
    (2, (2, 12, 12, 2, 8), [[3, 3], [3, 3]], (3, 3), (1, 1), None),
    (3, (2, 6, 8, 8, 2, 16), [[6, 8, 8], [4, 5, 7]], (3, 3, 3), (1, 1, 1), None),
]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("case", CASES, ids=lambda c: f"{c[0]}d-{c[1]}-{c[2]}")
def test_varlen_forward_matches_oracle(case, dtype):
    rank, shape, sizes, ks, dil, scale = case
    q, k, v, _ = _inputs(11, shape, dtype)
    sz = torch.tensor(sizes, dtype=torch.int32)
    arg = sz[:, 0] if rank == 1 else sz
    out = _fn(rank)(q.to(DEV), k.to(DEV), v.to(DEV), arg.to(DEV), kernel_size=ks, dilation=dil, scale=scale).cpu()
    ref = ORACLE[rank](q.float(), k.float(), v.float(), sz, ks, dil, scale)
    assert_parity(out, ref, dtype, "varlen out")
    for b, ext in enumerate(sizes):  # padding exactly zero
        mask = torch.ones(shape[1:1 + rank], dtype=torch.bool)
        mask[tuple(slice(0, n) for n in ext)] = False
        assert (out[b][mask] == 0).all()


@pytest.mark.parametrize("case", [CASES[0], CASES[2], CASES[3], CASES[6]], ids=lambda c: f"{c[0]}d-{c[2]}")
def test_varlen_backward_matches_oracle(case):
    rank, shape, sizes, ks, dil, scale = case
    q, k, v, do = _inputs(23, shape, torch.float32)
    sz = torch.tensor(sizes, dtype=torch.int32)
    arg = sz[:, 0] if rank == 1 else sz
    leaves = [t.to(DEV).requires_grad_(True) for t in (q, k, v)]
    out = _fn(rank)(*leaves, arg.to(DEV), kernel_size=ks, dilation=dil, scale=scale)
    out.backward(do.to(DEV))
    got = [t.grad.cpu() for t in leaves]
    ref_leaves = [t.clone().requires_grad_(True) for t in (q, k, v)]
    ORACLE[rank](*ref_leaves, sz, ks, dil, scale).backward(do)
    for name, a, b in zip("qkv", got, ref_leaves):
        torch.testing.assert_close(a, b.grad, atol=1e-4, rtol=1e-4, msg=lambda m: f"d{name}: {m}")
    for b, ext in enumerate(sizes):  # gradients at padding exactly zero
        mask = torch.ones(shape[1:1 + rank], dtype=torch.bool)
        mask[tuple(slice(0, n) for n in ext)] = False
        for g in got:
            assert (g[b][mask] == 0).all()


# bf16 / fp16 with head dims 32-128: the MFMA tile kernels' variable-length
# instances (sample extents read in the kernels, padding zeroed by a second
# launch).
TILE_CASES = [
    # rank, padded shape [B, *sp, H, D], per-sample sizes, kernel, dilation, scale
    (1, (3, 70, 4, 64), [[70], [41], [19]], (7,), (1,), None),
    (1, (2, 300, 2, 32), [[300], [133]], (33,), (2,), 0.2),
    (1, (2, 40, 2, 32), [[40], [26]], (6,), (1,), None),
    (2, (3, 20, 24, 2, 32), [[20, 24], [13, 9], [7, 16]], (5, 7), (1, 1), None),
    (2, (2, 16, 18, 4, 128), [[16, 18], [11, 12]], (3, 5), (1, 2), None),
    (2, (2, 14, 14, 2, 96), [[14, 14], [9, 10]], (3, 3), (1, 1), None),
    (3, (2, 8, 10, 12, 2, 64), [[8, 10, 12], [5, 6, 9]], (3, 3, 5), (1, 1, 1), None),
]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("case", TILE_CASES, ids=lambda c: f"{c[0]}d-D{c[1][-1]}-{c[2]}")
def test_varlen_tile_path(case, dtype):
    """Forward and all three gradients of the MFMA variable-length path
    against the oracle's per-sample composition in fp32 on the same rounded
    inputs; outputs and gradients exactly zero at padding."""
    from natten_mps_amd._core import _lib

    rank, shape, sizes, ks, dil, scale = case
    q, k, v, do = _inputs(31, shape, dtype)
    sz = torch.tensor(sizes, dtype=torch.int32)
    arg = sz[:, 0] if rank == 1 else sz
    leaves = [t.to(DEV).requires_grad_(True) for t in (q, k, v)]
    _lib.profile_read(reset=True)
    _lib.profile_enable(True)
    try:
        out = _fn(rank)(*leaves, arg.to(DEV), kernel_size=ks, dilation=dil, scale=scale)
        out.backward(do.to(DEV))
        torch.cuda.synchronize()
    finally:
        _lib.profile_enable(False)
    launched = set(_lib.profile_read(reset=True))
    assert {"na_varlen_fwd_mfma", "na_varlen_bwd_q_mfma", "na_varlen_bwd_kv_mfma", "na_varlen_pad_zero"} <= launched, \
        launched
    ref_leaves = [t.float().requires_grad_(True) for t in (q, k, v)]
    ref = ORACLE[rank](*ref_leaves, sz, ks, dil, scale)
    ref.backward(do.float())
    got = [out.detach().cpu()] + [t.grad.cpu() for t in leaves]
    want = [ref.detach()] + [t.grad for t in ref_leaves]
    for name, a, b in zip(("out", "dq", "dk", "dv"), got, want):
        assert_parity(a, b, dtype, f"varlen {name}")
    for b, ext in enumerate(sizes):  # padding exactly zero
        mask = torch.ones(shape[1:1 + rank], dtype=torch.bool)
        mask[tuple(slice(0, n) for n in ext)] = False
        for g in got:
            assert (g[b][mask] == 0).all()


def test_varlen_uniform_sizes_equal_na_on_gpu():
    """All sizes at the maximum: na2d_varlen == na2d (the reference's
    test_uniform_sizes)."""
    from natten_mps_amd import functional as F

    q, k, v, _ = (t.to(DEV) for t in _inputs(5, (2, 8, 8, 2, 16), torch.float32))
    sz = torch.tensor([[8, 8], [8, 8]], dtype=torch.int32, device=DEV)
    torch.testing.assert_close(F.na2d_varlen(q, k, v, sz, kernel_size=3), F.na2d(q, k, v, kernel_size=3),
                               atol=1e-5, rtol=1e-5)


def test_varlen_even_kernel_full_window_sample():
    """A sample whose extent equals an even kernel takes na*d's full-window
    path: plain softmax attention over the sample (closed form)."""
    from natten_mps_amd import functional as F

    q, k, v, _ = _inputs(7, (2, 10, 2, 8), torch.float32)
    lens = torch.tensor([4, 10], dtype=torch.int32)
    out = F.na1d_varlen(q.to(DEV), k.to(DEV), v.to(DEV), lens.to(DEV), kernel_size=4).cpu()
    s = torch.einsum("nhd,mhd->hnm", q[0, :4], k[0, :4]) * 8 ** -0.5
    ref0 = torch.einsum("hnm,mhd->nhd", s.softmax(-1), v[0, :4])
    torch.testing.assert_close(out[0, :4], ref0, atol=1e-5, rtol=1e-5)
    assert (out[0, 4:] == 0).all()
    ref1 = P.na1d_forward(q[1:], k[1:], v[1:], (4,), (1,), (1,), (False,), None)
    torch.testing.assert_close(out[1:], ref1, atol=1e-5, rtol=1e-5)


def test_varlen_is_one_launch_per_op():
    """The whole padded batch goes through one forward launch and one
    backward pair, whatever the batch size (no per-sample loop)."""
    from natten_mps_amd import functional as F
    from natten_mps_amd._core import _lib

    q, k, v, do = (t.to(DEV) for t in _inputs(9, (6, 30, 2, 32), torch.float32))
    leaves = [t.requires_grad_(True) for t in (q, k, v)]
    lens = torch.tensor([30, 29, 17, 12, 30, 8], dtype=torch.int32, device=DEV)
    F.na1d_varlen(*leaves, lens, kernel_size=5)  # warm caches
    torch.cuda.synchronize()
    _lib.profile_read(reset=True)
    _lib.profile_enable(True)
    try:
        out = F.na1d_varlen(*leaves, lens, kernel_size=5)
        out.backward(do)
        torch.cuda.synchronize()
    finally:
        _lib.profile_enable(False)
    stats = _lib.profile_read(reset=True)
    assert {n: c[0] for n, c in stats.items()} == {"na_varlen_forward": 1, "na_varlen_bwd_dq": 1,
                                                   "na_varlen_bwd_dkdv": 1}
