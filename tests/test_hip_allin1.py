"""extras/allin1 on the 'hip' backend (natten_hip_rpb_*) against the CPU
oracle (oracle/allin1.py): QK+RPB logits, AV, and the gradients of q, k,
rpb, attn and v, for 1-D and 2-D, odd and even kernels, with and without
dilation and bias.

Tolerances: fp32 1e-5 (logits, outputs, dq, dk, dattn, dv), 1e-4 for the
bias gradient (a sum over every query of the batch); bf16 logits/outputs
the half-precision bound of tests/_parity.py against the oracle in fp32 on
the same rounded inputs.

Odd kernels at head dims 32/64/128 in 16-bit run the products on the split
MFMA tile kernels (the shifted window equals the main window there, the
logits kernel adding the bias as it stores) and the bias gradient through
the two-pass reduction;
test_rpb_tile_path checks the launched kernels by name.
"""
from __future__ import annotations

import pytest
import torch

from _parity import assert_parity

import oracle.allin1 as A

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0") if torch.cuda.is_available() else None


def _rand(shape, seed, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g, dtype=torch.float32).to(dtype)


CASES_1D = [(2, 24, 3, 16, 5, 1), (1, 33, 2, 32, 7, 3), (2, 9, 2, 8, 2, 2), (1, 20, 4, 16, 4, 2), (2, 12, 2, 8, 3, 4)]
CASES_2D = [(2, 10, 12, 2, 16, 3, 1), (1, 14, 11, 3, 32, 5, 2), (1, 9, 9, 2, 8, 4, 2), (1, 7, 8, 2, 16, 7, 1)]


@pytest.mark.parametrize("with_rpb", [True, False])
@pytest.mark.parametrize("case", CASES_1D, ids=lambda c: "B{}L{}H{}D{}K{}d{}".format(*c))
def test_rpb_1d_forward_backward(case, with_rpb):
    from natten_mps_amd.extras.allin1 import na1d_av_fused, na1d_qk_rpb

    B, L, H, D, K, d = case
    q, k, v, go = (_rand((B, L, H, D), s) for s in (1, 2, 3, 4))
    rpb = _rand((H, 2 * K - 1), 5) if with_rpb else None
    ga = _rand((B, L, H, K), 6)
    # logits and their gradients
    leaves = [t.to(DEV).requires_grad_(True) for t in (q, k)]
    r_dev = rpb.to(DEV).requires_grad_(True) if with_rpb else None
    logits = na1d_qk_rpb(leaves[0], leaves[1], r_dev, K, d, scale=0.25)
    ref_leaves = [t.double().requires_grad_(True) for t in (q, k)]
    r_ref = rpb.double().requires_grad_(True) if with_rpb else None
    ref = A.na1d_qk_rpb(ref_leaves[0], ref_leaves[1], r_ref, K, d, scale=0.25)
    torch.testing.assert_close(logits.cpu().double(), ref, atol=1e-5, rtol=1e-5)
    fin = torch.isfinite(ref)
    ga_masked = torch.where(fin, ga.double(), torch.zeros((), dtype=torch.float64))
    (logits * ga_masked.float().to(DEV)).masked_fill(~fin.to(DEV), 0).sum().backward()
    (ref.masked_fill(~fin, 0) * ga_masked).sum().backward()
    for name, a, b in (("q", leaves[0], ref_leaves[0]), ("k", leaves[1], ref_leaves[1])):
        torch.testing.assert_close(a.grad.cpu().double(), b.grad, atol=1e-5, rtol=1e-5, msg=lambda m: f"d{name}: {m}")
    if with_rpb:
        torch.testing.assert_close(r_dev.grad.cpu().double(), r_ref.grad, atol=1e-4, rtol=1e-4)
    # AV and its gradients
    attn = ref.detach().float().softmax(-1)
    a_dev, v_dev = attn.to(DEV).requires_grad_(True), v.to(DEV).requires_grad_(True)
    out = na1d_av_fused(a_dev, v_dev, K, d)
    a_ref, v_ref = attn.double().requires_grad_(True), v.double().requires_grad_(True)
    out_ref = A.av_1d(a_ref, v_ref, K, d)
    torch.testing.assert_close(out.cpu().double(), out_ref, atol=1e-5, rtol=1e-5)
    out.backward(go.to(DEV))
    out_ref.backward(go.double())
    torch.testing.assert_close(a_dev.grad.cpu().double(), a_ref.grad, atol=1e-5, rtol=1e-5)
    torch.testing.assert_close(v_dev.grad.cpu().double(), v_ref.grad, atol=1e-5, rtol=1e-5)


@pytest.mark.parametrize("case", CASES_2D, ids=lambda c: "B{}X{}Y{}H{}D{}K{}d{}".format(*c))
def test_rpb_2d_forward_backward(case):
    from natten_mps_amd.extras.allin1 import na2d_av_fused, na2d_qk_rpb

    B, X, Y, H, D, K, d = case
    q, k, v, go = (_rand((B, X, Y, H, D), s) for s in (7, 8, 9, 10))
    rpb = _rand((H, 2 * K - 1, 2 * K - 1), 11)
    ga = _rand((B, X, Y, H, K * K), 12)
    leaves = [t.to(DEV).requires_grad_(True) for t in (q, k, rpb)]
    logits = na2d_qk_rpb(leaves[0], leaves[1], leaves[2], K, d)
    ref_leaves = [t.double().requires_grad_(True) for t in (q, k, rpb)]
    ref = A.na2d_qk_rpb(*ref_leaves, K, d)
    torch.testing.assert_close(logits.cpu().double(), ref, atol=1e-5, rtol=1e-5)
    fin = torch.isfinite(ref)
    ga_masked = torch.where(fin, ga.double(), torch.zeros((), dtype=torch.float64))
    (logits * ga_masked.float().to(DEV)).masked_fill(~fin.to(DEV), 0).sum().backward()
    (ref.masked_fill(~fin, 0) * ga_masked).sum().backward()
    for name, a, b, tol in (("q", leaves[0], ref_leaves[0], 1e-5), ("k", leaves[1], ref_leaves[1], 1e-5),
                            ("rpb", leaves[2], ref_leaves[2], 1e-4)):
        torch.testing.assert_close(a.grad.cpu().double(), b.grad, atol=tol, rtol=tol, msg=lambda m: f"d{name}: {m}")
    attn = ref.detach().float().softmax(-1)
    a_dev, v_dev = attn.to(DEV).requires_grad_(True), v.to(DEV).requires_grad_(True)
    out = na2d_av_fused(a_dev, v_dev, K, d)
    a_ref, v_ref = attn.double().requires_grad_(True), v.double().requires_grad_(True)
    out_ref = A.av_2d(a_ref, v_ref, K, d)
    torch.testing.assert_close(out.cpu().double(), out_ref, atol=1e-5, rtol=1e-5)
    out.backward(go.to(DEV))
    out_ref.backward(go.double())
    torch.testing.assert_close(a_dev.grad.cpu().double(), a_ref.grad, atol=1e-5, rtol=1e-5)
    torch.testing.assert_close(v_dev.grad.cpu().double(), v_ref.grad, atol=1e-5, rtol=1e-5)


def test_rpb_bias_gradient_counts_masked_entries():
    """The bias enters every logit, masked or not, so its gradient sums the
    upstream gradient over every entry (even kernel, dilation: some masked)."""
    from natten_mps_amd.extras.allin1 import na1d_qk_rpb

    B, L, H, D, K, d = 1, 5, 1, 4, 2, 2
    q, k = _rand((B, L, H, D), 13), _rand((B, L, H, D), 14)
    rpb = torch.zeros(H, 2 * K - 1, device=DEV, requires_grad=True)
    logits = na1d_qk_rpb(q.to(DEV), k.to(DEV), rpb, K, d)
    assert torch.isinf(logits).any()
    logits.backward(torch.ones_like(logits))
    r = rpb.detach().clone().cpu().double().requires_grad_(True)
    A.na1d_qk_rpb(q.double(), k.double(), r, K, d).backward(torch.ones(B, L, H, K, dtype=torch.float64))
    torch.testing.assert_close(rpb.grad.cpu().double(), r.grad, atol=0, rtol=0)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_rpb_half_precision(dtype):
    from natten_mps_amd.extras.allin1 import na2d_av_fused, na2d_qk_rpb

    q, k, v = (_rand((2, 12, 12, 2, 32), s, dtype) for s in (15, 16, 17))
    rpb = _rand((2, 9, 9), 18, dtype)
    logits = na2d_qk_rpb(q.to(DEV), k.to(DEV), rpb.to(DEV), 5, 2, scale=32 ** -0.5)
    ref = A.na2d_qk_rpb(q.float(), k.float(), rpb.float(), 5, 2, scale=32 ** -0.5)
    assert_parity(logits.cpu(), ref, dtype, "rpb logits")
    attn = ref.softmax(-1)
    out = na2d_av_fused(attn.to(dtype).to(DEV), v.to(DEV), 5, 2)
    assert_parity(out.cpu(), A.av_2d(attn.to(dtype).float(), v.float(), 5, 2), dtype, "rpb av")


def test_rpb_validation():
    from natten_mps_amd.extras.allin1 import na1d_qk_rpb, na2d_qk_rpb
    from natten_mps_amd.extras.allin1.functional import natten2dqkrpb

    q = torch.randn(1, 6, 2, 4, device=DEV)
    with pytest.raises(ValueError, match="kernel_size \\* dilation must be <= axis length"):
        na1d_qk_rpb(q, q, None, 4, 2)
    with pytest.raises(ValueError, match="4D"):
        na1d_qk_rpb(q[0], q[0], None, 3)
    q2 = torch.randn(1, 8, 8, 2, 4, device=DEV)
    with pytest.raises(ValueError, match="square kernels"):
        natten2dqkrpb(q2, q2, None, (3, 5), 1)
    with pytest.raises(ValueError, match="rpb must have shape"):
        na2d_qk_rpb(q2, q2, torch.zeros(2, 5, device=DEV), 3)


TILE_CASES = [
    (1, (96,), 2, 32, 7, 1),
    (1, (128,), 2, 64, 5, 3),
    (2, (20, 18), 2, 32, 7, 1),
    (2, (24, 24), 3, 64, 5, 2),
    (2, (16, 16), 2, 128, 3, 1),
]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("case", TILE_CASES, ids=lambda c: "r{}sp{}H{}D{}K{}d{}".format(*c))
def test_rpb_tile_path(case, dtype):
    """QK+RPB, AV and all five gradients on the tile path against the oracle."""
    import natten_mps_amd.extras.allin1 as X
    from natten_mps_amd._core import _lib

    rank, sp, H, D, K, d = case
    qk, av = getattr(X, f"na{rank}d_qk_rpb"), getattr(X, f"na{rank}d_av_fused")
    ref_qk, ref_av = getattr(A, f"na{rank}d_qk_rpb"), getattr(A, f"av_{rank}d")
    kv = K ** rank
    q, k, v = (_rand((2, *sp, H, D), s, dtype) for s in (21, 22, 23))
    rpb = _rand((H, *([2 * K - 1] * rank)), 24, dtype)
    ga = _rand((2, *sp, H, kv), 25, dtype)
    go = _rand((2, *sp, H, D), 26, dtype)
    scale = D ** -0.5
    _lib.profile_read(reset=True)
    _lib.profile_enable(True)
    try:
        leaves = [t.to(DEV).requires_grad_(True) for t in (q, k, rpb)]
        logits = qk(leaves[0], leaves[1], leaves[2], K, d, scale=scale)
        refs = [t.float().requires_grad_(True) for t in (q, k, rpb)]
        ref = ref_qk(refs[0], refs[1], refs[2], K, d, scale=scale)
        assert torch.isfinite(ref).all()
        assert_parity(logits, ref, dtype, "rpb logits")
        logits.backward(ga.to(DEV))
        ref.backward(ga.float())
        for name, a, b in zip(("dq", "dk", "drpb"), leaves, refs):
            assert_parity(a.grad, b.grad, dtype, name)
        attn = ref.detach().softmax(-1).to(dtype)
        a_dev, v_dev = attn.to(DEV).requires_grad_(True), v.to(DEV).requires_grad_(True)
        out = av(a_dev, v_dev, K, d)
        a_ref, v_ref = attn.float().requires_grad_(True), v.float().requires_grad_(True)
        out_ref = ref_av(a_ref, v_ref, K, d)
        assert_parity(out, out_ref, dtype, "rpb av")
        out.backward(go.to(DEV))
        out_ref.backward(go.float())
        assert_parity(a_dev.grad, a_ref.grad, dtype, "dattn")
        assert_parity(v_dev.grad, v_ref.grad, dtype, "dv")
        torch.cuda.synchronize()
    finally:
        _lib.profile_enable(False)
    ran = _lib.profile_read(reset=True)
    for name in ("na_rpb_qk_mfma", "na_rpb_dq_mfma", "na_rpb_dk_mfma", "na_rpb_dbias_part",
                 "na_rpb_dbias_sum", "na_rpb_av_mfma", "na_rpb_dattn_mfma", "na_rpb_dv_mfma"):
        alt = name.replace("_mfma", "_lean")  # key side on the 8x8 key tiles where those apply
        assert ran.get(name, (0,))[0] + ran.get(alt, (0,))[0] >= 1, (name, sorted(ran))
    for name in ("na_rpb_qk", "na_rpb_dq", "na_rpb_dk", "na_rpb_dbias", "na_rpb_av", "na_rpb_dattn", "na_rpb_dv"):
        assert name not in ran, (name, sorted(ran))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_rpb_bias_gradient_is_deterministic(dtype):
    """The two-pass bias gradient sums in a fixed order: repeated backward
    calls give the same bits (2-D, odd kernel, many chunks per workgroup)."""
    from natten_mps_amd._core import hip

    q, k = (_rand((4, 40, 44, 3, 32), s, dtype).to(DEV) for s in (31, 32))
    da = _rand((4, 40, 44, 3, 49), 33, dtype).to(DEV)
    runs = [hip.rpb_qk_backward(2, da, q, k, True, (7, 7), (2, 2))[2] for _ in range(3)]
    for r in runs[1:]:
        assert torch.equal(r, runs[0])
    r = torch.zeros(3, 13, 13, dtype=torch.float64, requires_grad=True)
    A.na2d_qk_rpb(q.cpu().double(), k.cpu().double(), r, 7, 2).backward(da.cpu().double())
    if dtype == torch.float32:
        torch.testing.assert_close(runs[0].cpu().double(), r.grad, atol=1e-4, rtol=1e-4)
    else:
        assert_parity(runs[0], r.grad, dtype, "drpb")


@pytest.mark.parametrize("rank", [1, 2])
def test_rpb_without_bias_equals_split_qk(rank):
    """Odd kernel, no bias: the QK+RPB logits are the split QK op's logits at
    scale 1, bit for bit (the same tile kernel and window); with a bias, each
    logit is the rounded product plus its table entry (the oracle's gather),
    rounded once more."""
    from natten_mps_amd import functional as F
    from natten_mps_amd.extras.allin1.functional import natten1dqkrpb, natten2dqkrpb

    sp, K, d = ((80,), 7, 2) if rank == 1 else ((18, 20), 5, 2)
    q, k = (_rand((2, *sp, 2, 32), s, torch.bfloat16).to(DEV) for s in (41, 42))
    qkrpb = natten1dqkrpb if rank == 1 else natten2dqkrpb
    plain = getattr(F, f"na{rank}d_qk")(q, k, (K,) * rank, (d,) * rank, scale=1.0)
    assert torch.equal(qkrpb(q, k, None, K, d), plain)
    rpb = _rand((2, *([2 * K - 1] * rank)), 43, torch.bfloat16)
    got = qkrpb(q, k, rpb.to(DEV), K, d).cpu().float()
    z = torch.zeros((2, *sp, 2, 1), dtype=torch.float64)
    gathered = (A.na1d_qk_rpb if rank == 1 else A.na2d_qk_rpb)(z, z, rpb.double(), K, d)  # q . k = 0
    want = (plain.cpu().float() + gathered.float()).to(torch.bfloat16).float()
    assert torch.equal(got, want)


def test_rpb_tile_path_on_qkv_views():
    """q, k, v as views into one projected qkv tensor ([B, X, Y, 3, H, D], the
    DiNAT block's layout): the tile path reads them through their strides."""
    import natten_mps_amd.extras.allin1 as X
    from natten_mps_amd._core import _lib

    B, Xn, Yn, H, D, K, d = 2, 16, 18, 2, 32, 5, 2
    qkv = _rand((B, Xn, Yn, 3, H, D), 51, torch.bfloat16)
    rpb = _rand((H, 2 * K - 1, 2 * K - 1), 52, torch.bfloat16)
    go = _rand((B, Xn, Yn, H, D), 53, torch.bfloat16)
    qkv_d = qkv.to(DEV).requires_grad_(True)
    q, k, v = qkv_d.unbind(3)
    _lib.profile_read(reset=True)
    _lib.profile_enable(True)
    try:
        attn = X.na2d_qk_rpb(q, k, rpb.to(DEV), K, d, scale=D ** -0.5).softmax(-1)
        out = X.na2d_av_fused(attn, v, K, d)
        out.backward(go.to(DEV))
        torch.cuda.synchronize()
    finally:
        _lib.profile_enable(False)
    ran = _lib.profile_read(reset=True)
    for name in ("na_rpb_qk_mfma", "na_rpb_av_mfma", "na_rpb_dq_mfma", "na_rpb_dk_mfma", "na_rpb_dattn_mfma",
                 "na_rpb_dv_mfma"):
        alt = name.replace("_mfma", "_lean")  # key side on the 8x8 key tiles where those apply
        assert ran.get(name, (0,))[0] + ran.get(alt, (0,))[0] >= 1, (name, sorted(ran))
    ref_qkv = qkv.float().requires_grad_(True)
    rq, rk, rv = ref_qkv.unbind(3)
    ref_attn = A.na2d_qk_rpb(rq, rk, rpb.float(), K, d, scale=D ** -0.5).softmax(-1)
    ref_out = A.av_2d(ref_attn, rv, K, d)
    ref_out.backward(go.float())
    assert_parity(out, ref_out, torch.bfloat16, "out")
    assert_parity(qkv_d.grad, ref_qkv.grad, torch.bfloat16, "dqkv")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_rpb_bias_gradient_workspace_entry_points(dtype):
    """natten_hip_rpb_qk_backward (no workspace: the one-pass bias gradient)
    and natten_hip_rpb_qk_backward_ws (the caller's workspace of
    natten_hip_rpb_dbias_workspace floats: two passes) give the same dq and
    dk bits and bias gradients within the bound of the dtype, both against
    the oracle in float64; a workspace one float short takes the one pass."""
    import ctypes

    from natten_mps_amd._core import _lib, hip

    q, k = (_rand((2, 24, 20, 2, 32), s, dtype).to(DEV) for s in (41, 42))
    da = _rand((2, 24, 20, 2, 25), 43, dtype).to(DEV)
    prob = hip._rpb_problem(2, q, 2, 32, 32, (5, 5), (2, 2))
    lib = _lib.load()
    need = int(lib.natten_hip_rpb_dbias_workspace(ctypes.byref(prob)))
    assert need > 0, need
    L = lambda t: ctypes.byref(_lib.layout(t, 2, 1))  # noqa: E731

    def run(work, nfloat):
        dq, dk = torch.empty_like(q), torch.empty_like(k)
        drpb = torch.empty((2, 9, 9), dtype=dtype, device=DEV)
        _lib.profile_enable(True)
        try:
            rc = lib.natten_hip_rpb_qk_backward_ws(
                ctypes.byref(prob), _lib.ptr(da), L(da), _lib.ptr(q), L(q), _lib.ptr(k), L(k), _lib.ptr(dq), L(dq),
                _lib.ptr(dk), L(dk), _lib.ptr(drpb), _lib.ptr(work), nfloat, _lib.stream_of(q))
            _lib.check(rc, "rpb_qk_backward_ws")
            torch.cuda.synchronize()
        finally:
            _lib.profile_enable(False)
        return dq, dk, drpb, _lib.profile_read(reset=True)

    work = torch.empty(need, dtype=torch.float32, device=DEV)
    two = run(work, need)
    short = run(work, need - 1)
    none = run(None, 0)
    assert "na_rpb_dbias_part" in two[3] and "na_rpb_dbias" not in two[3], sorted(two[3])
    for r in (short, none):
        assert "na_rpb_dbias" in r[3] and "na_rpb_dbias_part" not in r[3], sorted(r[3])
        assert torch.equal(r[0], two[0]) and torch.equal(r[1], two[1])
        assert torch.equal(r[2], none[2])
    rg = torch.zeros(2, 9, 9, dtype=torch.float64, requires_grad=True)
    A.na2d_qk_rpb(q.cpu().double(), k.cpu().double(), rg, 5, 2).backward(da.cpu().double())
    for r in (two, none):
        if dtype == torch.float32:
            torch.testing.assert_close(r[2].cpu().double(), rg.grad, atol=1e-4, rtol=1e-4)
        else:
            assert_parity(r[2], rg.grad, dtype, "drpb")


def _allin1_golden():
    import json
    import os

    import numpy as np

    here = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
    with open(os.path.join(here, "allin1.json")) as f:
        meta = json.load(f)
    return meta["cases"], np.load(os.path.join(here, "allin1.npz"))


_GOLDEN_CASES, _GOLDEN_ARRAYS = _allin1_golden()


@pytest.mark.parametrize("case", _GOLDEN_CASES, ids=lambda c: c["key"].rstrip("/"))
def test_rpb_matches_reference_fixtures(case):
    """The reference's own extras/allin1 outputs (tests/golden/allin1.npz,
    from its pure torch path: odd and even kernels, dilation 1 and > 1, 1-D
    and 2-D, with and without a bias) replayed through this package's
    extras.allin1 on the GPU in fp32: logits, dq, dk, out, dattn, dv within
    1e-5, the bias gradient (a sum over every logit of the batch) within
    1e-4.  The upstream logit gradient is the fixture's, masked entries
    included: they reach the bias gradient only."""
    from natten_mps_amd.extras import allin1 as M

    a = {n.split("/")[-1]: torch.from_numpy(_GOLDEN_ARRAYS[n]) for n in case["arrays"]}
    rank, K, d, scale = case["rank"], case["kernel_size"], case["dilation"], case["scale"]
    qk = M.na1d_qk_rpb if rank == 1 else M.na2d_qk_rpb
    av = M.na1d_av_fused if rank == 1 else M.na2d_av_fused
    q, k = (a[n].to(DEV).requires_grad_(True) for n in ("q", "k"))
    r = a["rpb"].to(DEV).requires_grad_(True) if case["with_rpb"] else None
    logits = qk(q, k, r, K, d, scale=scale)
    torch.testing.assert_close(logits.detach().cpu(), a["logits"], atol=1e-5, rtol=1e-5)
    grads = torch.autograd.grad(logits, [q, k] + ([r] if r is not None else []), a["dlogits"].to(DEV))
    torch.testing.assert_close(grads[0].cpu(), a["dq"], atol=1e-5, rtol=1e-5, msg=lambda m: f"dq: {m}")
    torch.testing.assert_close(grads[1].cpu(), a["dk"], atol=1e-5, rtol=1e-5, msg=lambda m: f"dk: {m}")
    if r is not None:
        torch.testing.assert_close(grads[2].cpu(), a["drpb"], atol=1e-4, rtol=1e-4, msg=lambda m: f"drpb: {m}")
    at, v = a["attn"].to(DEV).requires_grad_(True), a["v"].to(DEV).requires_grad_(True)
    out = av(at, v, K, d)
    torch.testing.assert_close(out.detach().cpu(), a["out"], atol=1e-5, rtol=1e-5)
    da, dv = torch.autograd.grad(out, [at, v], a["dout"].to(DEV))
    torch.testing.assert_close(da.cpu(), a["dattn"], atol=1e-5, rtol=1e-5, msg=lambda m: f"dattn: {m}")
    torch.testing.assert_close(dv.cpu(), a["dv"], atol=1e-5, rtol=1e-5, msg=lambda m: f"dv: {m}")


@pytest.mark.parametrize("with_rpb", [True, False])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_rpb_ops_through_the_binding_cache(with_rpb, dtype, monkeypatch):
    """The four relative-position-bias ops run wholly in the host binding
    once their signature is registered: repeated calls succeed with the
    Python layout builder switched off and give the bits of the first calls
    and of the ctypes path (bias gradient and its workspace included)."""
    from natten_mps_amd._core import _lib, hip

    b = _lib.binding()
    assert b is not None, "the host binding _natten_torch.so is not built"
    rank, ks, dil = 2, (5, 5), (2, 1)
    q, k, v = (_rand((2, 14, 12, 2, 32), 930 + i, dtype).to(DEV) for i in range(3))
    rpb = _rand((2, 9, 9), 933, dtype).to(DEV) if with_rpb else None
    da = _rand((2, 14, 12, 2, 25), 934, dtype).to(DEV)
    do = _rand((2, 14, 12, 2, 32), 935, dtype).to(DEV)

    def calls():
        attn = hip.rpb_qk_forward(rank, q, k, rpb, ks, dil)
        out = hip.rpb_av_forward(rank, attn.softmax(-1), v, ks, dil)
        dq, dk, drpb = hip.rpb_qk_backward(rank, da, q, k, with_rpb, ks, dil)
        dattn, dv = hip.rpb_av_backward(rank, do, attn.softmax(-1), v, ks, dil)
        torch.cuda.synchronize()
        return [attn, out, dq, dk, drpb, dattn, dv]

    names = ("attn", "out", "dq", "dk", "drpb", "dattn", "dv")
    b.clear()
    first = calls()

    def no_python_path(*a, **kw):
        raise AssertionError("a registered relative-position-bias signature went through hip.py")

    monkeypatch.setattr(_lib, "layout", no_python_path)
    second = calls()
    monkeypatch.undo()
    monkeypatch.setattr(_lib, "_bind", None)
    third = calls()
    monkeypatch.undo()
    for name, x, y, z in zip(names, first, second, third):
        if x is None:
            assert y is None and z is None, name
            continue
        assert torch.equal(x, y), f"{name}: binding cache differs from the first call"
        assert torch.equal(x, z), f"{name}: binding differs from the ctypes path"
