"""Edge cases of the 'hip' backend on the GPU: non-finite inputs outside a
window, operand extents the tile kernels must refuse, head dims of V that
differ from Q/K, the LDS audit of the tile kernels, and bitwise determinism
of the gathers.  Values are checked against the CPU oracle under the bounds
of tests/_parity.py.
"""
from __future__ import annotations

import ctypes

import pytest
import torch

import oracle.pure as P
from _parity import assert_parity

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0") if torch.cuda.is_available() else None


@pytest.fixture(autouse=True)
def _hip():
    import natten_mps_amd

    natten_mps_amd.set_backend("hip")


def _inputs(seed, shapes, dtype):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(s, generator=g, dtype=torch.float32).to(dtype) for s in shapes]


def _launched(run):
    """Run `run()` with the library's per-launch timing on; return the names
    of the kernels it launched."""
    from natten_mps_amd._core import _lib

    _lib.profile_read(reset=True)
    _lib.profile_enable(True)
    try:
        res = run()
        torch.cuda.synchronize()
    finally:
        _lib.profile_enable(False)
    return res, set(_lib.profile_read(reset=True))


# ---------------------------------------------------------------------------
# the tile kernels' constant LDS base
# ---------------------------------------------------------------------------


def test_mfma_kernels_have_no_static_lds():
    """Every tile-kernel instance (2 dtypes x 3 head dims x 24 fused (4
    layout groups), 4 global-key, 6 variable-length and 16 split instances
    (6 of them single-step, 4 with the relative-position bias), 2 dtypes x
    34 fused, global-key and variable-length instances at head dim 96, and
    2 dtypes x 4 head dims x 9 single-step (FLAT) fused instances, the lean
    2-D kernels: 2 dtypes x 2 head dims x 5 chunk counts x forward, dQ,
    dK/dV and the split key side, their 1-D forward, dQ and dK/dV, and the
    forward and dQ with two q heads per workgroup (2-D and 1-D), and
    fp32 x 2 head dims x 5 chunk counts x forward, dQ and dK/dV for 2-D, 1-D
    and 3-D (depth-walking) problems, and
    2 dtypes x 4 head dims x 11 dQ instances that
    take delta from P dP) reports 0 bytes of static LDS, so the operands the kernels
    stage at a constant LDS offset cannot overlap a __shared__ array; with
    one that did, the library would refuse the tile path."""
    from natten_mps_amd._core import _lib

    n = ctypes.c_int32(0)
    assert _lib.load().natten_hip_mfma_lds_check(ctypes.byref(n)) == 1
    assert n.value == 2 * 3 * (24 + 4 + 6 + 16) + 2 * (24 + 4 + 6) + 2 * 4 * 9 + 2 * 2 * 5 * 11 + 2 * 5 * 9 + 2 * 4 * 11


# ---------------------------------------------------------------------------
# extents the tile kernels must not take
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_split_av_with_attn_shorter_than_value(dtype):
    """na2d_av at stride 1 with attn covering fewer query positions than
    value has (attn[:, :10, :12] of a 14 x 15 problem; allowed by the
    reference, _core/pure.py:278-281): forward and backward match the oracle
    and run on the vector kernels, which decode over the attn extent."""
    from natten_mps_amd import functional as F

    (v,) = _inputs(301, [(2, 14, 15, 2, 32)], dtype)
    (logits,) = _inputs(302, [(2, 10, 12, 2, 49)], torch.float32)
    attn = torch.softmax(logits, -1).to(dtype)
    (do,) = _inputs(303, [(2, 10, 12, 2, 32)], dtype)

    ad, vd = attn.to(DEV).requires_grad_(True), v.to(DEV).requires_grad_(True)

    def run():
        out = F.na2d_av(ad, vd, 7, 1)
        out.backward(do.to(DEV))
        return out

    out, ran = _launched(run)
    assert {"na_av", "na_av_bwd_a", "na_av_bwd_v"} <= ran and not any(n.endswith("_mfma") for n in ran), ran
    ra, rv = attn.float().requires_grad_(True), v.float().requires_grad_(True)
    ref = P.na2d_av_forward(ra, rv, (7, 7), (1, 1), (1, 1), (False, False))
    ref.backward(do.float())
    assert_parity(out, ref, dtype, "out")
    assert_parity(ad.grad, ra.grad, dtype, "dattn")
    assert_parity(vd.grad, rv.grad, dtype, "dv")


def test_split_rows_past_the_31bit_byte_range_use_vector_kernels():
    """Logits of one (batch, head) of a 1024 x 1024, 8-head, 13 x 13 problem
    span 1.4e9 entries: their byte offsets exceed the 31-bit range of the
    tile kernels' row buffers, so na2d_qk runs on the vector kernel.  Values
    at an interior and a corner query against the window rule computed
    directly."""
    from natten_mps_amd import functional as F

    g = torch.Generator(device=DEV).manual_seed(304)
    q = torch.randn((1, 1024, 1024, 8, 32), generator=g, device=DEV).to(torch.bfloat16)
    k = torch.randn((1, 1024, 1024, 8, 32), generator=g, device=DEV).to(torch.bfloat16)
    logits, ran = _launched(lambda: F.na2d_qk(q, k, 13, 1))
    assert "na_qk" in ran and "na_qk_mfma" not in ran, ran
    for (y, x, h) in ((600, 700, 5), (0, 0, 2), (1023, 1017, 7)):
        y0 = min(max(y - 6, 0), 1024 - 13)
        x0 = min(max(x - 6, 0), 1024 - 13)
        win = k[0, y0:y0 + 13, x0:x0 + 13, h].float().reshape(169, 32)
        ref = win @ q[0, y, x, h].float()
        assert_parity(logits[0, y, x, h], ref, torch.bfloat16, f"logits at {(y, x, h)}")
    del logits, q, k
    torch.cuda.empty_cache()


# ---------------------------------------------------------------------------
# non-finite values outside a window stay outside it
# ---------------------------------------------------------------------------

NONFINITE_FUSED = [
    # rank, spatial, hq, hkv, dim, kernel, dilation, bad position, dtype
    (2, (20, 22), 2, 2, 32, (7, 7), (1, 1), (9, 10), torch.bfloat16),
    (2, (24, 24), 4, 2, 64, (5, 5), (2, 2), (11, 12), torch.float16),
    (3, (6, 12, 12), 2, 2, 32, (3, 5, 5), (1, 1, 2), (3, 6, 5), torch.bfloat16),
    (1, (200,), 4, 1, 64, (9,), (2,), (100,), torch.bfloat16),
    # fp32 on the 2-D tile kernels
    (2, (20, 22), 2, 2, 32, (7, 7), (1, 1), (9, 10), torch.float32),
    (2, (18, 20), 2, 2, 64, (5, 3), (1, 2), (8, 9), torch.float32),
]


@pytest.mark.parametrize("value", [float("inf"), float("nan")], ids=["inf", "nan"])
@pytest.mark.parametrize("which", ["q", "k", "v"])
@pytest.mark.parametrize("case", NONFINITE_FUSED, ids=lambda c: f"{c[0]}d-{c[4]}-{str(c[8])[6:]}")
def test_fused_nonfinite_stays_local(case, which, value):
    """One position of q, k or v (batch 0, every head) set to Inf or NaN.
    The tile kernels stage that row for neighbouring queries whose windows
    exclude it; their outputs and gradients must stay finite and equal the
    oracle's, and exactly the elements the oracle makes non-finite are
    non-finite."""
    from natten_mps_amd import functional as F

    rank, sp, hq, hkv, dim, ks, dil, bad, dtype = case
    q, k, v, do = _inputs(311, [(2, *sp, hq, dim), (2, *sp, hkv, dim), (2, *sp, hkv, dim), (2, *sp, hq, dim)],
                          dtype)
    t = {"q": q, "k": k, "v": v}[which]
    t[(0, *bad)] = value
    leaves = [x.to(DEV).requires_grad_(True) for x in (q, k, v)]
    out = getattr(F, f"na{rank}d")(*leaves, kernel_size=ks, dilation=dil)
    out.backward(do.to(DEV))
    rl = [x.float().requires_grad_(True) for x in (q, k, v)]
    ref = P.forward(rank, *rl, ks, (1,) * rank, dil, (False,) * rank, None)
    ref.backward(do.float())
    finite = torch.isfinite(ref)
    assert finite.any() and not finite.all()  # the case reaches some queries and not others
    assert_parity(out, ref, dtype, "out")
    for name, a, b in zip(("dq", "dk", "dv"), leaves, rl):
        assert_parity(a.grad, b.grad, dtype, name)


@pytest.mark.parametrize("which", ["q", "k"])
def test_split_qk_nonfinite_stays_local(which):
    """Split QK forward and backward (tile kernels) with an Inf row in q or
    k: logits, dq and dk against the oracle, finiteness included."""
    from natten_mps_amd import functional as F

    q, k = _inputs(321, [(2, 18, 20, 2, 32)] * 2, torch.bfloat16)
    {"q": q, "k": k}[which][0, 9, 9] = float("inf")
    qd, kd = q.to(DEV).requires_grad_(True), k.to(DEV).requires_grad_(True)
    logits, ran = _launched(lambda: F.na2d_qk(qd, kd, 5, (1, 2), scale=0.25))
    rq, rk = q.float().requires_grad_(True), k.float().requires_grad_(True)
    ref = P.na2d_qk_forward(rq, rk, (5, 5), (1, 2), (1, 1), (False, False), 0.25)
    assert_parity(logits, ref, torch.bfloat16, "logits")
    (dl,) = _inputs(322, [tuple(ref.shape)], torch.bfloat16)
    _, ran_b = _launched(lambda: logits.backward(dl.to(DEV)))
    assert {"na_qk_mfma", "na_qk_bwd_q_mfma"} <= ran | ran_b and {"na_qk_bwd_k_mfma", "na_qk_bwd_k_lean"} & ran_b
    ref.backward(dl.float())
    assert not torch.isfinite(rq.grad).all() or not torch.isfinite(rk.grad).all()
    assert_parity(qd.grad, rq.grad, torch.bfloat16, "dq")
    assert_parity(kd.grad, rk.grad, torch.bfloat16, "dk")


def test_split_av_nonfinite_stays_local():
    """Split AV forward and backward (tile kernels) with a NaN row in v."""
    from natten_mps_amd import functional as F

    (v,) = _inputs(331, [(2, 18, 20, 2, 32)], torch.bfloat16)
    v[1, 4, 15] = float("nan")
    (lg,) = _inputs(332, [(2, 18, 20, 2, 25)], torch.float32)
    attn = torch.softmax(lg, -1).to(torch.bfloat16)
    ad, vd = attn.to(DEV).requires_grad_(True), v.to(DEV).requires_grad_(True)
    (do,) = _inputs(333, [(2, 18, 20, 2, 32)], torch.bfloat16)

    def run():
        out = F.na2d_av(ad, vd, 5, (2, 1))
        out.backward(do.to(DEV))
        return out

    out, ran = _launched(run)
    assert {"na_av_mfma", "na_av_bwd_a_mfma"} <= ran and {"na_av_bwd_v_mfma", "na_av_bwd_v_lean"} & ran, ran
    ra, rv = attn.float().requires_grad_(True), v.float().requires_grad_(True)
    ref = P.na2d_av_forward(ra, rv, (5, 5), (2, 1), (1, 1), (False, False))
    ref.backward(do.float())
    assert torch.isfinite(ref).any() and not torch.isfinite(ref).all()
    assert_parity(out, ref, torch.bfloat16, "out")
    assert_parity(ad.grad, ra.grad, torch.bfloat16, "dattn")
    assert_parity(vd.grad, rv.grad, torch.bfloat16, "dv")


# ---------------------------------------------------------------------------
# V with its own head dim (functional.py:56-63 of the reference: NAF-style
# cross attention, D = 64 for q/k and 256 for v)
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rank", [1, 2, 3])
def test_dim_v_differs_forward_and_gradients(rank, dtype):
    from natten_mps_amd import functional as F

    sp, ks, dil = {1: ((40,), 7, 2), 2: ((12, 14), (5, 3), (1, 2)), 3: ((6, 7, 9), (3, 3, 5), (1, 2, 1))}[rank]
    q, k, v, do = _inputs(341, [(2, *sp, 2, 64), (2, *sp, 2, 64), (2, *sp, 2, 256), (2, *sp, 2, 256)], dtype)
    leaves = [x.to(DEV).requires_grad_(True) for x in (q, k, v)]
    out = getattr(F, f"na{rank}d")(*leaves, kernel_size=ks, dilation=dil)
    out.backward(do.to(DEV))
    assert out.shape == (2, *sp, 2, 256)
    kst = (ks,) * rank if isinstance(ks, int) else ks
    dlt = (dil,) * rank if isinstance(dil, int) else dil
    # the reference reaches V with its own head dim through its split
    # composition (its pure fused op requires identical shapes)
    rl = [x.float().requires_grad_(True) for x in (q, k, v)]
    nc = (False,) * rank
    logits = getattr(P, f"na{rank}d_qk_forward")(rl[0], rl[1], kst, dlt, (1,) * rank, nc, None) * 64 ** -0.5
    ref = getattr(P, f"na{rank}d_av_forward")(torch.softmax(logits, -1), rl[2], kst, dlt, (1,) * rank, nc)
    ref.backward(do.float())
    assert_parity(out, ref, dtype, "out")
    for name, a, b in zip(("dq", "dk", "dv"), leaves, rl):
        assert_parity(a.grad, b.grad, dtype, name)


# ---------------------------------------------------------------------------
# bitwise determinism of the gathers (no atomics anywhere)
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("dil", [1, 8])
def test_config3_backward_is_bitwise_deterministic(dil):
    """Config 3 (B=16, 56 x 56, 4 heads, D=32, K=7, bf16) forward and
    backward repeated: whole tensors equal bit for bit."""
    from natten_mps_amd import functional as F

    g = torch.Generator().manual_seed(1003)
    q, k, v, do = (torch.randn((16, 56, 56, 4, 32), generator=g).to(torch.bfloat16).to(DEV) for _ in range(4))
    leaves = [t.requires_grad_(True) for t in (q, k, v)]

    def step():
        out = F.na2d(*leaves, kernel_size=7, dilation=dil)
        return [out.detach()] + list(torch.autograd.grad(out, leaves, do))

    ref = step()
    for _ in range(4):
        for name, a, b in zip(("out", "dq", "dk", "dv"), step(), ref):
            assert torch.equal(a, b), f"{name}: {int((a != b).sum())} elements differ between runs"


def test_split_key_side_multi_slice_is_bitwise_deterministic():
    """The split ops' key-side tile kernel (dk of QK, dv of AV) on a 3-D
    problem whose key tiles walk several staged axis-0 slices: repeated
    backward passes agree bit for bit."""
    from natten_mps_amd import functional as F

    q, k, v = (t.to(DEV) for t in _inputs(351, [(2, 8, 16, 16, 4, 32)] * 3, torch.bfloat16))
    (dl,) = _inputs(352, [(2, 8, 16, 16, 4, 75)], torch.bfloat16)
    (do,) = _inputs(353, [(2, 8, 16, 16, 4, 32)], torch.bfloat16)
    dl, do = dl.to(DEV), do.to(DEV)
    leaves = [t.requires_grad_(True) for t in (q, k, v)]

    def step():
        logits = F.na3d_qk(leaves[0], leaves[1], (3, 5, 5), (2, 1, 2))
        attn = torch.softmax(logits.detach().float(), -1).to(torch.bfloat16)
        out = F.na3d_av(attn, leaves[2], (3, 5, 5), (2, 1, 2))
        return list(torch.autograd.grad(logits, leaves[:2], dl)) + list(torch.autograd.grad(out, [leaves[2]], do))

    (ref, ran) = _launched(step)
    assert {"na_qk_bwd_k_mfma", "na_av_bwd_v_mfma"} <= ran, ran
    for _ in range(4):
        for name, a, b in zip(("dq", "dk", "dv"), step(), ref):
            assert torch.equal(a, b), f"{name}: {int((a != b).sum())} elements differ between runs"


# ---------------------------------------------------------------------------
# the C++ host binding of the fused calls against the ctypes path
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("case", ["lean2d", "strided3d_lse"])
def test_host_binding_matches_ctypes_path(case, monkeypatch):
    """The fused forward / backward through the C++ host binding
    (_natten_torch.so) and through ctypes give the same bits: same kernels,
    same buffers' layouts; the binding allocates dq zeroed where stride > 1
    leaves non-query positions, as the ctypes path does.  An unsupported
    problem raises NotImplementedError through the binding."""
    from natten_mps_amd._core import _lib, hip

    assert _lib.binding() is not None, "the host binding _natten_torch.so is not built"
    if case == "lean2d":
        rank, shape, ks, st, dil, causal, dtype = 2, (2, 16, 24, 2, 32), (7, 7), (1, 1), (1, 1), (False, False), \
            torch.bfloat16
        dl = None
    else:
        rank, shape, ks, st, dil, causal, dtype = 3, (1, 6, 8, 9, 2, 16), (3, 3, 3), (1, 2, 1), (1, 1, 2), \
            (True, False, False), torch.float32
        dl = True
    q, k, v = (x.to(DEV) for x in _inputs(901, [shape] * 3, dtype))

    def run():
        hip._FWD_CACHE.clear()
        hip._BWD_CACHE.clear()
        out, lse = hip.forward_with_lse(rank, q, k, v, ks, st, dil, causal, None)
        g = torch.Generator().manual_seed(3)
        dout = torch.randn(out.shape, generator=g).to(dtype).to(DEV)
        dlse = torch.randn(lse.shape, generator=g).to(DEV) if dl else None
        grads = hip.fused_backward(rank, dout, q, k, v, out, lse, ks, dil, st, causal, None, dlse)
        torch.cuda.synchronize()
        return [out, lse, *grads]

    fast = run()
    assert all(s.fast is not None for s in hip._FWD_CACHE.values())
    monkeypatch.setattr(_lib, "_bind", None)
    slow = run()
    assert all(s.fast is None for s in hip._FWD_CACHE.values())
    for name, a, b in zip(("out", "lse", "dq", "dk", "dv"), fast, slow):
        assert torch.equal(a, b), name
    monkeypatch.undo()
    hip._FWD_CACHE.clear()
    x = torch.zeros((1, 6, 1, 32), device=DEV, dtype=torch.bfloat16)
    with pytest.raises(NotImplementedError):
        hip.forward_with_lse(1, x, x, x, (6,), (1,), (1,), (False,), None)


def test_binding_signature_cache():
    """The binding's own signature cache: a signature seen once runs wholly in
    C++ afterwards (hip.py's caches stay empty) with the same bits; arguments
    it does not take (a non-unit innermost stride, non-fp32 lse, a scale given
    as an int) go through hip.py and still give the same results."""
    from natten_mps_amd._core import _lib, hip

    b = _lib.binding()
    assert b is not None, "the host binding _natten_torch.so is not built"
    rank, ks, st, dil, causal = 2, (5, 5), (1, 1), (1, 1), (False, False)
    q, k, v, do = (x.to(DEV) for x in _inputs(907, [(2, 12, 20, 2, 32)] * 4, torch.bfloat16))
    b.clear()
    hip._FWD_CACHE.clear()
    hip._BWD_CACHE.clear()
    out, lse = hip.forward_with_lse(rank, q, k, v, ks, st, dil, causal, None)
    grads = hip.fused_backward(rank, do, q, k, v, out, lse, ks, dil, st, causal, None)
    assert len(hip._FWD_CACHE) == 1 and len(hip._BWD_CACHE) == 1
    hip._FWD_CACHE.clear()
    hip._BWD_CACHE.clear()
    out2, lse2 = hip.forward_with_lse(rank, q, k, v, ks, st, dil, causal, None)
    grads2 = hip.fused_backward(rank, do, q, k, v, out2, lse2, ks, dil, st, causal, None)
    assert not hip._FWD_CACHE and not hip._BWD_CACHE, "the second call did not stay in the binding"
    for name, a, c in zip(("out", "lse", "dq", "dk", "dv"), (out, lse, *grads), (out2, lse2, *grads2)):
        assert torch.equal(a, c), name
    # arguments the binding leaves to hip.py
    wide = torch.empty((*q.shape[:-1], 64), dtype=q.dtype, device=DEV)
    wide[..., ::2] = q
    qs = wide[..., ::2]
    assert qs.stride(-1) == 2
    out3, lse3 = hip.forward_with_lse(rank, qs, k, v, ks, st, dil, causal, None)
    assert torch.equal(out3, out) and torch.equal(lse3, lse)
    grads3 = hip.fused_backward(rank, do, q, k, v, out, lse.double(), ks, dil, st, causal, None)
    for name, a, c in zip(("dq", "dk", "dv"), grads, grads3):
        assert torch.equal(a, c), name
    out4, _ = hip.forward_with_lse(rank, q, k, v, ks, st, dil, causal, 1)
    out5, _ = hip.forward_with_lse(rank, q, k, v, ks, st, dil, causal, 1.0)
    assert torch.equal(out4, out5)
    # a registered signature on another stream runs on that stream
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        out6, lse6 = hip.forward_with_lse(rank, q, k, v, ks, st, dil, causal, None)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    assert torch.equal(out6, out) and torch.equal(lse6, lse)


@pytest.mark.parametrize("stride", [(1, 1), (2, 1)])
def test_split_ops_through_the_binding_cache(stride, monkeypatch):
    """The four split ops (QK, AV, their backward) run wholly in the binding
    once their signature is registered: the repeated calls below succeed with
    hip.py's layout builder switched off, and give the bits of the first
    calls and of the ctypes path.  dq of the strided QK backward is zero off
    the query positions in both.  A d_attn of another dtype is converted by
    hip.py (never registered) and matches too."""
    from natten_mps_amd._core import _lib, hip

    b = _lib.binding()
    assert b is not None, "the host binding _natten_torch.so is not built"
    rank, ks, dil, causal = 2, (5, 5), (1, 2), (False, False)
    q, k, v = (x.to(DEV) for x in _inputs(911, [(2, 14, 18, 2, 32)] * 3, torch.bfloat16))
    out_sp = tuple((n + s_ - 1) // s_ for n, s_ in zip(q.shape[1:3], stride))
    (da, do) = (x.to(DEV) for x in _inputs(912, [(2, *out_sp, 2, 25), (2, *out_sp, 2, 32)], torch.bfloat16))

    def calls():
        attn = hip.qk_forward(rank, q, k, ks, dil, stride, causal, 0.25)
        out = hip.av_forward(rank, attn, v, ks, dil, stride, causal)
        dq, dk = hip.qk_backward(rank, da, q, k, ks, dil, stride, causal, 0.25)
        dattn, dv = hip.av_backward(rank, do, attn, v, ks, dil, stride, causal)
        torch.cuda.synchronize()
        return [attn, out, dq, dk, dattn, dv]

    names = ("attn", "out", "dq", "dk", "dattn", "dv")
    b.clear()
    first = calls()

    def no_python_path(*a, **kw):
        raise AssertionError("a registered split-op signature went through hip.py")

    monkeypatch.setattr(_lib, "layout", no_python_path)
    second = calls()
    monkeypatch.undo()
    monkeypatch.setattr(_lib, "_bind", None)
    third = calls()
    monkeypatch.undo()
    for name, a, c, d in zip(names, first, second, third):
        assert torch.equal(a, c), f"{name}: binding cache differs from the first call"
        assert torch.equal(a, d), f"{name}: binding differs from the ctypes path"
    if stride != (1, 1):
        assert not first[2][:, 1::2].any(), "dq must be zero off the strided query positions"
    dq32, dk32 = hip.qk_backward(rank, da.float(), q, k, ks, dil, stride, causal, 0.25)
    assert torch.equal(dq32, first[2]) and torch.equal(dk32, first[3])


# ---------------------------------------------------------------------------
# fp32 on the 2-D tile kernels (v_mfma_f32_16x16x4_f32)
# ---------------------------------------------------------------------------

FP32_TILE = [
    # spatial, heads, dim, kernel, dilation, causal, scale
    ((32, 32), 4, 32, (7, 7), (1, 1), (False, False), None),
    ((17, 23), 2, 32, (5, 7), (2, 3), (True, False), 0.3),
    ((20, 16), 2, 64, (3, 5), (1, 2), (False, True), None),
    ((40, 36), 1, 64, (7, 7), (2, 1), (False, True), 0.125),
    ((9, 12), 3, 32, (4, 6), (1, 1), (False, False), None),
]


@pytest.mark.parametrize("case", FP32_TILE, ids=lambda c: f"{c[0]}-D{c[2]}-K{c[3]}-d{c[4]}-c{c[5]}")
def test_fp32_on_2d_tile_kernels(case):
    """fp32 2-D problems at head dim 32 / 64 run the 2-D tile kernels with
    fp32 MFMA (forward, dQ, dK/dV launches named na_*_lean) and match the
    oracle in fp32 within 1e-5 elementwise, odd and even kernels, dilation,
    causal axes."""
    from natten_mps_amd import functional as F

    sp, heads, dim, ks, dil, causal, scale = case
    q, k, v, do = _inputs(951, [(2, *sp, heads, dim)] * 4, torch.float32)
    leaves = [x.to(DEV).requires_grad_(True) for x in (q, k, v)]

    def run():
        out = F.na2d(*leaves, kernel_size=ks, dilation=dil, is_causal=causal, scale=scale)
        out.backward(do.to(DEV))
        return out

    out, ran = _launched(run)
    assert {"na_fwd_lean", "na_bwd_q_lean", "na_bwd_kv_lean"} <= ran, ran
    rl = [x.clone().requires_grad_(True) for x in (q, k, v)]
    ref = P.forward(2, *rl, ks, (1, 1), dil, causal, scale)
    ref.backward(do)
    assert_parity(out, ref, torch.float32, "out")
    for name, a, b in zip(("dq", "dk", "dv"), leaves, rl):
        assert_parity(a.grad, b.grad, torch.float32, name)


# ---------------------------------------------------------------------------
# the split key side's weight bands: K up to 9 (bands of up to 10 chunks),
# dilation, causal windows, non-square images, and weight planes at both
# 2-byte phases (2 heads of an odd number of weights each)
# ---------------------------------------------------------------------------

SPLIT_BANDS = [
    ((9, 11), (5, 5), (1, 1), (False, False)),
    ((10, 13), (9, 9), (1, 1), (False, False)),
    ((16, 12), (7, 3), (2, 1), (True, False)),
    ((12, 11), (5, 5), (1, 2), (False, True)),
]


@pytest.mark.parametrize("case", SPLIT_BANDS)
def test_split_key_side_weight_bands(case):
    """dk of QK's backward and dv of AV's backward on the key-side tile
    kernel, whose staging keeps only the band of each weight row that meets
    the key tile, against the oracle (with dq and dattn)."""
    from natten_mps_amd import functional as F

    sp, ks, dil, causal = case
    kv = ks[0] * ks[1]
    q, k, v, do = _inputs(351, [(2, *sp, 2, 32)] * 4, torch.bfloat16)
    (dl, lg) = _inputs(352, [(2, *sp, 2, kv)] * 2, torch.float32)
    rq, rk = q.float().requires_grad_(True), k.float().requires_grad_(True)
    ref_l = P.na2d_qk_forward(rq, rk, ks, dil, (1, 1), causal, None)
    finite = torch.isfinite(ref_l)
    dl = torch.where(finite, dl, torch.zeros_like(dl)).to(torch.bfloat16)
    attn = torch.softmax(torch.where(finite, lg, torch.full_like(lg, -1e30)), -1).to(torch.bfloat16)
    qd, kd = q.to(DEV).requires_grad_(True), k.to(DEV).requires_grad_(True)
    ad, vd = attn.to(DEV).requires_grad_(True), v.to(DEV).requires_grad_(True)

    def run():
        logits = F.na2d_qk(qd, kd, ks, dil, is_causal=causal)
        logits.backward(dl.to(DEV))
        out = F.na2d_av(ad, vd, ks, dil, is_causal=causal)
        out.backward(do.to(DEV))
        return out

    out, ran = _launched(run)
    assert {"na_qk_bwd_k_lean", "na_av_bwd_v_lean"} <= ran, ran
    ref_l.backward(dl.float())
    ra, rv = attn.float().requires_grad_(True), v.float().requires_grad_(True)
    ref_o = P.na2d_av_forward(ra, rv, ks, dil, (1, 1), causal)
    ref_o.backward(do.float())
    assert_parity(out, ref_o, torch.bfloat16, "out")
    for name, a, b in (("dq", qd, rq), ("dk", kd, rk), ("dattn", ad, ra), ("dv", vd, rv)):
        assert_parity(a.grad, b.grad, torch.bfloat16, name)
