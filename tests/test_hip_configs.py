"""The five BASELINE configurations on the 'hip' backend at their full sizes.

Inputs: ``torch.Generator().manual_seed(1000 + cfg)``, order q, k, v, dO, each
``randn`` in fp32 then cast.  The oracle is evaluated where it is exact and
affordable on the host:

* cfg 1, 2: the whole problem (cfg 1 also against the reference's golden output);
* cfg 3: batch items 0-1 (batch items are independent);
* cfg 4: batch item 0, the prefix of 2048 positions (a causal 1-D window never
  reaches forward, so a prefix is self-contained; dK/dV are compared where
  every contributing query lies in the prefix);
* cfg 5: batch item 0, head 0, and batch item 1, head 5 (heads are
  independent, Hq == Hkv);
* cfgs 3, 4, 5 at full size against the split composition (QK -> softmax ->
  AV, other kernels), every batch item, head and position.

Bounds: ``tests/_parity.py`` (bf16 within 2e-2 norm-wise relative with an
elementwise guard, the oracle run in fp32 on the same bf16 inputs; fp32
within 1e-5 elementwise).
"""
from __future__ import annotations

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


def _seeded(cfg, shapes, dtype):
    g = torch.Generator().manual_seed(1000 + cfg)
    return [torch.randn(s, generator=g, dtype=torch.float32).to(dtype) for s in shapes]


def _run(fn, q, k, v, do, **kw):
    leaves = [t.to(DEV).requires_grad_(True) for t in (q, k, v)]
    out = fn(*leaves, **kw)
    out.backward(do.to(DEV))
    torch.cuda.synchronize()
    return out.detach().cpu(), [t.grad.cpu() for t in leaves]


def _oracle(rank, q, k, v, do, ks, st, dil, causal):
    leaves = [t.float().clone().requires_grad_(True) for t in (q, k, v)]
    out = P.forward(rank, *leaves, ks, st, dil, causal, None)
    out.backward(do.float())
    return out.detach(), [t.grad for t in leaves]


def _close(a, b, tol, name):
    """tol 1e-5: the fp32 bound; 2e-2: the half-precision bound (both from
    tests/_parity.py); other values: an elementwise bound between two HIP
    paths (fused against the split composition)."""
    if tol in (1e-5, 2e-2):
        assert_parity(a, b, torch.float32 if tol == 1e-5 else torch.bfloat16, name)
    else:
        torch.testing.assert_close(a.float(), b.float(), atol=tol, rtol=tol, msg=lambda m: f"{name}: {m}")


def test_config1_na1d_fp32(golden):
    from natten_mps_amd import functional as F

    q, k, v = _seeded(1, [(2, 128, 4, 32)] * 3, torch.float32)
    out = F.na1d(q.to(DEV), k.to(DEV), v.to(DEV), kernel_size=7, scale=32 ** -0.5).cpu()
    _close(out, golden.tensor("cfg1/out"), 1e-5, "cfg1 out")


@pytest.mark.parametrize("causal", [(False, False), (True, False)])
def test_config2_na2d_fp32(causal):
    from natten_mps_amd import functional as F

    q, k, v, do = _seeded(2, [(2, 32, 32, 4, 32)] * 4, torch.float32)
    out, grads = _run(F.na2d, q, k, v, do, kernel_size=7, is_causal=causal)
    ref, rgrads = _oracle(2, q, k, v, do, (7, 7), (1, 1), (1, 1), causal)
    _close(out, ref, 1e-5, "out")
    for n, a, b in zip(("dq", "dk", "dv"), grads, rgrads):
        _close(a, b, 1e-5, n)


@pytest.mark.parametrize("dil", [1, 8])
def test_config3_na2d_bf16(dil):
    from natten_mps_amd import functional as F

    q, k, v, do = _seeded(3, [(16, 56, 56, 4, 32)] * 4, torch.bfloat16)
    out, grads = _run(F.na2d, q, k, v, do, kernel_size=7, dilation=dil)
    sl = slice(0, 2)
    ref, rgrads = _oracle(2, q[sl], k[sl], v[sl], do[sl], (7, 7), (1, 1), (dil, dil), (False, False))
    _close(out[sl], ref, 2e-2, "out")
    for n, a, b in zip(("dq", "dk", "dv"), grads, rgrads):
        _close(a[sl], b, 2e-2, n)
    # fused vs split QK -> softmax -> AV on the device, whole problem,
    # forward and backward (the split path rounds its logits, probabilities
    # and their gradients to bf16 on the way, hence the wider bound on the
    # gradients)
    qd, kd, vd = (t.to(DEV).requires_grad_(True) for t in (q, k, v))
    logits = F.na2d_qk(qd, kd, 7, dil) * 32 ** -0.5
    split = F.na2d_av(torch.softmax(logits.float(), -1).to(torch.bfloat16), vd, 7, dil)
    _close(split.detach().cpu(), out, 2e-2, "fused vs split")
    split.backward(do.to(DEV))
    for n, t, g in zip(("dq", "dk", "dv"), (qd, kd, vd), grads):
        _close(t.grad.cpu(), g, 5e-2, f"fused vs split {n}")


@pytest.mark.parametrize("dil", [1, 4])
def test_config4_na1d_gqa_causal_bf16(dil):
    from natten_mps_amd import functional as F

    q, k, v, do = _seeded(4, [(4, 16384, 8, 64), (4, 16384, 2, 64), (4, 16384, 2, 64), (4, 16384, 8, 64)],
                          torch.bfloat16)
    out, grads = _run(F.na1d, q, k, v, do, kernel_size=33, dilation=dil, is_causal=True)
    n = 2048
    ref, rgrads = _oracle(1, q[:1, :n], k[:1, :n], v[:1, :n], do[:1, :n], (33,), (1,), (dil,), (True,))
    _close(out[:1, :n], ref, 2e-2, "out")
    _close(grads[0][:1, :n], rgrads[0], 2e-2, "dq")
    m = n - 32 * dil
    _close(grads[1][:1, :m], rgrads[1][:, :m], 2e-2, "dk")
    _close(grads[2][:1, :m], rgrads[2][:, :m], 2e-2, "dv")


def test_config5_na3d_bf16():
    from natten_mps_amd import functional as F

    q, k, v, do = _seeded(5, [(2, 16, 32, 32, 8, 64)] * 4, torch.bfloat16)
    ks, dil = (3, 7, 7), (1, 2, 2)
    out, grads = _run(F.na3d, q, k, v, do, kernel_size=ks, dilation=dil)
    # (batch 0, head 0) and (batch 1, head 5): the oracle on one head of one
    # sample at a time
    for b, h in ((0, 0), (1, 5)):
        sl = (slice(b, b + 1), Ellipsis, slice(h, h + 1), slice(None))
        ref, rgrads = _oracle(3, q[sl], k[sl], v[sl], do[sl], ks, (1, 1, 1), dil, (False, False, False))
        _close(out[sl], ref, 2e-2, f"out[b{b},h{h}]")
        for n_, a, r in zip(("dq", "dk", "dv"), grads, rgrads):
            _close(a[sl], r, 2e-2, f"{n_}[b{b},h{h}]")


@pytest.mark.parametrize("cfg", [4, 5])
def test_backward_is_bitwise_deterministic(cfg):
    """The dK/dV gather has no atomics, so repeated backward passes agree bit
    for bit over the whole tensors (not only the slices the oracle checks).
    Covers the key-side walk over several staged slices per workgroup: the
    GQA group's q heads (cfg 4) and the axis-0 planes of a 3-D union (cfg 5),
    whose per-slice -lse / -delta rows go through LDS stores and a barrier."""
    from natten_mps_amd import functional as F

    if cfg == 4:
        shapes = [(4, 16384, 8, 64), (4, 16384, 2, 64), (4, 16384, 2, 64), (4, 16384, 8, 64)]
        fn, kw = F.na1d, dict(kernel_size=33, dilation=1, is_causal=True)
    else:
        shapes = [(2, 16, 32, 32, 8, 64)] * 4
        fn, kw = F.na3d, dict(kernel_size=(3, 7, 7), dilation=(1, 2, 2))
    q, k, v, do = (t.to(DEV) for t in _seeded(cfg, shapes, torch.bfloat16))
    leaves = [t.requires_grad_(True) for t in (q, k, v)]

    def step():
        out = fn(*leaves, **kw)
        return [out.detach()] + list(torch.autograd.grad(out, leaves, do))

    ref = step()
    for _ in range(4):
        for name, a, b in zip(("out", "dq", "dk", "dv"), step(), ref):
            assert torch.equal(a, b), f"{name}: {int((a != b).sum())} elements differ between runs"


# Full-size check: the fused path against the split composition on the whole
# problem.  The two share no kernel (fused forward/backward tile kernels
# against the split QK / AV tile kernels, torch's softmax in fp32 between
# them), so agreement over every batch item, head and position checks what
# the sliced oracle comparisons above leave out.  The split path rounds its
# logits and probabilities to bf16, so the bound is the half-precision one
# with the fused result as reference.
FULL = {
    3: dict(shape=(16, 56, 56), hq=4, hkv=4, dim=32, ks=(7, 7), dil=(1, 1), causal=(False, False)),
    4: dict(shape=(4, 16384), hq=8, hkv=2, dim=64, ks=(33,), dil=(1,), causal=(True,)),
    5: dict(shape=(2, 16, 32, 32), hq=8, hkv=8, dim=64, ks=(3, 7, 7), dil=(1, 2, 2), causal=(False, False, False)),
}


@pytest.mark.parametrize("cfg", sorted(FULL))
def test_full_size_fused_matches_split_composition(cfg):
    from natten_mps_amd import functional as F

    c = FULL[cfg]
    rank = len(c["ks"])
    B, sp = c["shape"][0], c["shape"][1:]
    q, k, v, do = _seeded(cfg, [(B, *sp, c["hq"], c["dim"]), (B, *sp, c["hkv"], c["dim"]),
                                (B, *sp, c["hkv"], c["dim"]), (B, *sp, c["hq"], c["dim"])], torch.bfloat16)
    kw = dict(kernel_size=c["ks"], dilation=c["dil"], is_causal=c["causal"])
    fn = {1: F.na1d, 2: F.na2d, 3: F.na3d}[rank]
    out, grads = _run(fn, q, k, v, do, **kw)

    rep = c["hq"] // c["hkv"]
    leaves = [t.to(DEV).requires_grad_(True) for t in (q, k, v)]
    kx, vx = (t.repeat_interleave(rep, dim=-2) if rep > 1 else t for t in leaves[1:])
    qk = {1: F.na1d_qk, 2: F.na2d_qk, 3: F.na3d_qk}[rank]
    av = {1: F.na1d_av, 2: F.na2d_av, 3: F.na3d_av}[rank]
    logits = qk(leaves[0], kx, c["ks"], c["dil"], is_causal=c["causal"], scale=c["dim"] ** -0.5)
    attn = torch.softmax(logits.float(), -1).to(torch.bfloat16)
    ref = av(attn, vx, c["ks"], c["dil"], is_causal=c["causal"])
    ref.backward(do.to(DEV))
    torch.cuda.synchronize()
    assert_parity(ref.detach(), out, torch.bfloat16, f"cfg{cfg} split out")
    for name, a, g in zip(("dq", "dk", "dv"), leaves, grads):
        assert_parity(a.grad, g, torch.bfloat16, f"cfg{cfg} split {name}")
