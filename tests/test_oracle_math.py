"""Pins the CPU oracle (oracle/pure.py) by what the mathematics fixes,
independently of the golden fixtures: closed forms, special cases and
identities chosen so that a plausible slip (a dropped scale, a wrong window
offset, a transposed operand, a missing causal mask, a wrong GQA head map)
fails at least one of them.  All on the CPU in float64 unless noted."""
from __future__ import annotations

import math

import pytest
import torch

import oracle.pure as P


def _rand(shape, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g, dtype=torch.float64)


def _dense(q, k, v, scale, mask=None):
    """Dense attention over the flattened spatial axes, per head:
    q [B, N, H, D], k/v [B, N, H, D] -> [B, N, H, D]."""
    logits = torch.einsum("bnhd,bmhd->bhnm", q, k) * scale
    if mask is not None:
        logits = logits.masked_fill(~mask, float("-inf"))
    return torch.einsum("bhnm,bmhd->bnhd", logits.softmax(-1), v)


def test_window_equal_to_axis_is_global_attention_1d():
    """Odd K == L, non-causal, dilation 1: every window is the whole axis."""
    B, L, H, D = 2, 9, 3, 8
    q, k, v = (_rand((B, L, H, D), s) for s in (1, 2, 3))
    out = P.na1d_forward(q, k, v, (L,), (1,), (1,), (False,), None)
    ref = _dense(q, k, v, D ** -0.5)
    torch.testing.assert_close(out, ref, atol=1e-12, rtol=1e-12)


def test_window_equal_to_extent_is_global_attention_2d_and_3d():
    B, H, D = 1, 2, 4
    q, k, v = (_rand((B, 5, 7, H, D), s) for s in (4, 5, 6))
    out = P.na2d_forward(q, k, v, (5, 7), (1, 1), (1, 1), (False, False), 0.3)
    ref = _dense(q.reshape(B, 35, H, D), k.reshape(B, 35, H, D), v.reshape(B, 35, H, D), 0.3)
    torch.testing.assert_close(out.reshape(B, 35, H, D), ref, atol=1e-12, rtol=1e-12)
    q, k, v = (_rand((B, 3, 3, 5, H, D), s) for s in (7, 8, 9))
    out = P.na3d_forward(q, k, v, (3, 3, 5), (1, 1, 1), (1, 1, 1), (False, False, False), None)
    ref = _dense(q.reshape(B, 45, H, D), k.reshape(B, 45, H, D), v.reshape(B, 45, H, D), D ** -0.5)
    torch.testing.assert_close(out.reshape(B, 45, H, D), ref, atol=1e-12, rtol=1e-12)


def test_causal_window_covering_axis_is_causal_attention():
    """Causal with K == L: query i attends keys 0..i (lower-triangular mask);
    query 0 returns v[0] exactly."""
    B, L, H, D = 2, 11, 2, 6
    q, k, v = (_rand((B, L, H, D), s) for s in (10, 11, 12))
    out = P.na1d_forward(q, k, v, (L,), (1,), (1,), (True,), None)
    mask = torch.ones(L, L, dtype=torch.bool).tril()
    torch.testing.assert_close(out, _dense(q, k, v, D ** -0.5, mask), atol=1e-12, rtol=1e-12)
    torch.testing.assert_close(out[:, 0], v[:, 0], atol=0, rtol=0)


def test_small_window_against_brute_force_window_definition():
    """Every query attends exactly the keys of its shifted window: brute
    force from the textbook rule (centred, shifted inwards at the borders,
    dilation keeps the residue class) on a dense mask."""
    B, L, H, D, K, d = 1, 13, 2, 5, 5, 2
    q, k, v = (_rand((B, L, H, D), s) for s in (13, 14, 15))
    mask = torch.zeros(L, L, dtype=torch.bool)
    for i in range(L):
        cls = [j for j in range(L) if j % d == i % d]      # the query's residue class
        pos = cls.index(i)
        start = min(max(pos - K // 2, 0), len(cls) - K)      # window of K class members
        for j in cls[start:start + K]:
            mask[i, j] = True
    out = P.na1d_forward(q, k, v, (K,), (1,), (d,), (False,), 0.7)
    torch.testing.assert_close(out, _dense(q, k, v, 0.7, mask), atol=1e-12, rtol=1e-12)


def test_fused_equals_split_composition_and_lse():
    """Fused forward == softmax(split QK with scale) -> split AV, and the
    log-sum-exp of the split logits is what a caller would recompute."""
    B, H, D = 2, 2, 8
    q, k, v = (_rand((B, 6, 7, H, D), s) for s in (16, 17, 18))
    ks, dil, causal = (3, 5), (2, 1), (True, False)
    fused = P.na2d_forward(q, k, v, ks, (1, 1), dil, causal, 0.25)
    logits = P.na2d_qk_forward(q, k, ks, dil, (1, 1), causal, 0.25)
    split = P.na2d_av_forward(logits.softmax(-1), v, ks, dil, (1, 1), causal)
    torch.testing.assert_close(fused, split, atol=1e-12, rtol=1e-12)
    lse = torch.logsumexp(logits, -1)
    assert torch.isfinite(lse).all()


def test_scale_enters_once():
    """scale s on the fused op equals pre-scaling q by s with scale 1."""
    B, L, H, D = 1, 10, 1, 4
    q, k, v = (_rand((B, L, H, D), s) for s in (19, 20, 21))
    a = P.na1d_forward(q, k, v, (3,), (1,), (1,), (False,), 0.5)
    b = P.na1d_forward(q * 0.5, k, v, (3,), (1,), (1,), (False,), 1.0)
    torch.testing.assert_close(a, b, atol=1e-12, rtol=1e-12)


def test_gqa_equals_repeated_kv():
    """Query head h reads kv head h // (Hq / Hkv): equals expanding k, v."""
    B, L, Hq, Hkv, D = 2, 12, 6, 2, 4
    q = _rand((B, L, Hq, D), 22)
    k, v = _rand((B, L, Hkv, D), 23), _rand((B, L, Hkv, D), 24)
    rep = Hq // Hkv
    ke, ve = k.repeat_interleave(rep, dim=2), v.repeat_interleave(rep, dim=2)
    out = P.forward(1, q, ke, ve, (5,), (1,), (1,), (False,), None)
    for h in range(Hq):
        single = P.na1d_forward(q[:, :, h:h + 1], k[:, :, h // rep:h // rep + 1], v[:, :, h // rep:h // rep + 1],
                                (5,), (1,), (1,), (False,), None)
        torch.testing.assert_close(out[:, :, h:h + 1], single, atol=1e-12, rtol=1e-12)


@pytest.mark.parametrize("causal", [False, True])
def test_gradients_against_finite_differences(causal):
    """float64 gradcheck of the oracle forward (the backward the reference
    takes from autograd, _core/pure.py:680-696)."""
    B, L, H, D = 1, 7, 1, 3
    q, k, v = (_rand((B, L, H, D), s).requires_grad_(True) for s in (25, 26, 27))
    f = lambda a, b, c: P.na1d_forward(a, b, c, (3,), (1,), (2,), (causal,), 0.9)  # noqa: E731
    assert torch.autograd.gradcheck(f, (q, k, v), eps=1e-6, atol=1e-7, rtol=1e-5)


def test_softmax_gradient_identity():
    """dS = P (dP - sum(P dP)) -- the identity the fused backward uses --
    matches autograd through the split composition."""
    B, L, H, D = 1, 9, 2, 4
    q, k, v, g = (_rand((B, L, H, D), s) for s in (28, 29, 30, 31))
    q.requires_grad_(True)
    logits = P.na1d_qk_forward(q, k, (5,), (1,), (1,), (False,), 0.6)
    p = logits.softmax(-1)
    out = P.na1d_av_forward(p, v, (5,), (1,), (1,), (False,))
    (dq_auto,) = torch.autograd.grad(out, q, g)
    # manual: dP[o, e] = g[o] . v[nbr(o, e)], dS = P (dP - delta) with delta = sum_e P dP = g . out
    flat, _ = P.neighborhood(1, (L,), (5,), (1,), (1,), (False,))
    vn = v[:, flat.reshape(-1)].reshape(B, L, 5, H, D)
    dp = torch.einsum("blhd,blehd->blhe", g, vn)
    delta = (g * out.detach()).sum(-1, keepdim=True)
    ds = p.detach() * (dp - delta)
    kn = k[:, flat.reshape(-1)].reshape(B, L, 5, H, D)
    dq_manual = torch.einsum("blhe,blehd->blhd", ds, kn) * 0.6
    torch.testing.assert_close(dq_auto, dq_manual, atol=1e-12, rtol=1e-10)
    assert math.isfinite(float(delta.sum()))
