"""Pins the allin1 oracle (oracle/allin1.py, the reference's extras/allin1
pure ops) by what the definitions fix, on the CPU:

* for odd kernels the NATTEN 0.17 window equals the main operators' window
  (utils/window.py), so QK+RPB (zero bias) -> softmax -> AV equals the main
  oracle's na1d/na2d forward -- two independent constructions agree;
* the bias index of a valid neighbour is its relative offset
  (key - query)/dilation + K - 1 (the DiNAT relative-position table) for odd
  kernels;
* for an even kernel with dilation the window may start below zero; those
  neighbours are masked (-inf) and read nothing;
* float64 gradcheck of q, k, rpb and of attn, v (the reference's
  tests/test_extras_backward.py), plus the shapes and scale of
  tests/test_extras_allin1.py.
"""
from __future__ import annotations

import pytest
import torch

import oracle.allin1 as A
import oracle.pure as P


def _rand(shape, seed, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g, dtype=dtype)


@pytest.mark.parametrize("L,K,d", [(13, 5, 1), (17, 3, 3), (20, 7, 2)])
def test_odd_kernel_windows_equal_main_rule_1d(L, K, d):
    q, k, v = (_rand((2, L, 3, 4), s) for s in (1, 2, 3))
    logits = A.qkrpb_1d(q * 0.5, k, None, K, d)
    out = A.av_1d(logits.softmax(-1), v, K, d)
    ref = P.na1d_forward(q, k, v, (K,), (1,), (d,), (False,), 0.5)
    torch.testing.assert_close(out, ref, atol=1e-12, rtol=1e-12)


def test_odd_kernel_windows_equal_main_rule_2d():
    q, k, v = (_rand((1, 9, 11, 2, 4), s) for s in (4, 5, 6))
    logits = A.qkrpb_2d(q * 0.3, k, None, 3, 2)
    out = A.av_2d(logits.softmax(-1), v, 3, 2)
    ref = P.na2d_forward(q, k, v, (3, 3), (1, 1), (2, 2), (False, False), 0.3)
    torch.testing.assert_close(out, ref, atol=1e-12, rtol=1e-12)


@pytest.mark.parametrize("L,K,d", [(11, 5, 1), (19, 3, 2), (23, 7, 3)])
def test_bias_index_is_relative_offset(L, K, d):
    pos, valid, bias = A.axis_tables(L, K, d)
    i = torch.arange(L).reshape(L, 1)
    rel = (pos - i) // d + K - 1
    assert valid.all()
    assert torch.equal(bias, rel)
    # and through the op: a bias table holding its own index, zero query
    rpb = torch.arange(2 * K - 1, dtype=torch.float64).reshape(1, -1).repeat(2, 1)
    q = torch.zeros(1, L, 2, 4, dtype=torch.float64)
    logits = A.qkrpb_1d(q, _rand((1, L, 2, 4), 7), rpb, K, d)
    assert torch.equal(logits[0, :, 0], rel.to(torch.float64))


def test_key_within_k_class_steps_of_its_query():
    """Every valid neighbour shares the query's residue class and lies at
    most K class steps away (the bound the key-side gathers scan)."""
    for L in range(1, 30):
        for K in range(1, L + 1):
            for d in range(1, L // K + 1):
                pos, valid, _ = A.axis_tables(L, K, d)
                i = torch.arange(L).reshape(L, 1)
                diff = (pos - i)[valid]
                assert (diff % d == 0).all()
                assert (diff.abs() // d <= K).all()


def test_even_kernel_with_dilation_masks_negative_starts():
    L, K, d = 5, 2, 2
    pos, valid, _ = A.axis_tables(L, K, d)
    assert ((pos[~valid] < 0) | (pos[~valid] >= L)).all()
    q, k = _rand((1, L, 1, 3), 8), _rand((1, L, 1, 3), 9)
    logits = A.qkrpb_1d(q, k, None, K, d)
    assert torch.isinf(logits[0, :, 0][~valid]).all()
    assert torch.isfinite(logits[0, :, 0][valid]).all()
    assert (~valid).any()  # this configuration does reach below zero


@pytest.mark.parametrize("K,d", [(3, 1), (5, 1), (3, 2)])
def test_gradcheck_1d(K, d):
    L = max(K * 2 * d, 8)
    q, k = (_rand((1, L, 2, 4), s).requires_grad_(True) for s in (10, 11))
    rpb = _rand((2, 2 * K - 1), 12).requires_grad_(True)
    assert torch.autograd.gradcheck(lambda a, b, c: A.na1d_qk_rpb(a, b, c, K, d), (q, k, rpb), eps=1e-6, atol=1e-4,
                                    rtol=1e-3)
    attn, v = _rand((1, L, 2, K), 13).requires_grad_(True), _rand((1, L, 2, 4), 14).requires_grad_(True)
    assert torch.autograd.gradcheck(lambda a, b: A.av_1d(a, b, K, d), (attn, v), eps=1e-6, atol=1e-4, rtol=1e-3)


def test_gradcheck_2d():
    K = 3
    q, k = (_rand((1, 6, 6, 2, 3), s).requires_grad_(True) for s in (15, 16))
    rpb = _rand((2, 5, 5), 17).requires_grad_(True)
    assert torch.autograd.gradcheck(lambda a, b, c: A.na2d_qk_rpb(a, b, c, K), (q, k, rpb), eps=1e-6, atol=1e-4,
                                    rtol=1e-3)
    attn, v = _rand((1, 6, 6, 2, 9), 18).requires_grad_(True), _rand((1, 6, 6, 2, 3), 19).requires_grad_(True)
    assert torch.autograd.gradcheck(lambda a, b: A.av_2d(a, b, K, 1), (attn, v), eps=1e-6, atol=1e-4, rtol=1e-3)


def test_shapes_scale_and_none_rpb():
    q, k = _rand((1, 8, 2, 4), 20), _rand((1, 8, 2, 4), 21)
    a = A.na1d_qk_rpb(q, k, None, 3, scale=0.288)
    b = A.qkrpb_1d(q * 0.288, k, torch.zeros(2, 5, dtype=torch.float64), 3, 1)
    assert a.shape == (1, 8, 2, 3)
    torch.testing.assert_close(a, b, atol=0, rtol=0)
    q2 = _rand((2, 6, 7, 3, 4), 22)
    assert A.na2d_qk_rpb(q2, q2, None, 3).shape == (2, 6, 7, 3, 9)


def _allin1_golden():
    import json
    import os

    import numpy as np

    here = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
    with open(os.path.join(here, "allin1.json")) as f:
        meta = json.load(f)
    arrays = np.load(os.path.join(here, "allin1.npz"))
    return meta["cases"], arrays


_ALLIN1_CASES, _ALLIN1_ARRAYS = _allin1_golden()


@pytest.mark.parametrize("case", _ALLIN1_CASES, ids=lambda c: c["key"].rstrip("/"))
def test_oracle_matches_reference_allin1_fixtures(case):
    """The reference's own extras/allin1 ops (pure torch path on the CPU,
    tests/golden/make_golden.py --allin1): odd and even kernels, dilation
    1 and > 1, 1-D and 2-D, with and without a bias.  The oracle in fp32 on
    the same inputs gives the logits, dq, dk, drpb, out, dattn and dv within
    1e-5 (fp32 summation order aside, the same arithmetic)."""
    a = {n.split("/")[-1]: torch.from_numpy(_ALLIN1_ARRAYS[n]) for n in case["arrays"]}
    rank, K, d, scale = case["rank"], case["kernel_size"], case["dilation"], case["scale"]
    qk = A.na1d_qk_rpb if rank == 1 else A.na2d_qk_rpb
    av = A.av_1d if rank == 1 else A.av_2d
    q, k = a["q"].clone().requires_grad_(True), a["k"].clone().requires_grad_(True)
    r = a["rpb"].clone().requires_grad_(True) if case["with_rpb"] else None
    logits = qk(q, k, r, K, d, scale)
    torch.testing.assert_close(logits, a["logits"], atol=1e-5, rtol=1e-5)
    grads = torch.autograd.grad(logits, [q, k] + ([r] if r is not None else []), a["dlogits"])
    torch.testing.assert_close(grads[0], a["dq"], atol=1e-5, rtol=1e-5)
    torch.testing.assert_close(grads[1], a["dk"], atol=1e-5, rtol=1e-5)
    if r is not None:
        torch.testing.assert_close(grads[2], a["drpb"], atol=1e-4, rtol=1e-5)
    at, v = a["attn"].clone().requires_grad_(True), a["v"].clone().requires_grad_(True)
    out = av(at, v, K, d)
    torch.testing.assert_close(out, a["out"], atol=1e-5, rtol=1e-5)
    da, dv = torch.autograd.grad(out, [at, v], a["dout"])
    torch.testing.assert_close(da, a["dattn"], atol=1e-5, rtol=1e-5)
    torch.testing.assert_close(dv, a["dv"], atol=1e-5, rtol=1e-5)
