"""Pins the CPU oracle (oracle/pure.py) and the host composition layer to the
reference's own outputs: every golden case written from the reference by
tests/golden/make_golden.py.  Forward outputs and index maps must match bit
for bit on the same torch build; fp32 gradients within atol 5e-6 / rtol 1e-5,
because torch's CPU backward of the neighbour gather accumulates in a
thread-dependent order (two runs of the reference itself differ by up to
~1e-6 on O(0.1) values; a dropped or misplaced term moves them by O(1e-2))."""
from __future__ import annotations

import hashlib

import pytest
import torch

import oracle.pure as P


def _same(a, b):
    if torch.__version__ == _same.version:
        assert torch.equal(a, b), (a - b).abs().max()
    else:
        torch.testing.assert_close(a, b, atol=1e-6, rtol=1e-6)


_same.version = None


@pytest.fixture(autouse=True)
def _version(golden):
    _same.version = golden.meta["torch_version"]


def _close_grad(a, b):
    if a.dtype == torch.float32:
        torch.testing.assert_close(a, b, atol=5e-6, rtol=1e-5)
    else:
        torch.testing.assert_close(a, b, atol=1e-2, rtol=1e-2)


def _grads(fn, inputs, out_grad):
    leaves = [t.clone().requires_grad_(True) for t in inputs]
    out = fn(*leaves)
    return out, torch.autograd.grad(out, leaves, out_grad)


def test_fused_forward_and_grads(golden):
    cases = golden.cases("fwd")
    assert len(cases) >= 16
    for c in cases:
        p = c["key"]
        q, k, v, do = (golden.tensor(p + n) for n in ("q", "k", "v", "dout"))
        fn = getattr(P, f"na{c['rank']}d_forward")
        args = (tuple(c["kernel_size"]), tuple(c["stride"]), tuple(c["dilation"]), tuple(c["is_causal"]), c["scale"])
        out, (dq, dk, dv) = _grads(lambda a, b, d: fn(a, b, d, *args), (q, k, v), do)
        _same(out.detach(), golden.tensor(p + "out"))
        _close_grad(dq, golden.tensor(p + "dq"))
        _close_grad(dk, golden.tensor(p + "dk"))
        _close_grad(dv, golden.tensor(p + "dv"))


def test_split_qk_av_and_grads(golden):
    for c in golden.cases("split"):
        p, r = c["key"], c["rank"]
        ks, dil, st, causal = tuple(c["kernel_size"]), tuple(c["dilation"]), tuple(c["stride"]), tuple(c["is_causal"])
        q, k, v = (golden.tensor(p + n) for n in ("q", "k", "v"))
        qk = getattr(P, f"na{r}d_qk_forward")
        logits, (dq, dk) = _grads(lambda a, b: qk(a, b, ks, dil, st, causal, c["scale"]), (q, k),
                                  golden.tensor(p + "dlogits"))
        _same(logits.detach(), golden.tensor(p + "logits"))
        _close_grad(dq, golden.tensor(p + "dq"))
        _close_grad(dk, golden.tensor(p + "dk"))
        av = getattr(P, f"na{r}d_av_forward")
        out, (da, dv) = _grads(lambda a, b: av(a, b, ks, dil, st, causal), (golden.tensor(p + "attn"), v),
                               golden.tensor(p + "dout"))
        _same(out.detach(), golden.tensor(p + "out"))
        _close_grad(da, golden.tensor(p + "dattn"))
        _close_grad(dv, golden.tensor(p + "dv"))


def test_index_maps(golden):
    for c in golden.cases("map"):
        flat, valid = P.neighborhood(c["rank"], c["spatial"], c["kernel_size"], c["dilation"], c["stride"],
                                     c["is_causal"])
        assert torch.equal(flat, golden.tensor(c["key"] + "flat"))
        if valid is None:
            assert len(c["arrays"]) == 1
        else:
            assert torch.equal(valid.to(torch.uint8), golden.tensor(c["key"] + "valid").to(torch.uint8))
    for c in golden.cases("map_digest"):
        flat, _ = P.neighborhood(c["rank"], c["spatial"], c["kernel_size"], c["dilation"], c["stride"],
                                 c["is_causal"])
        digest = hashlib.sha256(flat.contiguous().numpy().astype("<i8").tobytes()).hexdigest()
        assert digest == c["sha256"]
        assert torch.equal(flat.reshape(-1)[::c["sample_step"]], golden.tensor(c["key"] + "sample"))
    (c,) = golden.cases("map1d_causal")
    idx, valid = P.axis_indices(torch.arange(c["length"]), c["length"], c["kernel"], c["dilation"], True, "cpu")
    assert torch.equal(idx, golden.tensor("mapc/idx"))
    assert torch.equal(valid.to(torch.uint8), golden.tensor("mapc/valid").to(torch.uint8))


def test_window_starts(golden):
    table = golden.tensor("starts/table").to(torch.long)
    got = torch.tensor([P.window_start(int(i), int(L), int(K), int(d)) for L, K, d, i, _ in table.tolist()])
    assert torch.equal(got, table[:, 4])
    vec = []
    for L in (17, 56):
        for K in (3, 4, 7):
            for d in (1, 2, 3, 8):
                if d * K <= L:
                    vec.append(P.window_start_vec(torch.arange(L), L, K, d))
    assert torch.equal(torch.cat(vec), golden.tensor("starts/vec"))


def test_config1_output(golden):
    g = torch.Generator().manual_seed(1001)
    q, k, v = (torch.randn((2, 128, 4, 32), generator=g, dtype=torch.float32) for _ in range(3))
    out = P.na1d_forward(q, k, v, (7,), (1,), (1,), (False,), 32 ** -0.5)
    _same(out, golden.tensor("cfg1/out"))


def test_functional_layer_on_oracle(golden, pure_backend):
    """The package's functional layer (GQA, SDPA fast path, return_lse,
    additional_keys + merge) over the oracle backend equals the reference's
    functional API over its pure backend."""
    import natten_mps_amd.functional as F

    cases = golden.cases("func")
    assert len(cases) >= 7
    for c in cases:
        p = c["key"]
        leaves = [golden.tensor(p + n).requires_grad_(True) for n in ("q", "k", "v")]
        extra = [None, None]
        if c["n_extra"]:
            extra = [golden.tensor(p + n).requires_grad_(True) for n in ("ak", "av")]
        fn = getattr(F, f"na{c['rank']}d")
        res = fn(*leaves, kernel_size=c["kernel_size"], stride=c["stride"], dilation=c["dilation"],
                 is_causal=c["is_causal"], return_lse=c["return_lse"], additional_keys=extra[0],
                 additional_values=extra[1])
        out, lse = res if c["return_lse"] else (res, None)
        torch.testing.assert_close(out.detach(), golden.tensor(p + "out"), atol=1e-6, rtol=1e-6)
        terms, grads_in = [out], [golden.tensor(p + "dout")]
        if lse is not None:
            torch.testing.assert_close(lse.detach(), golden.tensor(p + "lse"), atol=1e-6, rtol=1e-6)
            terms.append(lse)
            grads_in.append(golden.tensor(p + "dlse"))
        wrt = leaves + ([extra[0], extra[1]] if c["n_extra"] else [])
        got = torch.autograd.grad(terms, wrt, grads_in)
        names = ["dq", "dk", "dv"] + (["dak", "dav"] if c["n_extra"] else [])
        for n, g in zip(names, got):
            torch.testing.assert_close(g, golden.tensor(p + n), atol=1e-5, rtol=1e-5)
