"""The parity bound of the 'hip' backend against the oracle, stated once and
used by every GPU test that compares values.

* fp32 (north star: within 1e-5 abs/rel): elementwise
  ``|a - b| <= 1e-5 + 1e-5 |b|`` against the oracle evaluated in fp32.  Where
  a result sums hundreds of products (3-D windows of 125-343 neighbours) the
  oracle's own fp32 summation order is not more exact than the kernels', so
  those cases compare against the oracle evaluated in float64 instead
  (``ref_dtype=torch.float64`` in the callers), with the same bound.
* bf16 / fp16 (north star: within 2e-2 relative): the kernels round the
  probabilities and score gradients to the input dtype before the second
  product, so the error is a rounding noise spread over the tensor.  The
  bound is relative over the whole compared tensor,
  ``||a - b||_2 <= 2e-2 ||b||_2``, against the oracle evaluated in fp32 on
  the same rounded inputs, together with an elementwise guard
  ``|a - b| <= 5e-2 + 5e-2 |b|``: a wrong or missing neighbour changes an
  element by the size of the values themselves and fails the guard even
  where the norm-wise bound would absorb it.
"""
from __future__ import annotations

import os

import torch

FP32_TOL = 1e-5
HALF_NORM_REL = 2e-2
HALF_GUARD = 5e-2

# (test, tensor, dtype, norm-wise relative error, largest elementwise
# |a - b| / (1 + |b|)) of every half-precision comparison of the session;
# conftest prints the largest at the end, so a drift towards the guard stays
# visible.
RECORD: list = []


def assert_parity(got: torch.Tensor, ref: torch.Tensor, dtype: torch.dtype, name: str = "") -> None:
    """Check ``got`` (the HIP result, any device) against ``ref`` (the
    oracle) under the bound of ``dtype``, the arithmetic type of the call."""
    a = got.detach().float().cpu()
    b = ref.detach().float().cpu()
    assert a.shape == b.shape, f"{name}: shape {tuple(a.shape)} != {tuple(b.shape)}"
    if dtype == torch.float32:
        # NaN where the oracle has NaN (and Inf exactly where it has Inf)
        torch.testing.assert_close(a, b, atol=FP32_TOL, rtol=FP32_TOL, equal_nan=True, msg=lambda m: f"{name}: {m}")
        return
    fa, fb = torch.isfinite(a), torch.isfinite(b)
    assert torch.equal(fa, fb), f"{name}: {int((fa != fb).sum())} elements differ in finiteness"
    a, b = a[fb], b[fb]
    if b.numel() == 0:
        return
    err = float((a.double() - b.double()).norm())
    scale = float(b.double().norm())
    elem = float(((a.double() - b.double()).abs() / (1.0 + b.double().abs())).max())
    test = os.environ.get("PYTEST_CURRENT_TEST", "").split(" ")[0]
    RECORD.append((test, name, str(dtype).replace("torch.", ""), err / max(scale, 1e-30), elem))
    assert err <= HALF_NORM_REL * scale + 1e-12, (
        f"{name}: relative error {err / max(scale, 1e-30):.3g} exceeds {HALF_NORM_REL} (norm-wise); "
        f"largest elementwise |a-b|/(1+|b|) {elem:.3g}")
    torch.testing.assert_close(a, b, atol=HALF_GUARD, rtol=HALF_GUARD,
                               msg=lambda m: f"{name} (guard; norm-wise {err / max(scale, 1e-30):.3g}): {m}")
