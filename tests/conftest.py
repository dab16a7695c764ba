"""Shared test set-up.

* puts the repo root (for ``oracle``) and ``natten-mps_amd/`` (for the
  ``natten_mps_amd`` package) on sys.path;
* registers the ``gpu`` marker: GPU tests run the HIP library on a ROCm
  device and are skipped when none is present;
* ``pure_backend``: registers the CPU oracle (``oracle/pure.py``) as the
  ``'pure'`` backend for the duration of a test, the way the reference's tests
  switch to its pure backend.
"""
from __future__ import annotations

import json
import os
import sys

import numpy as np
import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "natten-mps_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

GOLDEN_DIR = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU and the built libnatten_hip.so")


def pytest_collection_modifyitems(config, items):
    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no ROCm GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


def pytest_terminal_summary(terminalreporter):
    """The largest half-precision errors of the session against the oracle
    (tests/_parity.py records every comparison), elementwise and norm-wise,
    so that a drift between the 2e-2 norm-wise bound and the 5e-2 guard shows
    in the output of every run."""
    try:
        from _parity import RECORD
    except ImportError:
        return
    if not RECORD:
        return
    tr = terminalreporter
    tr.section("half-precision parity: largest errors against the oracle")
    tr.write_line(f"{len(RECORD)} comparisons; bounds: norm-wise 2e-2, elementwise guard 5e-2 (+5e-2 |ref|)")
    for label, key in (("elementwise |a-b|/(1+|b|)", 4), ("norm-wise relative", 3)):
        tr.write_line(f"largest {label}:")
        for rec in sorted(RECORD, key=lambda r: -r[key])[:8]:
            tr.write_line(f"  {rec[key]:.4g}  {rec[1]:5s} {rec[2]:8s} {rec[0]}")


@pytest.fixture
def pure_backend():
    import natten_mps_amd
    from natten_mps_amd._core import ops
    import oracle.pure as oracle_pure

    prev = ops._ACTIVE_BACKEND
    natten_mps_amd.register_backend("pure", oracle_pure)
    natten_mps_amd.set_backend("pure")
    try:
        yield oracle_pure
    finally:
        ops.unregister_backend("pure")
        ops._ACTIVE_BACKEND = prev if prev in ops._BACKEND_REGISTRY or prev == "auto" else "auto"


class Golden:
    """Reader for tests/golden/golden.{json,npz} (written by make_golden.py)."""

    def __init__(self):
        with open(os.path.join(GOLDEN_DIR, "golden.json")) as f:
            self.meta = json.load(f)
        self.npz = np.load(os.path.join(GOLDEN_DIR, "golden.npz"), allow_pickle=False)

    def cases(self, kind):
        return [c for c in self.meta["cases"] if c["kind"] == kind]

    def tensor(self, key, dtype="float32"):
        a = self.npz[key]
        if a.dtype == np.uint16:  # raw bf16 bits
            return torch.from_numpy(a.view(np.int16).copy()).view(torch.bfloat16)
        t = torch.from_numpy(a.copy())
        if t.dtype == torch.int32:
            t = t.to(torch.long)
        return t


@pytest.fixture(scope="session")
def golden():
    return Golden()
