"""The C-ABI library without a GPU: it loads, exports every entry point
include/natten_hip.h declares, its structs have the layout the ctypes binding
assumes, and argument validation (host code that runs before any launch)
returns the documented status codes."""
from __future__ import annotations

import ctypes
import os
import re
import subprocess

import pytest

from conftest import ROOT
from natten_mps_amd._core import _lib

HEADER = os.path.join(ROOT, "include", "natten_hip.h")


def _declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:int|int64_t|const char \*)\s*(natten_hip_\w+)\(", text, re.M)))


@pytest.fixture(scope="module")
def lib():
    if not _lib.is_built():
        pytest.fail("libnatten_hip.so is not built (run python natten-mps_amd/build_lib.py)")
    return _lib.load()


def test_exports_every_declared_symbol(lib):
    declared = _declared()
    assert len(declared) >= 9
    assert set(declared) == set(_lib.ENTRY_POINTS)
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    exported = set(re.findall(r"\bT (natten_hip_\w+)", out))
    assert set(declared) <= exported
    assert lib.natten_hip_abi_version() == _lib.ABI_VERSION


def test_struct_layout_matches_header(tmp_path):
    src = tmp_path / "probe.c"
    src.write_text(r'''
#include <stddef.h>
#include <stdio.h>
#include "natten_hip.h"
int main(void) {
  printf("%zu %zu %zu %zu %zu %zu\n", sizeof(natten_problem_t), offsetof(natten_problem_t, scale),
         offsetof(natten_problem_t, length), offsetof(natten_problem_t, causal),
         sizeof(natten_layout_t), offsetof(natten_layout_t, head));
  return 0;
}
''')
    exe = tmp_path / "probe"
    subprocess.run(["gcc", "-I" + os.path.join(ROOT, "include"), str(src), "-o", str(exe)], check=True)
    got = [int(x) for x in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()]
    P, L = _lib.Problem, _lib.Layout
    assert got == [ctypes.sizeof(P), P.scale.offset, P.length.offset, P.causal.offset, ctypes.sizeof(L),
                   L.head.offset]


def _prob(**over):
    kw = dict(batch=1, heads_q=2, heads_kv=2, dim_qk=8, dim_v=8, dtype=_lib.F32, length=(16,), out_length=(16,),
              kernel_size=(5,), dilation=(1,), stride=(1,), is_causal=(False,), scale=0.5)
    kw.update(over)
    return _lib.problem(**kw)


@pytest.mark.parametrize("over, code, text", [
    (dict(kernel_size=(5,), dilation=(4,)), 1, "exceeds length"),
    (dict(heads_q=3, heads_kv=2), 1, "divisible"),
    (dict(dim_qk=300, dim_v=300), 2, "above 256"),
    (dict(out_length=(8,)), 1, "query extent"),
    (dict(length=(6,), out_length=(6,), kernel_size=(6,)), 2, "even kernel"),
    (dict(dtype=7), 1, "dtype"),
    (dict(batch=0), 1, "batch"),
])
def test_validation_codes(lib, over, code, text):
    lay = ctypes.byref(_lib.Layout())
    dummy = ctypes.c_void_p(16)  # never dereferenced: validation fails first
    rc = lib.natten_hip_forward(ctypes.byref(_prob(**over)), dummy, lay, dummy, lay, dummy, lay, dummy, lay,
                                dummy, lay, None)
    assert rc == code
    assert text in lib.natten_hip_last_error().decode()


def test_null_operand_rejected(lib):
    lay = ctypes.byref(_lib.Layout())
    rc = lib.natten_hip_forward(ctypes.byref(_prob()), None, lay, None, lay, None, lay, None, lay, None, lay, None)
    assert rc == 1 and "NULL" in lib.natten_hip_last_error().decode()


def test_split_ops_need_equal_heads(lib):
    lay = ctypes.byref(_lib.Layout())
    d = ctypes.c_void_p(16)
    rc = lib.natten_hip_qk_forward(ctypes.byref(_prob(heads_q=4, heads_kv=2)), d, lay, d, lay, d, lay, None)
    assert rc == 1 and "heads_q == heads_kv" in lib.natten_hip_last_error().decode()


def test_python_errors_map_to_exceptions(lib):
    with pytest.raises(ValueError, match="exceeds length"):
        _lib.check(lib.natten_hip_forward(ctypes.byref(_prob(dilation=(4,))), *([ctypes.c_void_p(16),
                   ctypes.byref(_lib.Layout())] * 5), None), "forward")


def test_ctypes_arity_matches_header():
    """Every binding takes exactly the parameters the header declares."""
    import re as _re

    text = open(HEADER).read()
    for name, (args, _) in _lib._SIGNATURES.items():
        m = _re.search(rf"\b{name}\(([^)]*)\)", text)
        assert m, name
        params = [p for p in m.group(1).split(",") if p.strip() and p.strip() != "void"]
        assert len(params) == len(args), (name, len(params), len(args))


def test_torch_binding_loads_against_the_same_library(lib):
    """The C++ host binding (_natten_torch.so) is built beside the library,
    needs it by soname and resolves to the copy already loaded: one
    libnatten_hip.so mapping in the process.  Its call object rejects
    malformed descriptors before any device work."""
    import torch

    b = _lib.binding()
    assert b is not None, "the host binding _natten_torch.so is not built"
    assert b.abi_version == _lib.ABI_VERSION
    maps = {line.split()[-1] for line in open("/proc/self/maps") if line.rstrip().endswith("libnatten_hip.so")}
    assert len(maps) == 1, maps
    needed = subprocess.run(["readelf", "-d", _lib.BIND_PATH], capture_output=True, text=True, check=True).stdout
    assert "[libnatten_hip.so]" in needed
    with pytest.raises(ValueError, match="problem size"):
        b.FusedCall(b"\0" * 4, bytes(_lib.Layout()) * 5, [1], [1], False)
    call = b.FusedCall(bytes(_prob()), bytes(_lib.Layout()) * 5, [1], [1], False)
    with pytest.raises(ValueError, match="not a backward signature"):
        z = torch.zeros(1)
        call.backward(z, z, z, z, z, z, None, 0)


def test_every_device_function_is_inlined_into_a_kernel():
    """The non-finite recomputation paths read the kernel-argument pointer,
    which only the kernel's own code may do: the built gfx950 code objects
    hold no device function outside a kernel (each FUNC symbol has its
    kernel descriptor).  build_lib.build() runs the same check."""
    import sys

    sys.path.insert(0, os.path.join(ROOT, "natten-mps_amd"))
    import build_lib

    objs = [cmd[-1] for cmd in build_lib.commands()[0]]
    if not all(os.path.exists(o) for o in objs):
        pytest.skip("objects not built here (natten-mps_amd/_build)")
    for o in objs:
        assert build_lib.outlined_device_functions(o) == [], o
