"""Fused forward + backward captured in a HIP graph (``torch.cuda.graph``) and
replayed, through the 'hip' backend's host binding.

* warm: the step runs eagerly first (on a side stream, as torch asks before a
  capture), so the call signatures and the tile geometry tables exist and
  their uploads are seen complete; the graph then holds the same kernels as
  the eager step, and every replay must equal an eager step bit for bit.
* cold: a shape captured before any eager call. Under capture the library
  builds no geometry table (that needs an allocation and a host-to-device
  copy) and queries no upload event, so the graph holds the tile kernels
  that compute their geometry themselves; the eager step afterwards may take
  the table-driven kernels.
  Replays must equal each other bit for bit and the eager step within the
  half-precision bound of ``tests/_parity.py``.

Each replay is followed by eager work and a synchronisation, and the graph's
outputs are checked after every replay.  The library records no memset
nodes: the only zero-fill (dq where stride > 1 leaves non-query positions)
is a torch fill kernel.
"""
from __future__ import annotations

import pytest
import torch

from _parity import assert_parity

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0") if torch.cuda.is_available() else None

# name: rank, spatial, heads q / kv, dim, kernel, dilation, causal, stride, dtype
CASES = {
    "lean2d_bf16": (2, (2, 24, 20), 2, 2, 32, (7, 7), (1, 1), (False, False), (1, 1), torch.bfloat16),
    "lean2d_fp32": (2, (1, 20, 18), 2, 2, 32, (5, 5), (1, 2), (False, True), (1, 1), torch.float32),
    "gqa1d_causal": (1, (2, 300), 4, 2, 64, (9,), (2,), (True,), (1,), torch.bfloat16),
    "tiles3d": (3, (1, 6, 10, 12), 2, 2, 32, (3, 5, 5), (1, 2, 1), (False, False, False), (1, 1, 1),
                torch.float16),
    "strided2d": (2, (1, 18, 20), 2, 2, 32, (5, 5), (1, 1), (False, False), (2, 1), torch.bfloat16),
}


@pytest.fixture(autouse=True)
def _hip():
    import natten_mps_amd

    natten_mps_amd.set_backend("hip")


def _step_fn(case, seed, spatial=None):
    from natten_mps_amd import functional as F

    rank, sp, hq, hkv, dim, ks, dil, causal, stride, dtype = CASES[case]
    sp = spatial or sp
    g = torch.Generator().manual_seed(seed)
    mk = lambda h: torch.randn((*sp, h, dim), generator=g).to(dtype).to(DEV)  # noqa: E731
    q, k, v = mk(hq), mk(hkv), mk(hkv)
    leaves = [t.requires_grad_(True) for t in (q, k, v)]
    fn = {1: F.na1d, 2: F.na2d, 3: F.na3d}[rank]
    out_sp = tuple((n + st - 1) // st for n, st in zip(sp[1:], stride))
    do = torch.randn((sp[0], *out_sp, hq, dim), generator=g).to(dtype).to(DEV)

    def step():
        out = fn(*leaves, kernel_size=ks, stride=stride, dilation=dil, is_causal=causal)
        return [out.detach()] + list(torch.autograd.grad(out, leaves, do))

    return step, dtype


def _capture(step, warm):
    if warm:
        # the warm-up on a side stream; the last call, after a synchronisation,
        # sees the geometry tables' uploads complete
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(2):
                step()
            torch.cuda.synchronize()
            step()
        torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = step()
    torch.cuda.synchronize()
    return graph, outs


@pytest.mark.parametrize("case", sorted(CASES))
def test_graph_replay_equals_eager_step(case):
    step, _ = _step_fn(case, 700 + sorted(CASES).index(case))
    graph, outs = _capture(step, warm=True)
    for i in range(3):
        ref = [t.clone() for t in step()]
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for name, a, b in zip(("out", "dq", "dk", "dv"), outs, ref):
            assert torch.equal(a, b), f"{case} replay {i}: {name} differs from the eager step"


@pytest.mark.parametrize("case", ["lean2d_bf16", "tiles3d"])
def test_graph_captured_before_any_eager_call(case):
    # a spatial extent no other test uses, so no geometry table exists yet
    sp = {"lean2d_bf16": (1, 26, 22), "tiles3d": (1, 7, 11, 13)}[case]
    step, dtype = _step_fn(case, 800 + len(case), spatial=sp)
    graph, outs = _capture(step, warm=False)
    first = None
    for i in range(3):
        graph.replay()
        torch.cuda.synchronize()
        got = [t.clone() for t in outs]
        if first is None:
            first = got
        else:
            for name, a, b in zip(("out", "dq", "dk", "dv"), got, first):
                assert torch.equal(a, b), f"{case} replay {i}: {name} differs from the first replay"
        ref = step()
        torch.cuda.synchronize()
        for name, a, b in zip(("out", "dq", "dk", "dv"), got, ref):
            assert_parity(a, b, dtype, f"{case} replay {i} {name}")
