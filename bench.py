"""Benchmark of the hot path on one MI355X.

    python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--dilation 1] [--no-cpu] [--no-graph]
                    [--no-split] [--no-all] [--config N] [--causal FF]

Default workload: na2d forward+backward at DiNAT scale (B=16, 56x56, 4 heads,
head dim 32, kernel 7, bf16), BASELINE config 3, the headline; the same JSON
line then carries ``all_configs``: one row per other BASELINE config and
variant (config 1; config 2 non-causal and causal on axis 0; config 3 at
dilation 8; config 4 at dilation 1 and 4; config 5), each with its step time,
TFLOP/s, step HBM-floor fraction, per-kernel launch times, its dominant
kernel's fraction of 8 TB/s and its own CPU baseline (``--no-all`` skips
them).  ``--config N`` runs that config alone (``--dilation`` for configs 3
and 4, ``--causal TF`` for config 2).

A step is one pass through the public API (``natten_mps_amd.na{1,2,3}d``, then
``torch.autograd.grad`` for the configs with a backward) on synthetic seeded
inputs already resident in HBM.  The step is timed eagerly and, captured once
in a HIP graph (torch.cuda.CUDAGraph), as graph replays whose outputs are
checked equal to eager steps; the step time reported is the replay's (the
eager one is in ``config.eager_ms_per_step``, and with torch's autograd
engine kept on the calling thread in
``config.eager_ms_per_step_autograd_one_thread``).  Prints one JSON line:

* value / unit: effective TFLOP/s = (fwd 4*P*D + bwd 10*P*D) / step time,
  with P = B * Hq * (valid query-key pairs of the neighbourhood map);
* roofline: for the kernel with the largest share of GPU time, its
  algorithmic HBM bytes per launch / its mean launch time (HIP events
  bracketing each launch on its stream, over K eager steps that the host
  queues while the GPU spins, so host launch gaps stay out), against 8 TB/s; ``traffic`` is the HBM bytes per launch measured with
  rocprofv3 (FETCH_SIZE x 2 + WRITE_SIZE, calibrated on a copy kernel) for
  the same kernel and workload, read from profiles/traffic.txt when present;
* mfma: useful MFMA throughput of each fused tile kernel (the products it
  needs per valid pair: forward 4·D, dQ 6·D, dK/dV 8·D flops) over its mean
  launch time, against the 2.5 PFLOP/s dense bf16 peak;
* cpu_baseline: the CPU oracle (the reference's pure algorithm) timed on the
  host over the same full workload: forward, forward + backward, and the
  backward as their difference;
* split_path (config 3): the split composition na2d_qk -> softmax -> na2d_av
  (forward + backward) timed eagerly, and its largest absolute difference
  from the fused path's outputs and gradients;
* config.host_us_per_step (config 3): the library's own host time per eager
  step -- the backend's forward and backward calls, timed on the CPU while
  the GPU is held behind a spin (torch's autograd engine excluded).
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "natten-mps_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0
MFMA_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 / fp16
METRIC = "na2d fwd+bwd ms & effective TFLOP/s (56×56,K=7,bf16); % of roofline"

# BASELINE configs
CONFIGS = {
    1: dict(batch=2, spatial=(128,), heads=4, kv_heads=4, dim=32, kernel=(7,), dilation=(1,), causal=(False,),
            dtype="float32", backward=False, seed=1001),
    2: dict(batch=2, spatial=(32, 32), heads=4, kv_heads=4, dim=32, kernel=(7, 7), dilation=(1, 1),
            causal=(False, False), dtype="float32", backward=True, seed=1002),
    3: dict(batch=16, spatial=(56, 56), heads=4, kv_heads=4, dim=32, kernel=(7, 7), dilation=(1, 1),
            causal=(False, False), dtype="bfloat16", backward=True, seed=1003),
    4: dict(batch=4, spatial=(16384,), heads=8, kv_heads=2, dim=64, kernel=(33,), dilation=(1,), causal=(True,),
            dtype="bfloat16", backward=True, seed=1004),
    5: dict(batch=2, spatial=(16, 32, 32), heads=8, kv_heads=8, dim=64, kernel=(3, 7, 7), dilation=(1, 2, 2),
            causal=(False, False, False), dtype="bfloat16", backward=True, seed=1005),
}
DTYPE_TAG = {"float32": "fp32", "bfloat16": "bf16", "float16": "fp16"}


def _log(*a):
    print(*a, file=sys.stderr, flush=True)


def _valid_pairs(spatial, kernel, dilation, causal, device):
    from natten_mps_amd._core import hip

    ones = (1,) * len(spatial)
    _, valid = hip.neighborhood_map(len(spatial), spatial, kernel, dilation, ones, causal, device)
    return int(valid.sum().item())


def kernel_bytes(name, B, N, Hq, Hkv, D, esz, rank=2):
    """Algorithmic HBM bytes of one launch (compulsory traffic: every operand
    read once, every result written once; K/V at Hkv heads; fp32 LSE/delta).
    The dQ tile kernels of 1-D and 2-D problems take delta from their own
    P dP and do not read o; those of 3-D problems read o for delta = dO . o."""
    tq, tkv, lse = B * N * Hq * D * esz, B * N * Hkv * D * esz, B * N * Hq * 4
    fwd = tq + 2 * tkv + tq + lse                 # q, k, v -> out, lse
    bwd_q = tq + 2 * tkv + tq + lse + tq + lse    # q, k, v, dout, lse -> dq, delta
    bwd_q_mfma = bwd_q + (tq if rank == 3 else 0)  # ... 3-D: the tile kernel also reads o
    bwd_kv = tq + 2 * tkv + tq + 2 * lse + 2 * tkv  # q, k, v, dout, lse, delta -> dk, dv
    return {
        "na_forward": fwd, "na_fwd_mfma": fwd, "na_fwd_lean": fwd,
        "na_bwd_dq": bwd_q, "na_bwd_q_mfma": bwd_q_mfma, "na_bwd_q_lean": bwd_q,
        "na_bwd_dkdv": bwd_kv, "na_bwd_kv_mfma": bwd_kv, "na_bwd_kv_lean": bwd_kv,
    }.get(name)


def step_bytes(B, N, Hq, Hkv, D, esz, backward):
    """Compulsory HBM bytes of a step: forward reads q, k, v and writes out,
    lse; backward reads q, k, v, out, dout, lse and writes dq, dk, dv."""
    tq, tkv, lse = B * N * Hq * D * esz, B * N * Hkv * D * esz, B * N * Hq * 4
    fwd = 2 * tq + 2 * tkv + lse
    bwd = 3 * tq + 2 * tkv + lse + tq + 2 * tkv
    return fwd + (bwd if backward else 0)


def copy_bandwidth(torch, nbytes, cycles_per_ms, reps=20):
    """Measured HBM bandwidth of a plain device copy that moves nbytes in
    total (nbytes / 2 read, nbytes / 2 written), the practical ceiling a
    kernel of that many bytes is compared with next to the 8 TB/s spec:
    HIP events around reps copies queued behind a GPU spin."""
    n = max(nbytes // 4, 1)
    src = torch.ones(n, dtype=torch.bfloat16, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    torch.cuda._sleep(int(2.0 * cycles_per_ms))
    a.record()
    for _ in range(reps):
        dst.copy_(src)
    b.record()
    torch.cuda.synchronize()
    return 2 * n * 2 / (a.elapsed_time(b) / reps * 1e-3) / 1e9


def measured_traffic(kernel, workload):
    """HBM bytes per launch from profiles/traffic.txt ("kernel workload bytes")."""
    path = os.path.join(ROOT, "profiles", "traffic.txt")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        for line in f:
            parts = line.split()
            if len(parts) >= 3 and not line.startswith("#") and parts[0] == kernel and parts[1] == workload:
                return int(parts[2])
    return None


def compare_split(leaves, do, cfg, timed, args):
    """The split composition of config 3 (na2d_qk -> softmax -> na2d_av,
    forward + autograd backward) timed like the fused eager step, and its
    largest absolute difference from the fused path (outputs and gradients)."""
    import torch

    from natten_mps_amd import functional as F

    ks, dil = cfg["kernel"], cfg["dilation"]
    scale = cfg["dim"] ** -0.5

    def split_step():
        attn = F.na2d_qk(leaves[0], leaves[1], kernel_size=ks, dilation=dil, scale=scale)
        out = F.na2d_av(attn.softmax(-1), leaves[2], kernel_size=ks, dilation=dil)
        return (out,) + torch.autograd.grad(out, leaves, do)

    def fused_full():
        out = F.na2d(*leaves, kernel_size=ks, dilation=dil)
        return (out,) + torch.autograd.grad(out, leaves, do)

    from natten_mps_amd._core import _lib

    for _ in range(args.warmup):
        split_step()
    ms = timed(split_step)
    # per-launch event timing of the library's kernels (the softmax and its
    # gradient are torch's own), queued behind a spin as for the fused step
    _lib.profile_read(reset=True)
    timed(split_step, profile=True, head_start_ms=2.0 * args.steps * ms + 5.0)
    kernels = {name: round(tot / n * 1e3, 1) for name, (n, tot, _, _) in _lib.profile_read(reset=True).items()}
    # every split launch reads or writes two [B, *sp, H, D] operands and one
    # [B, *sp, H, KV] tensor of logits / weights (algorithmic bytes)
    q = leaves[0]
    kv = ks[0] * ks[1]
    split_bytes = q.numel() * q.element_size() * (2 + kv / q.shape[-1])
    kernel_frac = {name: round(split_bytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 3)
                   for name, us in kernels.items() if name.endswith(("_mfma", "_lean")) and us > 0}
    # the same split step replayed from a HIP graph (checked equal to eager
    # steps, as for the fused step): GPU time without the host's per-op work
    ms_graph = None
    if not args.no_graph:
        try:
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                for _ in range(3):
                    split_step()
            torch.cuda.current_stream().wait_stream(side)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                g_out = split_step()
            ok = True
            for _ in range(3):
                ref = [t.clone() for t in split_step()]
                torch.cuda.synchronize()
                graph.replay()
                torch.cuda.synchronize()
                ok &= all(torch.equal(x, y) for x, y in zip(g_out, ref))
            if ok:
                ms_graph = round(timed(graph.replay, head_start_ms=2.0 * args.steps * max(ms, 0.05) + 5.0), 4)
        except Exception as e:  # an optimisation of the timing, never required
            _log("split-path graph capture failed:", repr(e))
    a, b = fused_full(), split_step()
    diff = max(float((x.detach().float() - y.detach().float()).abs().max()) for x, y in zip(a, b))
    return {"ms_per_step": round(ms, 4), "graph_ms_per_step": ms_graph, "max_abs_diff": diff, "timing": "eager",
            "ops": "na2d_qk -> softmax -> na2d_av, forward + backward", "kernel_mean_us": kernels,
            "kernel_alg_bytes": int(split_bytes), "kernel_hbm_frac": kernel_frac}


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def cpu_baseline(cfg, pairs, budget_s=30.0):
    """The oracle (the reference's pure algorithm, ``oracle/pure.py``: torch
    on the host CPU) over the FULL workload of the config, in the config's
    dtype: the forward alone (no autograd), then forward + backward through
    autograd; the backward is their difference.  GQA K/V are expanded first,
    as the reference's functional layer does before its pure backend
    (``functional.py:27-31,65-71``).  Each figure is the median of the
    timed runs (the first run excluded once there are three), bounded by the
    budget; ``value`` is the forward + backward (or forward-only) rate in
    the metric's unit."""
    import torch

    import oracle.pure as P

    threads = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    torch.set_num_threads(threads)
    rank = len(cfg["spatial"])
    dtype = getattr(torch, cfg["dtype"])
    B, Hq, Hkv, D = cfg["batch"], cfg["heads"], cfg["kv_heads"], cfg["dim"]
    g = torch.Generator().manual_seed(cfg["seed"])

    def make(h):
        return torch.randn((B, *cfg["spatial"], h, D), generator=g).to(dtype)

    q, k, v, do = make(Hq), make(Hkv), make(Hkv), make(Hq)
    fwd = getattr(P, f"na{rank}d_forward")
    rep = Hq // Hkv
    params = (cfg["kernel"], (1,) * rank, cfg["dilation"], cfg["causal"], None)

    def forward(qq, kk, vv):
        if rep != 1:
            kk, vv = kk.repeat_interleave(rep, dim=-2), vv.repeat_interleave(rep, dim=-2)
        return fwd(qq, kk, vv, *params)

    def run_forward():
        with torch.no_grad():
            forward(q, k, v)

    def run_step():
        leaves = [t.detach().requires_grad_(True) for t in (q, k, v)]
        torch.autograd.grad(forward(*leaves), leaves, do)

    def median_time(fn, share):
        times, t_end = [], time.perf_counter() + share
        while not times or (time.perf_counter() < t_end and len(times) < 8):
            t0 = time.perf_counter()
            fn()
            times.append(time.perf_counter() - t0)
        return statistics.median(times[1:] if len(times) >= 3 else times), len(times)

    t_fwd, n_fwd = median_time(run_forward, budget_s / 3)
    fwd_flops = 4.0 * pairs * D
    res = {"unit": "TFLOP/s", "cores": torch.get_num_threads(), "kind": "port",
           "fwd_ms": round(t_fwd * 1e3, 1)}
    if cfg["backward"]:
        t_step, n_step = median_time(run_step, 2 * budget_s / 3)
        res["value"] = 14.0 * pairs * D / t_step / 1e12
        res["step_ms"] = round(t_step * 1e3, 1)
        res["bwd_ms"] = round((t_step - t_fwd) * 1e3, 1)
        timed_runs = f"forward {n_fwd} runs, forward + backward {n_step} runs"
    else:
        res["value"] = fwd_flops / t_fwd / 1e12
        res["step_ms"] = res["fwd_ms"]
        timed_runs = f"{n_fwd} runs"
    res["value"] = round(res["value"], 5)
    res["sample"] = (f"the full workload (batch {B}), oracle/pure.py in {cfg['dtype']} on the host CPU, "
                     f"{threads} torch threads, median of {timed_runs}; CPU: {_cpu_model()}, "
                     f"os.cpu_count()={os.cpu_count()}")
    return res


def rpb_step(torch, steps, warmup):
    """The DiNAT relative-position-bias ops (extras.allin1) on their own: one
    JSON line with the eager step time and each library kernel's mean launch
    time (per-launch events).  Not the headline metric."""
    from natten_mps_amd._core import _lib
    from natten_mps_amd.extras.allin1 import na2d_av_fused, na2d_qk_rpb

    B, X, H, D, K = 16, 56, 4, 32, 7
    g = torch.Generator().manual_seed(0)
    dev = torch.device("cuda:0")
    q, k, v = (torch.randn(B, X, X, H, D, generator=g).to(torch.bfloat16).to(dev) for _ in range(3))
    rpb = torch.randn(H, 2 * K - 1, 2 * K - 1, generator=g).to(torch.bfloat16).to(dev)
    ga = torch.randn(B, X, X, H, K * K, generator=g).to(torch.bfloat16).to(dev)
    go = torch.randn(B, X, X, H, D, generator=g).to(torch.bfloat16).to(dev)

    def step():
        qq, kk, rr = (t.detach().requires_grad_(True) for t in (q, k, rpb))
        logits = na2d_qk_rpb(qq, kk, rr, K, 1, scale=D ** -0.5)
        logits.backward(ga)
        a = logits.detach().softmax(-1).requires_grad_(True)
        vv = v.detach().requires_grad_(True)
        na2d_av_fused(a, vv, K, 1).backward(go)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    _lib.profile_read(reset=True)
    _lib.profile_enable(True)
    try:
        for _ in range(steps):
            step()
        torch.cuda.synchronize()
    finally:
        _lib.profile_enable(False)
    kernels = {name: round(tot / n * 1e3, 1) for name, (n, tot, _, _) in _lib.profile_read(reset=True).items()}
    print(json.dumps({"workload": "extras.allin1 na2d QK+RPB -> softmax -> AV, fwd+bwd, B=16 56x56 heads=4 dim=32 "
                                  "K=7 bf16", "ms_per_step_eager": round(e0.elapsed_time(e1) / steps, 4),
                      "kernel_mean_us": kernels, "kernel_sum_us": round(sum(kernels.values()), 1)}), flush=True)


def host_time_per_step(torch, rank, leaves, do, cfg, steps, cycles_per_ms, blocks=5):
    """Host (CPU) time of the library's own work per eager step: the 'hip'
    backend's forward and backward hooks (argument checks, cached problem
    and layouts, output allocation, the C call), timed on the host in
    ``blocks`` blocks of ``max(steps, 200)`` forward calls then as many
    backward calls, each block while the GPU is held behind a spin so that no
    call waits for the device; the median block of each.  torch's autograd
    engine is not included."""
    from natten_mps_amd._core import _lib, hip

    steps = max(steps, 200)
    q, k, v = (t.detach() for t in leaves)
    ks, dil, causal = cfg["kernel"], cfg["dilation"], cfg["causal"]
    stride = (1,) * rank
    out, lse = hip.forward_with_lse(rank, q, k, v, ks, stride, dil, causal, None)
    hip.fused_backward(rank, do, q, k, v, out, lse, ks, dil, stride, causal, None)
    fwd, bwd = [], []
    for _ in range(blocks):
        torch.cuda.synchronize()
        torch.cuda._sleep(int((steps * 0.05 + 20.0) * cycles_per_ms))
        t0 = time.perf_counter()
        for _ in range(steps):
            hip.forward_with_lse(rank, q, k, v, ks, stride, dil, causal, None)
        t1 = time.perf_counter()
        for _ in range(steps):
            hip.fused_backward(rank, do, q, k, v, out, lse, ks, dil, stride, causal, None)
        t2 = time.perf_counter()
        fwd.append((t1 - t0) / steps * 1e6)
        bwd.append((t2 - t1) / steps * 1e6)
    torch.cuda.synchronize()
    f, b = sorted(fwd)[blocks // 2], sorted(bwd)[blocks // 2]
    return {"forward_us": round(f, 2), "backward_us": round(b, 2), "step_us": round(f + b, 2),
            "blocks": blocks, "calls_per_block": steps,
            "binding": "c++ (_natten_torch.so)" if _lib.binding() is not None else "ctypes"}


def measure(torch, cid, steps, warmup, dilation=None, causal=None, graph=True, split=False, cpu=True,
            cpu_budget=30.0, host=False):
    """One config: eager and graph-replayed step times, per-kernel launch
    times, roofline and MFMA figures, the CPU baseline; the JSON record."""
    import natten_mps_amd
    from natten_mps_amd import functional as F
    from natten_mps_amd._core import _lib

    cfg = dict(CONFIGS[cid])
    rank = len(cfg["spatial"])
    if dilation is not None and cid in (3, 4):
        cfg["dilation"] = (dilation,) * rank
    if causal is not None and cid == 2:
        cfg["causal"] = tuple(c.upper() == "T" for c in causal)
    natten_mps_amd.set_backend("hip")
    dev = torch.device("cuda:0")
    dtype = getattr(torch, cfg["dtype"])
    B, Hq, Hkv, D = cfg["batch"], cfg["heads"], cfg["kv_heads"], cfg["dim"]
    N = 1
    for s in cfg["spatial"]:
        N *= s
    g = torch.Generator().manual_seed(cfg["seed"])

    def make(h):
        return torch.randn((B, *cfg["spatial"], h, D), generator=g).to(dtype).to(dev)

    q, k, v, do = make(Hq), make(Hkv), make(Hkv), make(Hq)
    na = {1: F.na1d, 2: F.na2d, 3: F.na3d}[rank]
    leaves = (q, k, v)
    if cfg["backward"]:
        for t in leaves:
            t.requires_grad_(True)

    def step():
        out = na(q, k, v, kernel_size=cfg["kernel"], dilation=cfg["dilation"], is_causal=cfg["causal"])
        if not cfg["backward"]:
            return (out,)
        return torch.autograd.grad(out, leaves, do)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    _lib.profile_read(reset=True)

    def spin_cycles_per_ms():
        """GPU clock cycles of torch's spin kernel per millisecond."""
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda._sleep(1000)
        a.record()
        torch.cuda._sleep(2_000_000)
        b.record()
        torch.cuda.synchronize()
        return 2_000_000 / max(a.elapsed_time(b), 1e-3)

    cycles_per_ms = spin_cycles_per_ms()

    def timed(run, profile=False, head_start_ms=0.0):
        """Mean GPU time per call of run() over K calls.  With head_start_ms
        the stream first spins that long, so that the host queues the K calls
        while the GPU is busy and no host launch gap falls inside the timed
        region (or inside the per-launch intervals)."""
        _lib.profile_enable(profile)
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        if head_start_ms > 0:
            torch.cuda._sleep(int(head_start_ms * cycles_per_ms))
        start.record()
        for _ in range(steps):
            run()
        stop.record()
        torch.cuda.synchronize()
        _lib.profile_enable(False)
        return start.elapsed_time(stop) / steps

    # eager step time with the per-launch event timing off; the same K steps
    # are then repeated with every library launch bracketed by HIP events on
    # its stream, which gives the per-kernel durations for the roofline.  The
    # host is slower than the GPU on an eager step, so the bracketed pass
    # starts behind a spin long enough for the host to queue all K steps.
    ms_eager = timed(step)
    # The same eager step with torch's autograd engine running backward on
    # the calling thread: the difference is the engine's hand-off to its
    # per-device worker thread and back (thread wake-ups on the host), not
    # work of this library.
    ms_eager_one_thread = None
    if cfg["backward"]:
        torch.autograd.set_multithreading_enabled(False)
        try:
            ms_eager_one_thread = timed(step)
        finally:
            torch.autograd.set_multithreading_enabled(True)
    ms_profiled = timed(step, profile=True, head_start_ms=2.0 * steps * ms_eager + 5.0)
    stats = _lib.profile_read(reset=True)
    _log(f"[config {cid}] eager step {ms_eager:.4f} ms (queued ahead, with per-launch events: {ms_profiled:.4f} ms)")
    if ms_eager_one_thread is not None:
        _log(f"[config {cid}] eager step with autograd on the calling thread {ms_eager_one_thread:.4f} ms")

    # the same step captured once in a HIP graph (forward + autograd backward)
    # and replayed: identical kernels and buffers without the per-step host
    # work.  Every replay is checked bit for bit against an eager step, with
    # eager work and synchronisation between the replays.
    ms_graph = None
    if graph:
        try:
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                for _ in range(3):
                    step()
            torch.cuda.current_stream().wait_stream(side)
            cg = torch.cuda.CUDAGraph()
            with torch.cuda.graph(cg):
                g_out = step()
            ref = [t.clone() for t in step()]
            graph_ok = True
            for _ in range(3):
                cg.replay()
                torch.cuda.synchronize()
                graph_ok &= all(torch.equal(a, b) for a, b in zip(g_out, ref))
                ref = [t.clone() for t in step()]
                torch.cuda.synchronize()
            if graph_ok:
                # replays queued behind a spin, so that the host's graph
                # launch cost (tens of µs) stays out of a short step's time
                ms_graph = timed(cg.replay, head_start_ms=2.0 * steps * max(ms_eager, 0.05) + 5.0)
                _log(f"[config {cid}] graph step {ms_graph:.4f} ms")
            else:
                _log(f"[config {cid}] graph replay differs from the eager step; reporting the eager time")
        except Exception as e:  # capture is an optimisation of the timing, never required
            _log(f"[config {cid}] graph capture failed:", repr(e))
    ms = ms_graph if ms_graph is not None else ms_eager

    pairs = B * Hq * _valid_pairs(cfg["spatial"], cfg["kernel"], cfg["dilation"], cfg["causal"], dev)
    flops = (14.0 if cfg["backward"] else 4.0) * pairs * D
    tflops = flops / (ms * 1e-3) / 1e12
    esz = torch.tensor([], dtype=dtype).element_size()
    sbytes = step_bytes(B, N, Hq, Hkv, D, esz, cfg["backward"])

    gpu_total = sum(st[1] for st in stats.values())
    for name, (n, tot, mn, mx) in sorted(stats.items(), key=lambda kv: -kv[1][1]):
        _log(f"  {name:14s} launches={n:4d} mean={tot / n * 1e3:8.1f} us  min={mn * 1e3:8.1f}  max={mx * 1e3:8.1f}"
             f"  share={tot / gpu_total:5.1%}")
    kernel_mean_us = {name: round(tot / n * 1e3, 2) for name, (n, tot, _, _) in stats.items()}
    dils = [str(d) for d in cfg["dilation"]]
    dil_tag = dils[0] if len(set(dils)) == 1 else "x".join(dils)
    workload = f"config{cid}_d{dil_tag}"
    dom_name, (dn, dtot, _, _) = max(stats.items(), key=lambda kv: kv[1][1])
    nbytes = kernel_bytes(dom_name, B, N, Hq, Hkv, D, esz, rank)
    mean_s = dtot / dn * 1e-3
    roof = None
    if nbytes is not None:
        gbs = nbytes / mean_s / 1e9
        copy_gbs = copy_bandwidth(torch, nbytes, cycles_per_ms)
        roof = {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": measured_traffic(dom_name, workload),
                "kernel": dom_name, "mean_us": round(mean_s * 1e6, 2), "alg_bytes": nbytes,
                "copy_gbs": round(copy_gbs, 1), "frac_of_copy": round(gbs / copy_gbs, 4)}
        _log(f"[config {cid}] device copy moving the kernel's {nbytes / 1e6:.1f} MB: {copy_gbs:.0f} GB/s "
             f"({copy_gbs / HBM_PEAK_GBS:.1%} of 8 TB/s); {dom_name} reaches {gbs / copy_gbs:.1%} of it")
    # MFMA utilisation of the fused tile kernels, on useful work: the MFMA
    # products each kernel needs per valid (query, key) pair and head dim --
    # forward q.k and p.v (4 flops), dQ kernel q.k, dO.v, dS.k (6), dK/dV
    # kernel q.k, dO.v, p.dO, dS.q (8) -- over its mean launch time, against
    # the dense bf16/fp16 MFMA peak.  (The tiles also compute the masked
    # pairs of their unions; those executed flops are in the counter
    # profiles, not here.)
    mfma = None
    per_pair = {"na_fwd_mfma": 4.0, "na_bwd_q_mfma": 6.0, "na_bwd_kv_mfma": 8.0,
                "na_fwd_lean": 4.0, "na_bwd_q_lean": 6.0, "na_bwd_kv_lean": 8.0}
    if dtype != torch.float32:
        kern = {}
        for name, (n, tot, _, _) in stats.items():
            if name in per_pair:
                t = tot / n * 1e-3
                useful = per_pair[name] * pairs * D / t / 1e12
                kern[name] = {"useful_tflops": round(useful, 2), "frac": round(useful / MFMA_PEAK_TFLOPS, 4),
                              "mean_us": round(t * 1e6, 2)}
        mfma = {"peak_tflops": MFMA_PEAK_TFLOPS, "useful_tflops_step": round(tflops, 2),
                "useful_frac_step": round(tflops / MFMA_PEAK_TFLOPS, 4), "kernels": kern}
    _log(f"[config {cid}] step {ms:.4f} ms  {tflops:.2f} TFLOP/s  {sbytes / (ms * 1e-3) / 1e9:.0f} GB/s  "
         f"HBM floor {sbytes / 8e12 * 1e6:.1f} us -> {sbytes / 8e12 / (ms * 1e-3):.1%} of roofline (step)")

    # config 3 asks for the fused path against the split composition
    # na2d_qk -> softmax -> na2d_av (forward and backward through autograd):
    # its step time (eager, queued ahead like the fused eager step) and the
    # largest difference between the two paths' outputs and gradients
    split_path = None
    if split and cid == 3:
        try:
            ns = argparse.Namespace(steps=steps, warmup=warmup, no_graph=not graph)
            split_path = compare_split(leaves, do, cfg, timed, ns)
            _log(f"split path step {split_path['ms_per_step']:.4f} ms eager, {split_path['graph_ms_per_step']} ms "
                 f"graph, max |fused - split| {split_path['max_abs_diff']:.3g}")
        except Exception as e:  # a comparison, never required
            _log("split comparison failed:", repr(e))

    host_us = None
    if host and cfg["backward"]:
        try:
            host_us = host_time_per_step(torch, rank, leaves, do, cfg, steps, cycles_per_ms)
            _log(f"[config {cid}] library host time per step: {host_us}")
        except Exception as e:  # reported, never required
            _log("host timing failed:", repr(e))

    cpu_rec = None
    if cpu:
        try:
            cpu_rec = cpu_baseline(cfg, pairs, budget_s=cpu_budget)
            _log(f"[config {cid}] cpu baseline: forward {cpu_rec['fwd_ms']} ms, step {cpu_rec['step_ms']} ms, "
                 f"{cpu_rec['value']} TFLOP/s ({cpu_rec['cores']} threads)")
        except Exception as e:  # the baseline is reported, never required
            _log("cpu baseline failed:", repr(e))

    shape = "x".join(str(s) for s in cfg["spatial"])
    causal_tag = "".join("T" if c else "F" for c in cfg["causal"])
    desc = (f"na{rank}d {'fwd+bwd' if cfg['backward'] else 'fwd'} B={B} {shape} heads={Hq}/{Hkv} dim={D} "
            f"K={cfg['kernel']} dilation={cfg['dilation']} causal={causal_tag} {DTYPE_TAG[cfg['dtype']]} "
            f"(BASELINE config {cid})")
    return {
        "metric": METRIC if cid == 3 else f"na{rank}d step ms & effective TFLOP/s (config {cid})",
        "value": round(tflops, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": DTYPE_TAG[cfg["dtype"]],
        "data": "synthetic (seeded randn, resident in HBM)",
        "config": {"workload": desc, "global_batch": B, "seq_len": N, "parallelism": "single GPU",
                   "timing": "HIP graph replay of the eager step (checked equal)" if ms_graph is not None
                   else "eager", "eager_ms_per_step": round(ms_eager, 4),
                   "eager_ms_per_step_autograd_one_thread": None if ms_eager_one_thread is None
                   else round(ms_eager_one_thread, 4),
                   "host_us_per_step": host_us,
                   "step_hbm_bytes": sbytes, "step_gbs": round(sbytes / (ms * 1e-3) / 1e9, 1),
                   "hbm_floor_frac_step": round(sbytes / 8e12 / (ms * 1e-3), 4),
                   "kernel_mean_us": kernel_mean_us},
        "roofline": roof,
        "mfma": mfma,
        "cpu_baseline": cpu_rec,
        "split_path": split_path,
    }


# The rows beside the headline (config 3, dilation 1) in the default run:
# every BASELINE config and variant, each with its own CPU baseline.
OTHER_ROWS = [(1, {}), (2, {"causal": "FF"}), (2, {"causal": "TF"}), (3, {"dilation": 8}), (4, {"dilation": 1}),
              (4, {"dilation": 4}), (5, {})]


def summary(rec):
    """The per-config fields of an all_configs row."""
    roof = rec["roofline"] or {}
    return {"workload": rec["config"]["workload"], "ms_per_step": rec["ms_per_step"],
            "timing": rec["config"]["timing"], "eager_ms_per_step": rec["config"]["eager_ms_per_step"],
            "tflops": rec["value"], "hbm_floor_frac_step": rec["config"]["hbm_floor_frac_step"],
            "kernel_mean_us": rec["config"]["kernel_mean_us"],
            "dominant_kernel": roof.get("kernel"), "dominant_frac": roof.get("frac"),
            "dominant_frac_of_copy": roof.get("frac_of_copy"),
            "mfma_useful_frac_step": (rec["mfma"] or {}).get("useful_frac_step"),
            "cpu_baseline": rec["cpu_baseline"]}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", type=int, default=None, choices=sorted(CONFIGS),
                    help="only this config (default: the headline, config 3, plus a row per config)")
    ap.add_argument("--dilation", type=int, default=None, help="dilation of configs 3 and 4 (default 1)")
    ap.add_argument("--causal", default=None, help="config 2 causal flags, e.g. TF")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-graph", action="store_true", help="time eager steps only")
    ap.add_argument("--no-split", action="store_true", help="skip the split-path comparison of config 3")
    ap.add_argument("--no-all", action="store_true", help="the headline config only, no per-config rows")
    ap.add_argument("--copy-probe", type=float, default=None, metavar="MB",
                    help="only run device-to-device copies of this many MB (calibrates rocprofv3 byte counters)")
    ap.add_argument("--rpb", action="store_true",
                    help="only time the extras.allin1 QK+RPB -> softmax -> AV step at DiNAT scale "
                         "(B=16, 56x56, 4 heads, dim 32, K=7, bf16), forward + backward")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (got --gpus {args.gpus}); every GPU box of this "
              "pool has one GPU, and no multi-GPU figure is measured.", file=sys.stderr)
        sys.exit(2)

    import torch

    if args.copy_probe is not None:
        # a plain copy of known size: its FETCH_SIZE / WRITE_SIZE per dispatch
        # give the factors that turn those counters into HBM bytes
        n = int(args.copy_probe * 1e6) // 2
        src = torch.randn(n, device="cuda:0").to(torch.bfloat16)
        dst = torch.empty_like(src)
        for _ in range(args.steps):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_probe_bytes": 2 * n, "copies": args.steps}), flush=True)
        return

    if args.rpb:
        rpb_step(torch, args.steps, args.warmup)
        return

    cid = 3 if args.config is None else args.config
    rec = measure(torch, cid, args.steps, args.warmup, dilation=args.dilation, causal=args.causal,
                  graph=not args.no_graph, split=not args.no_split, cpu=not args.no_cpu, host=cid == 3)
    if args.config is None and not args.no_all:
        rows = []
        for other, kw in OTHER_ROWS:
            try:
                r = measure(torch, other, min(args.steps, 10), min(args.warmup, 3), graph=not args.no_graph,
                            cpu=not args.no_cpu, cpu_budget=6.0, **kw)
                rows.append(summary(r))
            except Exception as e:  # a row that fails is reported as such, never fatal
                rows.append({"config": other, **kw, "error": repr(e)})
        rec["all_configs"] = rows
    print(json.dumps(rec), flush=True)


if __name__ == "__main__":
    main()
