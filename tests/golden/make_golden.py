"""Write the golden vectors in tests/golden/ from the reference itself.

Run in the build container only (the reference is not on the GPU box):

    python tests/golden/make_golden.py /root/reference/src

It imports the reference's pure backend and functional API (CPU, torch) and
records inputs and outputs for small seeded cases:

* ``fwd_*``   -- ``_core/pure.py`` fused forward (fp32 and bf16) + autograd grads
* ``qk_*`` / ``av_*`` -- split ops, with and without scale
* ``maps_*``  -- ``_build_2d_neighborhood`` / ``_build_3d_neighborhood`` /
  ``_causal_1d_indices`` and the window starts of ``utils/window.py``
* ``func_*``  -- ``functional.na{1,2,3}d`` on the pure backend: GQA,
  ``return_lse``, ``additional_keys`` (+ merge), and their gradients
* ``cfg1``    -- BASELINE config 1 (na1d fp32 B=2 L=128 h=4 D=32 K=7, seed 1001)

Outputs: ``golden.npz`` (arrays; bf16 kept as raw uint16 bits, int64 maps as int32) and
``golden.json`` (the case list: op, rank, parameters, dtype, array keys).

With ``--allin1`` it writes ``allin1.npz`` / ``allin1.json`` instead: the
reference's ``extras/allin1`` ops through its public functions
(``na{1,2}d_qk_rpb``, ``na{1,2}d_av_fused``; on the CPU these take the pure
torch path of ``extras/allin1/functional.py:47-325`` and its autograd
fallback), fp32, odd and even kernels, dilation 1 and > 1, 1-D and 2-D,
with a random bias and with none: logits, dq, dk, drpb for the QK+RPB op,
out, dattn, dv for the AV op.
"""
from __future__ import annotations

import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def _gen(seed):
    return torch.Generator().manual_seed(seed)


def _randn(g, shape, dtype):
    return torch.randn(shape, generator=g, dtype=torch.float32).to(dtype)


def main(ref_src: str) -> None:
    sys.path.insert(0, ref_src)
    os.environ["NATTEN_BACKEND"] = "pure"
    import natten_mps
    from natten_mps import functional as RF
    from natten_mps._core import pure as RP
    from natten_mps.utils import window as RW

    natten_mps.set_backend("pure")
    arrays: dict[str, np.ndarray] = {}
    cases: list[dict] = []

    def put(key, t):
        t = t.detach()
        if t.dtype == torch.bfloat16:
            arrays[key] = t.view(torch.int16).numpy().view(np.uint16)  # raw bf16 bits
        elif t.is_floating_point():
            arrays[key] = t.to(torch.float32).numpy()
        elif t.dtype == torch.long and t.numel() and int(t.abs().max()) < 2**31:
            arrays[key] = t.to(torch.int32).numpy()
        else:
            arrays[key] = t.numpy()
        return key

    # bf16 arrays are stored as their uint16 bit patterns (see golden.json "dtype")

    # -- fused forward + autograd grads ---------------------------------
    fwd_cases = [
        # rank, spatial, heads, dim, kernel, stride, dilation, causal, scale, dtype
        (1, (24,), 2, 8, (5,), (1,), (1,), (False,), None, "float32"),
        (1, (24,), 2, 8, (5,), (1,), (3,), (False,), None, "float32"),
        (1, (24,), 2, 8, (7,), (1,), (2,), (True,), 0.3, "float32"),
        (1, (23,), 2, 8, (5,), (2,), (1,), (False,), None, "float32"),
        (1, (23,), 2, 8, (5,), (3,), (2,), (True,), None, "float32"),
        (1, (16,), 2, 8, (4,), (1,), (1,), (False,), None, "float32"),
        (2, (10, 12), 2, 8, (3, 5), (1, 1), (1, 2), (False, False), None, "float32"),
        (2, (10, 12), 2, 8, (5, 5), (1, 1), (2, 1), (True, False), None, "float32"),
        (2, (10, 12), 2, 8, (3, 3), (2, 1), (1, 1), (False, True), None, "float32"),
        (2, (9, 11), 2, 8, (3, 5), (2, 3), (1, 2), (True, True), 0.5, "float32"),
        (2, (12, 12), 2, 16, (7, 7), (1, 1), (1, 1), (False, False), None, "bfloat16"),
        (2, (12, 12), 2, 16, (3, 3), (1, 1), (4, 4), (True, False), None, "bfloat16"),
        (3, (5, 6, 7), 2, 8, (3, 3, 5), (1, 1, 1), (1, 2, 1), (False, False, False), None, "float32"),
        (3, (6, 5, 6), 2, 8, (3, 3, 3), (1, 2, 1), (2, 1, 1), (False, True, False), None, "float32"),
        (3, (5, 6, 7), 2, 8, (3, 3, 3), (1, 1, 2), (1, 1, 2), (True, True, True), None, "float32"),
        (3, (4, 6, 6), 2, 8, (3, 5, 5), (1, 1, 1), (1, 1, 1), (False, False, False), None, "bfloat16"),
    ]
    for ci, (rank, sp, heads, dim, ks, st, dil, causal, scale, dt) in enumerate(fwd_cases):
        dtype = getattr(torch, dt)
        g = _gen(2000 + ci)
        shape = (2, *sp, heads, dim)
        q, k, v = (_randn(g, shape, dtype) for _ in range(3))
        qg, kg, vg = (t.clone().requires_grad_(True) for t in (q, k, v))
        fn = getattr(RP, f"na{rank}d_forward")
        out = fn(qg, kg, vg, ks, st, dil, causal, scale)
        do = _randn(g, tuple(out.shape), dtype)
        dq, dk, dv = torch.autograd.grad(out, (qg, kg, vg), do)
        p = f"fwd{ci}/"
        cases.append(dict(
            kind="fwd", key=p, rank=rank, spatial=list(sp), kernel_size=list(ks), stride=list(st),
            dilation=list(dil), is_causal=list(causal), scale=scale, dtype=dt,
            arrays=[put(p + n, t) for n, t in
                    (("q", q), ("k", k), ("v", v), ("out", out), ("dout", do), ("dq", dq), ("dk", dk), ("dv", dv))],
        ))

    # -- split QK / AV ---------------------------------------------------
    split_cases = [
        (1, (20,), (5,), (2,), (1,), (False,), None),
        (1, (21,), (5,), (1,), (2,), (True,), 0.25),
        (2, (9, 10), (3, 5), (1, 2), (1, 1), (True, False), None),
        (2, (9, 10), (3, 3), (1, 1), (2, 2), (False, False), 0.7),
        (3, (4, 6, 5), (3, 3, 3), (1, 2, 1), (1, 1, 2), (False, False, True), None),
    ]
    for ci, (rank, sp, ks, dil, st, causal, scale) in enumerate(split_cases):
        g = _gen(3000 + ci)
        shape = (2, *sp, 2, 8)
        q, k, v = (_randn(g, shape, torch.float32) for _ in range(3))
        qg, kg = q.clone().requires_grad_(True), k.clone().requires_grad_(True)
        logits = getattr(RP, f"na{rank}d_qk_forward")(qg, kg, ks, dil, st, causal, scale)
        dlog = _randn(g, tuple(logits.shape), torch.float32)
        dlog_f = torch.where(torch.isfinite(logits), dlog, torch.zeros_like(dlog))
        dq, dk = torch.autograd.grad(logits, (qg, kg), dlog_f)
        attn = torch.softmax(_randn(g, tuple(logits.shape), torch.float32), dim=-1)
        ag, vg = attn.clone().requires_grad_(True), v.clone().requires_grad_(True)
        out = getattr(RP, f"na{rank}d_av_forward")(ag, vg, ks, dil, st, causal)
        do = _randn(g, tuple(out.shape), torch.float32)
        da, dv = torch.autograd.grad(out, (ag, vg), do)
        p = f"split{ci}/"
        cases.append(dict(
            kind="split", key=p, rank=rank, spatial=list(sp), kernel_size=list(ks), stride=list(st),
            dilation=list(dil), is_causal=list(causal), scale=scale, dtype="float32",
            arrays=[put(p + n, t) for n, t in
                    (("q", q), ("k", k), ("v", v), ("logits", logits), ("dlogits", dlog_f), ("dq", dq),
                     ("dk", dk), ("attn", attn), ("out", out), ("dout", do), ("dattn", da), ("dv", dv))],
        ))

    # -- index maps and window starts -----------------------------------
    map_cases = [
        (2, (10, 12), (3, 5), (1, 2), (1, 1), (False, False)),
        (2, (10, 12), (5, 3), (2, 1), (2, 3), (True, False)),
        (2, (56, 56), (7, 7), (8, 8), (1, 1), (False, False)),
        (3, (6, 7, 8), (3, 3, 5), (1, 2, 1), (1, 1, 2), (False, True, False)),
        (3, (16, 32, 32), (3, 7, 7), (1, 2, 2), (1, 1, 1), (False, False, False)),
    ]
    for ci, (rank, sp, ks, dil, st, causal) in enumerate(map_cases):
        pos = [RP._output_positions(n, s, torch.device("cpu")) for n, s in zip(sp, st)]
        if rank == 2:
            flat, valid = RP._build_2d_neighborhood(pos[0], pos[1], sp[0], sp[1], ks, dil, causal, torch.device("cpu"))
        else:
            flat, valid = RP._build_3d_neighborhood(pos[0], pos[1], pos[2], *sp, ks, dil, causal, torch.device("cpu"))
        p = f"maps{ci}/"
        if flat.numel() > 200_000:
            # large maps: sha256 of the int64 little-endian bytes + a strided sample
            import hashlib
            digest = hashlib.sha256(flat.contiguous().numpy().astype("<i8").tobytes()).hexdigest()
            step = flat.numel() // 4093
            cases.append(dict(kind="map_digest", key=p, rank=rank, spatial=list(sp), kernel_size=list(ks),
                              stride=list(st), dilation=list(dil), is_causal=list(causal), sha256=digest,
                              sample_step=step, arrays=[put(p + "sample", flat.reshape(-1)[::step])]))
            continue
        keys = [put(p + "flat", flat)]
        if valid is not None:
            keys.append(put(p + "valid", valid.to(torch.uint8)))
        cases.append(dict(kind="map", key=p, rank=rank, spatial=list(sp), kernel_size=list(ks), stride=list(st),
                          dilation=list(dil), is_causal=list(causal), arrays=keys))
    pos = torch.arange(40)
    idx, valid = RP._causal_1d_indices(pos, 40, 9, 3, torch.device("cpu"))
    cases.append(dict(kind="map1d_causal", key="mapc/", length=40, kernel=9, dilation=3,
                      arrays=[put("mapc/idx", idx), put("mapc/valid", valid.to(torch.uint8))]))
    starts = []
    for L in range(1, 25):
        for K in range(1, L + 1):
            for d in range(1, L // K + 1):
                for i in range(L):
                    starts.append((L, K, d, i, RW.get_window_start(i, L, K, d)))
    st_arr = torch.tensor(starts, dtype=torch.int16)
    vec = []
    for L in (17, 56):
        for K in (3, 4, 7):
            for d in (1, 2, 3, 8):
                if d * K <= L:
                    vec.append(RW.get_window_start_vectorized(torch.arange(L), L, K, d))
    cases.append(dict(kind="starts", key="starts/", arrays=[put("starts/table", st_arr),
                                                             put("starts/vec", torch.cat(vec))]))

    # -- functional layer on the pure backend ----------------------------
    func_cases = [
        # rank, spatial, hq, hkv, dim, ks, st, dil, causal, return_lse, n_extra
        (1, (20,), 4, 2, 8, 5, 1, 1, False, True, 0),
        (2, (9, 10), 4, 1, 8, (3, 5), 1, (1, 2), (False, True), True, 0),
        (2, (9, 10), 2, 2, 8, 3, 1, 1, False, False, 2),
        (2, (9, 10), 4, 2, 8, 3, 1, 2, False, True, 1),
        (3, (5, 6, 7), 2, 2, 8, 3, 1, 1, (True, False, False), True, 0),
        (1, (20,), 4, 4, 8, 5, 2, 1, True, False, 0),
        (2, (6, 6), 2, 2, 8, 6, 1, 1, False, True, 0),
    ]
    for ci, (rank, sp, hq, hkv, dim, ks, st, dil, causal, rlse, n_extra) in enumerate(func_cases):
        g = _gen(4000 + ci)
        q = _randn(g, (2, *sp, hq, dim), torch.float32)
        k = _randn(g, (2, *sp, hkv, dim), torch.float32)
        v = _randn(g, (2, *sp, hkv, dim), torch.float32)
        ak = av = None
        if n_extra:
            ak = _randn(g, (2, n_extra, hkv, dim), torch.float32)
            av = _randn(g, (2, n_extra, hkv, dim), torch.float32)
        leaves = [t.clone().requires_grad_(True) for t in (q, k, v)]
        extra = [t.clone().requires_grad_(True) for t in (ak, av)] if n_extra else [None, None]
        fn = getattr(RF, f"na{rank}d")
        res = fn(*leaves, kernel_size=ks, stride=st, dilation=dil, is_causal=causal,
                 return_lse=rlse, additional_keys=extra[0], additional_values=extra[1])
        out, lse = (res if rlse else (res, None))
        do = _randn(g, tuple(out.shape), torch.float32)
        loss_terms = [(out, do)]
        dl = None
        if rlse:
            dl = _randn(g, tuple(lse.shape), torch.float32)
            loss_terms.append((lse, dl))
        wrt = leaves + ([extra[0], extra[1]] if n_extra else [])
        grads = torch.autograd.grad([t for t, _ in loss_terms], wrt, [gd for _, gd in loss_terms])
        p = f"func{ci}/"
        named = [("q", q), ("k", k), ("v", v), ("out", out), ("dout", do), ("dq", grads[0]),
                 ("dk", grads[1]), ("dv", grads[2])]
        if rlse:
            named += [("lse", lse), ("dlse", dl)]
        if n_extra:
            named += [("ak", ak), ("av", av), ("dak", grads[3]), ("dav", grads[4])]
        cases.append(dict(
            kind="func", key=p, rank=rank, spatial=list(sp), heads_q=hq, heads_kv=hkv, dim=dim,
            kernel_size=ks if isinstance(ks, int) else list(ks), stride=st,
            dilation=dil if isinstance(dil, int) else list(dil),
            is_causal=causal if isinstance(causal, bool) else list(causal),
            return_lse=rlse, n_extra=n_extra, dtype="float32",
            arrays=[put(p + n, t) for n, t in named],
        ))

    # -- BASELINE config 1 -------------------------------------------------
    g = _gen(1001)
    q, k, v = (_randn(g, (2, 128, 4, 32), torch.float32) for _ in range(3))
    out = RP.na1d_forward(q, k, v, (7,), (1,), (1,), (False,), 32 ** -0.5)
    cases.append(dict(kind="cfg1", key="cfg1/", seed=1001, arrays=[put("cfg1/out", out)]))

    np.savez_compressed(os.path.join(HERE, "golden.npz"), **arrays)
    with open(os.path.join(HERE, "golden.json"), "w") as f:
        json.dump(dict(torch_version=torch.__version__, reference="natten_mps " + natten_mps.__version__,
                       cases=cases), f, indent=1)
    print(f"wrote {len(cases)} cases, {len(arrays)} arrays")


# rank, spatial, heads, dim, kernel, dilation, with a bias, scale
ALLIN1_CASES = [
    (1, (24,), 2, 8, 5, 1, True, 0.5),
    (1, (24,), 2, 8, 4, 2, True, None),
    (1, (23,), 3, 8, 7, 3, True, 0.3),
    (1, (16,), 2, 8, 2, 1, True, None),
    (1, (18,), 2, 8, 6, 3, False, 0.4),
    (2, (10, 12), 2, 8, 3, 2, True, 0.5),
    (2, (9, 11), 2, 8, 4, 1, True, None),
    (2, (12, 10), 2, 8, 4, 2, True, 0.3),
    (2, (11, 13), 2, 8, 5, 2, False, None),
    (2, (7, 8), 2, 8, 6, 1, True, 0.25),
]


def main_allin1(ref_src: str) -> None:
    sys.path.insert(0, ref_src)
    import natten_mps
    from natten_mps.extras import allin1 as RA

    arrays: dict[str, np.ndarray] = {}
    cases: list[dict] = []
    for ci, (rank, sp, heads, dim, K, dil, with_rpb, scale) in enumerate(ALLIN1_CASES):
        g = _gen(7000 + ci)
        q = _randn(g, (2, *sp, heads, dim), torch.float32)
        k = _randn(g, (2, *sp, heads, dim), torch.float32)
        v = _randn(g, (2, *sp, heads, dim), torch.float32)
        rpb = _randn(g, (heads, *([2 * K - 1] * rank)), torch.float32) if with_rpb else None
        kv = K ** rank
        dlog = _randn(g, (2, *sp, heads, kv), torch.float32)
        dout = _randn(g, (2, *sp, heads, dim), torch.float32)
        ql, kl = q.clone().requires_grad_(True), k.clone().requires_grad_(True)
        rl = rpb.clone().requires_grad_(True) if with_rpb else None
        qk = RA.na1d_qk_rpb if rank == 1 else RA.na2d_qk_rpb
        av = RA.na1d_av_fused if rank == 1 else RA.na2d_av_fused
        logits = qk(ql, kl, rl, K, dil, scale=scale)
        wrt = [ql, kl] + ([rl] if with_rpb else [])
        g_qk = torch.autograd.grad(logits, wrt, dlog)
        # the AV op on softmax-normalised weights of the same logits (masked
        # entries are -inf, so their weights are 0)
        attn = torch.softmax(logits.detach(), -1)
        al, vl = attn.clone().requires_grad_(True), v.clone().requires_grad_(True)
        out = av(al, vl, K, dil)
        g_av = torch.autograd.grad(out, [al, vl], dout)
        p = f"allin1_{ci}/"
        named = [("q", q), ("k", k), ("v", v), ("dlogits", dlog), ("dout", dout), ("logits", logits),
                 ("dq", g_qk[0]), ("dk", g_qk[1]), ("attn", attn), ("out", out), ("dattn", g_av[0]),
                 ("dv", g_av[1])]
        if with_rpb:
            named += [("rpb", rpb), ("drpb", g_qk[2])]
        cases.append(dict(kind="allin1", key=p, rank=rank, spatial=list(sp), heads=heads, dim=dim,
                          kernel_size=K, dilation=dil, with_rpb=with_rpb, scale=scale, dtype="float32",
                          arrays=[p + n for n, _ in named]))
        for n, t in named:
            arrays[p + n] = t.detach().to(torch.float32).numpy()

    np.savez_compressed(os.path.join(HERE, "allin1.npz"), **arrays)
    with open(os.path.join(HERE, "allin1.json"), "w") as f:
        json.dump(dict(torch_version=torch.__version__, reference="natten_mps " + natten_mps.__version__,
                       source="natten_mps.extras.allin1 na{1,2}d_qk_rpb / na{1,2}d_av_fused on the CPU",
                       cases=cases), f, indent=1)
    print(f"wrote {len(cases)} allin1 cases, {len(arrays)} arrays")


if __name__ == "__main__":
    args = [a for a in sys.argv[1:] if not a.startswith("--")]
    src = args[0] if args else "/root/reference/src"
    if "--allin1" in sys.argv:
        main_allin1(src)
    else:
        main(src)
