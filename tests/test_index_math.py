"""Window rule and index maps: the oracle (Python and C), and the device index
code (na_common.h, built for the host) against the reference's known answers,
a textbook definition, brute force, and each other."""
from __future__ import annotations

import ctypes
import itertools
import os
import subprocess

import numpy as np
import pytest
import torch

import oracle.pure as P
from conftest import ROOT
from natten_mps_amd._core import _lib

BUILD = os.path.join(ROOT, "tests", "native", "_build")


@pytest.fixture(scope="module")
def host_idx():
    os.makedirs(BUILD, exist_ok=True)
    out = os.path.join(BUILD, "libindex_host.so")
    subprocess.run(["/opt/rocm/bin/hipcc", "-O1", "-std=c++17", "-fPIC", "-shared",
                    "-I" + os.path.join(ROOT, "include"), "-I" + os.path.join(ROOT, "natten-mps_amd", "csrc"),
                    os.path.join(ROOT, "tests", "native", "index_host.cpp"), "-o", out], check=True)
    lib = ctypes.CDLL(out)
    lib.host_window_start.restype = ctypes.c_int
    lib.host_window_start.argtypes = [ctypes.c_int] * 4
    lib.host_neighbor_map.argtypes = [ctypes.POINTER(_lib.Problem), ctypes.c_void_p, ctypes.c_void_p]
    lib.host_inverse_mismatch.argtypes = [ctypes.POINTER(_lib.Problem)]
    lib.host_inverse_mismatch.restype = ctypes.c_longlong
    lib.host_class_mismatch.argtypes = [ctypes.POINTER(_lib.Problem)]
    lib.host_class_mismatch.restype = ctypes.c_longlong
    lib.host_query_item_mismatch.argtypes = [ctypes.POINTER(_lib.Problem)]
    lib.host_query_item_mismatch.restype = ctypes.c_longlong
    lib.host_fastdiv_errors.argtypes = [ctypes.c_uint32, ctypes.c_int, ctypes.c_int]
    lib.host_fastdiv_errors.restype = ctypes.c_longlong
    lib.host_tile_geometry_mismatch.argtypes = [ctypes.c_int] * 7
    lib.host_tile_geometry_mismatch.restype = ctypes.c_longlong
    return lib


def test_tile_geometry_against_brute_force(host_idx):
    """axis_geometry -- the per-axis tile geometry the tile kernels read from
    host-built tables or compute in-kernel -- against brute-force window
    enumeration: union boxes exact, wave boxes containing (and, with every
    key attended, equal to) what their items need; all residues, tiles and
    wave item ranges, query and key tiles, causal and not."""
    n = 0
    for L in (1, 2, 3, 5, 8, 13, 24):
        for K in range(1, min(L, 9) + 1):
            for d in range(1, 5):
                if K * d > L and not (d == 1):
                    continue
                for causal in (0, 1):
                    if not causal and d == 1 and K % 2 == 0 and K == L:
                        continue
                    for s in range(1, K + 1 if d == 1 else 2):
                        for T in (1, 2, 4, 8, 16):
                            for key in (0, 1):
                                assert host_idx.host_tile_geometry_mismatch(L, K, d, causal, T, key, s) == 0, \
                                    (L, K, d, causal, T, key, s)
                                n += 1
    assert n > 1000


@pytest.fixture(scope="module")
def host_union():
    os.makedirs(BUILD, exist_ok=True)
    out = os.path.join(BUILD, "libunion_host.so")
    subprocess.run(["/opt/rocm/bin/hipcc", "--offload-arch=gfx950", "-O1", "-std=c++17", "-fPIC", "-shared",
                    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
                    "-I" + os.path.join(ROOT, "include"), "-I" + os.path.join(ROOT, "natten-mps_amd", "csrc"),
                    os.path.join(ROOT, "tests", "native", "union_host.hip"), "-o", out], check=True)
    lib = ctypes.CDLL(out)
    lib.host_union_upto_undersized.argtypes = [ctypes.c_int] * 6
    lib.host_union_upto_undersized.restype = ctypes.c_int
    return lib


def test_varlen_tile_sizing_covers_every_sample_extent(host_union):
    """The variable-length tile kernels size LDS for the largest union any
    tile can have at any sample extent up to the padded one
    (union_extent_upto): checked against brute force over axis_geometry at
    every extent, for query and key tiles, all residues, causal and not."""
    n = 0
    for Lmax in (5, 9, 16, 23, 40, 61):
        for K in (2, 3, 4, 5, 7, 9):
            for d in (1, 2, 3):
                if K * d > Lmax:
                    continue
                for causal in (0, 1):
                    for T in (1, 2, 8, 16, 64):
                        for key in (0, 1):
                            assert host_union.host_union_upto_undersized(Lmax, K, d, causal, T, key) == 0, \
                                (Lmax, K, d, causal, T, key)
                            n += 1
    assert n > 1000


def test_fastdiv_matches_integer_division(host_idx):
    """The multiply-high division the tile kernels decode workgroup indices
    with equals n // d: every n below 2^20 for d <= 300 and every power of
    two, and a stride-sampled sweep up to 2^31 - 1 (plus its top 4096
    values) for divisors near powers of two and a few large odd ones."""
    small = list(range(1, 301)) + [1 << k for k in range(9, 31)]
    for d in small:
        assert host_idx.host_fastdiv_errors(d, 1 << 20, 1) == 0, d
    large = [(1 << k) + o for k in range(2, 31) for o in (-1, 1)] + [3, 7, 641, 65537, 999983, 2147483647]
    for d in large:
        assert host_idx.host_fastdiv_errors(d, (1 << 31) - 1, 9973) == 0, d


def test_class_coordinate_closed_forms(host_idx):
    """The division-free class-coordinate window start and inverse span used
    by the MFMA tile kernels equal the window rule and brute-force membership
    for every (L, K, d, causal, residue) with L <= 30."""
    n = 0
    for L, K, d in _sweep_starts(30):
        if d == 1 and K % 2 == 0 and K == L:
            continue
        for c in (False, True):
            assert host_idx.host_class_mismatch(ctypes.byref(_problem((L,), (K,), (d,), (1,), (c,)))) == 0, \
                (L, K, d, c)
            n += 1
    assert n > 1000


def test_query_item_closed_forms(host_idx):
    """Query items of the strided tile path: item t is the query at position
    stride * t (dilation 1); its window start and the items attending each
    key equal the window rule and brute-force membership for every (L, K,
    stride <= K, causal) with L <= 30, and at stride 1 for every dilation."""
    n = 0
    for L, K, d in _sweep_starts(30):
        if d == 1 and K % 2 == 0 and K == L:
            continue
        for s in range(1, K + 1 if d == 1 else 2):
            for c in (False, True):
                prob = _problem((L,), (K,), (d,), (s,), (c,))
                assert host_idx.host_query_item_mismatch(ctypes.byref(prob)) == 0, (L, K, d, s, c)
                n += 1
    assert n > 3000


@pytest.fixture(scope="module")
def c_oracle():
    subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle")], check=True)
    lib = ctypes.CDLL(os.path.join(ROOT, "oracle", "_build", "liboracle_window.so"))
    lib.oracle_window_start.restype = ctypes.c_int64
    lib.oracle_window_start.argtypes = [ctypes.c_int64] * 4
    return lib


def _problem(spatial, ks, dil, st, causal):
    return _lib.problem(batch=1, heads_q=1, heads_kv=1, dim_qk=1, dim_v=1, dtype=_lib.F32, length=spatial,
                        out_length=[(n + s - 1) // s for n, s in zip(spatial, st)], kernel_size=ks,
                        dilation=dil, stride=st, is_causal=causal, scale=None)


def _sweep_starts(maxL=30):
    for L in range(1, maxL + 1):
        for K in range(1, L + 1):
            for d in range(1, L // K + 1):
                yield L, K, d


# -- window start ---------------------------------------------------------


def test_known_answers():
    # tests/test_shift_semantics.py:66-99 of the reference
    assert P.window_start(0, 10, 3, 1) == 0
    assert P.window_start(9, 10, 3, 1) == 7
    assert P.window_start(5, 11, 5, 1) == 3
    for i in range(20):
        s = P.window_start(i, 20, 3, 2)
        assert 0 <= s and s + 2 * 2 <= 19
        assert len({s + k * 2 for k in range(3)}) == 3
    assert P.window_end(4, 9, 5, 1) == P.window_start(4, 9, 5, 1) + 4


def test_odd_kernel_matches_textbook_definition():
    """Odd K: the window is the run of K positions of i's residue class,
    centred on i and shifted inwards to fit the axis."""
    for L, K, d in _sweep_starts():
        if K % 2 == 0:
            continue
        for i in range(L):
            r, j = i % d, i // d
            n_cls = (L - r + d - 1) // d
            want = r + min(max(j - K // 2, 0), n_cls - K) * d
            assert P.window_start(i, L, K, d) == want, (i, L, K, d)


def test_vectorised_equals_scalar():
    for L, K, d in _sweep_starts(24):
        got = P.window_start_vec(torch.arange(L), L, K, d).tolist()
        assert got == [P.window_start(i, L, K, d) for i in range(L)]


def test_out_of_range_only_for_even_kernel_equal_to_axis():
    """The device code rejects exactly this case; everywhere else every window
    lies inside the axis and starts are non-decreasing along a residue class
    (what the key -> queries enumeration relies on)."""
    for L, K, d in _sweep_starts():
        starts = [P.window_start(i, L, K, d) for i in range(L)]
        oor = any(s < 0 or s + (K - 1) * d > L - 1 for s in starts)
        assert oor == (d == 1 and K % 2 == 0 and K == L), (L, K, d)
        if oor:
            continue
        for r in range(d):
            cls = starts[r::d]
            assert all(a <= b for a, b in zip(cls, cls[1:])), (L, K, d, r)
            assert all(s % d == r for s in cls)


def test_c_oracle_and_device_rule_agree(c_oracle, host_idx):
    for L, K, d in _sweep_starts(24):
        for i in range(L):
            want = P.window_start(i, L, K, d)
            assert c_oracle.oracle_window_start(i, L, K, d) == want
            assert host_idx.host_window_start(i, L, K, d) == want


# -- neighbourhood maps ------------------------------------------------------

MAP_CASES = [
    ((37,), (5,), (1,), (1,), (False,)),
    ((37,), (5,), (3,), (2,), (True,)),
    ((40,), (9,), (4,), (3,), (False,)),
    ((16,), (4,), (1,), (1,), (False,)),
    ((10, 12), (3, 5), (1, 2), (1, 1), (False, False)),
    ((10, 12), (5, 3), (2, 1), (2, 3), (True, False)),
    ((9, 11), (3, 5), (3, 2), (3, 1), (True, True)),
    ((56, 56), (7, 7), (8, 8), (1, 1), (False, False)),
    ((6, 7, 8), (3, 3, 5), (1, 2, 1), (1, 1, 2), (False, True, False)),
    ((5, 6, 7), (3, 3, 3), (1, 1, 2), (2, 1, 1), (True, True, True)),
    ((16, 32, 32), (3, 7, 7), (1, 2, 2), (1, 1, 1), (False, False, False)),
]


def _oracle_map(spatial, ks, dil, st, causal):
    flat, valid = P.neighborhood(len(spatial), spatial, ks, dil, st, causal)
    if len(spatial) == 1:
        flat = flat  # [n_out, K]
    if valid is None:
        valid = torch.ones_like(flat, dtype=torch.bool)
    return flat.reshape(-1, flat.shape[-1]), valid.reshape(-1, flat.shape[-1])


@pytest.mark.parametrize("case", MAP_CASES)
def test_device_index_code_map_equals_oracle(case, host_idx, c_oracle):
    spatial, ks, dil, st, causal = case
    flat, valid = _oracle_map(spatial, ks, dil, st, causal)
    prob = _problem(spatial, ks, dil, st, causal)
    got_f = np.empty(flat.numel(), dtype=np.int64)
    got_v = np.empty(flat.numel(), dtype=np.uint8)
    host_idx.host_neighbor_map(ctypes.byref(prob), got_f.ctypes.data, got_v.ctypes.data)
    assert np.array_equal(got_f, flat.reshape(-1).numpy())
    assert np.array_equal(got_v.astype(bool), valid.reshape(-1).numpy())
    # the C restatement of the oracle
    pad = lambda v, f: [f] * (3 - len(v)) + list(v)  # noqa: E731
    arr = lambda v: (ctypes.c_int64 * 3)(*pad(v, 1))  # noqa: E731
    cf = np.empty(flat.numel(), dtype=np.int64)
    cv = np.empty(flat.numel(), dtype=np.uint8)
    c_oracle.oracle_neighborhood(arr(spatial), arr(ks), arr(dil), arr(st),
                                 (ctypes.c_int * 3)(*pad([int(c) for c in causal], 0)),
                                 cf.ctypes.data_as(ctypes.c_void_p), cv.ctypes.data_as(ctypes.c_void_p))
    assert np.array_equal(cf, flat.reshape(-1).numpy())
    assert np.array_equal(cv.astype(bool), valid.reshape(-1).numpy())


def test_inverse_enumeration_is_exact(host_idx):
    """Key -> queries enumeration (used by every dK/dV kernel) visits exactly
    the valid (query, neighbour) pairs of the forward, for a sweep of 1-D and
    2-D shapes including causal, stride and dilation."""
    n = 0
    for L, K, d in _sweep_starts(14):
        if d == 1 and K % 2 == 0 and K == L:
            continue
        for s, c in itertools.product((1, 2, 3), (False, True)):
            if s > K:
                continue
            assert host_idx.host_inverse_mismatch(ctypes.byref(_problem((L,), (K,), (d,), (s,), (c,)))) == 0
            n += 1
    for case in MAP_CASES[4:]:
        spatial, ks, dil, st, causal = case
        if np.prod(spatial) > 2000:
            continue
        assert host_idx.host_inverse_mismatch(ctypes.byref(_problem(spatial, ks, dil, st, causal))) == 0
    assert n > 500
