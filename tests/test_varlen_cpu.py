"""Variable-length attention on the CPU: the oracle's varlen restatement
(oracle/pure.py, following _core/pure.py:573-673) pinned by what the
definition fixes, and the functional layer's validation (the reference's
tests/test_varlen_na{1,2,3}d.py validation classes), which runs before any
backend is called."""
from __future__ import annotations

import pytest
import torch

import oracle.pure as P


def _rand(shape, seed, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g, dtype=dtype)


def _masked_dense_1d(q, k, v, L, K, d, scale):
    """Dense attention over the first L positions with the textbook window
    of K class members (centred, shifted inwards, residue class kept) --
    the brute-force definition, independent of the oracle's index maps."""
    mask = torch.zeros(L, L, dtype=torch.bool)
    for i in range(L):
        cls = [j for j in range(L) if j % d == i % d]
        pos = cls.index(i)
        start = min(max(pos - K // 2, 0), len(cls) - K)
        for j in cls[start:start + K]:
            mask[i, j] = True
    logits = torch.einsum("nhd,mhd->hnm", q[:L], k[:L]) * scale
    logits = logits.masked_fill(~mask, float("-inf"))
    return torch.einsum("hnm,mhd->nhd", logits.softmax(-1), v[:L])


def test_oracle_varlen_uniform_sizes_equal_na():
    q, k, v = (_rand((2, 9, 10, 2, 4), s) for s in (1, 2, 3))
    sizes = torch.tensor([[9, 10], [9, 10]])
    out = P.na2d_varlen_forward(q, k, v, sizes, (3, 5), (1, 2), None)
    ref = P.na2d_forward(q, k, v, (3, 5), (1, 1), (1, 2), (False, False), None)
    torch.testing.assert_close(out, ref, atol=0, rtol=0)


def test_oracle_varlen_windows_follow_each_samples_length():
    """Sample b's windows are those of an axis of length seq_lens[b] (shifted
    inwards at its own border), not of L_max; padding stays zero."""
    B, L, H, D, K, d = 3, 17, 2, 5, 5, 2
    q, k, v = (_rand((B, L, H, D), s) for s in (4, 5, 6))
    lens = torch.tensor([17, 12, 10])
    out = P.na1d_varlen_forward(q, k, v, lens, (K,), (d,), 0.4)
    for b, n in enumerate(lens.tolist()):
        torch.testing.assert_close(out[b, :n], _masked_dense_1d(q[b], k[b], v[b], n, K, d, 0.4),
                                   atol=1e-12, rtol=1e-12)
        assert (out[b, n:] == 0).all()


def test_oracle_varlen_3d_per_sample_and_padding():
    q, k, v = (_rand((2, 5, 6, 7, 2, 3), s) for s in (7, 8, 9))
    sizes = torch.tensor([[5, 6, 7], [3, 4, 5]])
    out = P.na3d_varlen_forward(q, k, v, sizes, (3, 3, 3), (1, 1, 1), None)
    sub = P.na3d_forward(q[1:, :3, :4, :5], k[1:, :3, :4, :5], v[1:, :3, :4, :5], (3, 3, 3), (1, 1, 1),
                         (1, 1, 1), (False, False, False), None)
    torch.testing.assert_close(out[1:, :3, :4, :5], sub, atol=0, rtol=0)
    assert (out[1, 3:] == 0).all() and (out[1, :3, 4:] == 0).all() and (out[1, :3, :4, 5:] == 0).all()


# ---------------------------------------------------------------------------
# functional validation (messages as in functional.py:678-787)
# ---------------------------------------------------------------------------


def _qkv(shape):
    return (torch.randn(shape) for _ in range(3))


def test_varlen_rejects_small_and_large_lengths():
    from natten_mps_amd.functional import na1d_varlen, na2d_varlen

    q, k, v = _qkv((2, 12, 2, 8))
    with pytest.raises(ValueError, match="kernel_size"):
        na1d_varlen(q, k, v, torch.tensor([12, 4], dtype=torch.int32), kernel_size=5)
    with pytest.raises(ValueError, match="L_max"):
        na1d_varlen(q, k, v, torch.tensor([12, 13], dtype=torch.int32), kernel_size=3)
    q, k, v = _qkv((2, 12, 12, 2, 8))
    with pytest.raises(ValueError, match="max_spatial"):
        na2d_varlen(q, k, v, torch.tensor([[12, 12], [12, 13]], dtype=torch.int32), kernel_size=3)
    with pytest.raises(ValueError, match="kernel_size"):
        na2d_varlen(q, k, v, torch.tensor([[12, 12], [4, 12]], dtype=torch.int32), kernel_size=5)


def test_varlen_rejects_bad_size_tensors_and_shapes():
    from natten_mps_amd.functional import na1d_varlen, na2d_varlen, na3d_varlen

    q, k, v = _qkv((2, 12, 2, 8))
    with pytest.raises(ValueError, match="1-D tensor of length B=2"):
        na1d_varlen(q, k, v, torch.tensor([[12], [8]], dtype=torch.int32), kernel_size=3)
    with pytest.raises(ValueError, match="int32 or int64"):
        na1d_varlen(q, k, v, torch.tensor([12.0, 8.0]), kernel_size=3)
    q, k, v = _qkv((2, 12, 12, 2, 8))
    with pytest.raises(ValueError, match=r"\[B, 2\]"):
        na2d_varlen(q, k, v, torch.tensor([8, 8], dtype=torch.int32), kernel_size=3)
    with pytest.raises(ValueError, match="identical shapes"):
        na2d_varlen(q, k[..., :7], v, torch.tensor([[12, 12], [8, 8]], dtype=torch.int32), kernel_size=3)
    q, k, v = _qkv((1, 6, 6, 6, 2, 4))
    with pytest.raises(ValueError, match="shape"):
        na3d_varlen(q[0], k[0], v[0], torch.tensor([[6, 6, 6]], dtype=torch.int32), kernel_size=3)


def test_varlen_rejects_dilated_kernel_larger_than_a_sample():
    """na*d on a sample's slice requires dilation * kernel <= its extent
    (utils/params.py checks, as the reference's per-sample call would)."""
    from natten_mps_amd.functional import na1d_varlen

    q, k, v = _qkv((2, 16, 2, 8))
    with pytest.raises(ValueError, match="exceeds input spatial size"):
        na1d_varlen(q, k, v, torch.tensor([16, 5], dtype=torch.int32), kernel_size=3, dilation=2)


def test_varlen_through_a_registered_pure_backend(pure_backend):
    """Backends without fused varlen ops run the per-sample composition."""
    from natten_mps_amd.functional import na1d_varlen

    q, k, v = (_rand((2, 11, 2, 4), s, torch.float32) for s in (10, 11, 12))
    lens = torch.tensor([11, 7])
    out = na1d_varlen(q, k, v, lens, kernel_size=3)
    ref = P.na1d_varlen_forward(q, k, v, lens, (3,), (1,), None)
    torch.testing.assert_close(out, ref, atol=1e-6, rtol=1e-6)
