"""Oracle: CPU restatement of the reference's ``pure`` backend.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).  Never imported by the
shipped package.

Every function follows the reference op for op -- the same gathers, the same
einsum subscripts, ``* scale`` after the contraction, ``masked_fill(-inf)``,
``softmax`` over the last axis -- so that, on the same torch build, it returns
the same bits as the reference.  Citations are to files under
``/root/reference/src/natten_mps``.

Backward: like the reference (``_core/pure.py:680-696``) this module has no
hand-written backward; gradients come from torch autograd through the forward
graph, and the ``*_backward`` hooks return ``None``.
"""
from __future__ import annotations

from typing import Optional, Sequence, Tuple

import torch


def is_available() -> bool:
    return True


# ---------------------------------------------------------------------------
# Window rule (utils/window.py)
# ---------------------------------------------------------------------------


def window_start(index: int, length: int, kernel_size: int, dilation: int) -> int:
    """Scalar non-causal window start (``utils/window.py:91-111``)."""
    half = kernel_size // 2
    if dilation <= 1:
        s = max(index - half, 0)
        if index + half >= length:
            s += length - index - half - 1
        return s
    if index - half * dilation < 0:
        return index % dilation
    if index + half * dilation >= length:
        res = index % dilation
        full = (length // dilation) * dilation
        tail = length - full
        if res < tail:
            return length - tail + res - 2 * half * dilation
        return full + res - kernel_size * dilation
    return index - half * dilation


def window_end(index: int, length: int, kernel_size: int, dilation: int) -> int:
    """Inclusive window end (``utils/window.py:114-116``)."""
    return window_start(index, length, kernel_size, dilation) + (kernel_size - 1) * dilation


def window_start_vec(idx: torch.Tensor, length: int, kernel_size: int, dilation: int) -> torch.Tensor:
    """Vectorised non-causal window start (``utils/window.py:6-46``)."""
    half = kernel_size // 2
    idx = idx.to(dtype=torch.long)
    if dilation <= 1:
        s = torch.clamp(idx - half, min=0)
        at_right = idx + half >= length
        return s + at_right.to(dtype=s.dtype) * (length - idx - half - 1)

    plain = idx - half * dilation
    at_left = plain < 0
    from_left = torch.remainder(idx, dilation)
    at_right = idx + half * dilation >= length
    res = torch.remainder(idx, dilation)
    full = (length // dilation) * dilation
    tail = length - full
    from_right = torch.where(
        res < tail,
        length - tail + res - 2 * half * dilation,
        full + res - kernel_size * dilation,
    )
    out = torch.where(at_left, from_left, plain)
    return torch.where((~at_left) & at_right, from_right, out)


# ---------------------------------------------------------------------------
# Index maps (_core/pure.py:22-129, 335-387)
# ---------------------------------------------------------------------------


def _default_scale(t: torch.Tensor) -> float:
    return t.shape[-1] ** -0.5


def output_positions(length: int, stride: int, device) -> torch.Tensor:
    """``arange(ceil(L/s)) * s`` (``pure.py:22-24``)."""
    n = (length + stride - 1) // stride
    return torch.arange(n, device=device, dtype=torch.long) * stride


def axis_indices(pos: torch.Tensor, length: int, kernel_size: int, dilation: int,
                 causal: bool, device) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
    """Per-axis neighbour indices ``[n, K]`` and validity.

    Non-causal: window start + k*dilation, always valid (``pure.py:27-42``).
    Causal: start ``i-(K-1)*d``, validity ``0 <= j <= i``, indices clamped to
    ``[0, L-1]`` (``pure.py:45-56``).
    """
    steps = torch.arange(kernel_size, device=device, dtype=torch.long) * dilation
    if causal:
        first = pos - (kernel_size - 1) * dilation
        raw = first.unsqueeze(-1) + steps.unsqueeze(0)
        ok = (raw >= 0) & (raw <= pos.unsqueeze(-1))
        return raw.clamp(0, length - 1), ok
    first = window_start_vec(pos, length=length, kernel_size=kernel_size, dilation=dilation)
    return first.unsqueeze(-1) + steps.unsqueeze(0), None


def neighborhood_1d(pos, length, kernel_size, dilation, causal, device):
    return axis_indices(pos, length, kernel_size, dilation, causal, device)


def neighborhood_2d(ph, pw, height, width, kernel_size, dilation, is_causal, device):
    """Flattened 2-D map ``[oh, ow, kh*kw]`` + validity (``pure.py:91-129``)."""
    kh, kw = kernel_size
    ih, vh = axis_indices(ph, height, kh, dilation[0], is_causal[0], device)
    iw, vw = axis_indices(pw, width, kw, dilation[1], is_causal[1], device)
    if vh is None:
        vh = torch.ones_like(ih, dtype=torch.bool)
    if vw is None:
        vw = torch.ones_like(iw, dtype=torch.bool)
    oh, ow = ph.numel(), pw.numel()
    gh = ih[:, None, :, None].expand(oh, ow, kh, kw)
    gw = iw[None, :, None, :].expand(oh, ow, kh, kw)
    flat = (gh * width + gw).reshape(oh, ow, kh * kw)
    valid = None
    if is_causal[0] or is_causal[1]:
        valid = (vh[:, None, :, None] & vw[None, :, None, :]).reshape(oh, ow, kh * kw)
    return flat, valid


def neighborhood_3d(pd, ph, pw, depth, height, width, kernel_size, dilation, is_causal, device):
    """Flattened 3-D map ``[od, oh, ow, kd*kh*kw]`` + validity (``pure.py:335-387``)."""
    kd, kh, kw = kernel_size
    idd, vd = axis_indices(pd, depth, kd, dilation[0], is_causal[0], device)
    ih, vh = axis_indices(ph, height, kh, dilation[1], is_causal[1], device)
    iw, vw = axis_indices(pw, width, kw, dilation[2], is_causal[2], device)
    if vd is None:
        vd = torch.ones_like(idd, dtype=torch.bool)
    if vh is None:
        vh = torch.ones_like(ih, dtype=torch.bool)
    if vw is None:
        vw = torch.ones_like(iw, dtype=torch.bool)
    od, oh, ow = pd.numel(), ph.numel(), pw.numel()
    gd = idd[:, None, None, :, None, None].expand(od, oh, ow, kd, kh, kw)
    gh = ih[None, :, None, None, :, None].expand(od, oh, ow, kd, kh, kw)
    gw = iw[None, None, :, None, None, :].expand(od, oh, ow, kd, kh, kw)
    flat = ((gd * height + gh) * width + gw).reshape(od, oh, ow, kd * kh * kw)
    valid = None
    if any(is_causal):
        valid = (
            vd[:, None, None, :, None, None]
            & vh[None, :, None, None, :, None]
            & vw[None, None, :, None, None, :]
        ).reshape(od, oh, ow, kd * kh * kw)
    return flat, valid


def _split_positions(length, stride, n_out, device):
    """Query positions of the split ops: strided grid, or ``arange(n_out)``
    when the stride is 1 (``pure.py:235,259,300-302,446-448,538-539``)."""
    if stride != 1:
        return output_positions(length, stride, device)
    return torch.arange(n_out, device=device, dtype=torch.long)


# ---------------------------------------------------------------------------
# Fused forward (pure.py:146-220, 391-434)
# ---------------------------------------------------------------------------


def _check_same(q, k, v, ndim, layout):
    if q.ndim != ndim or k.ndim != ndim or v.ndim != ndim:
        raise ValueError(f"inputs must have shape {layout}.")
    if q.shape != k.shape or q.shape != v.shape:
        raise ValueError("query, key, and value must have identical shapes.")


def na1d_forward(q, k, v, kernel_size, stride, dilation, is_causal, scale):
    _check_same(q, k, v, 4, "[B, L, H, D]")
    sc = float(_default_scale(q) if scale is None else scale)
    length = q.shape[1]
    pos = output_positions(length, stride[0], q.device)
    qs = q.index_select(1, pos)
    idx, valid = neighborhood_1d(pos, length, kernel_size[0], dilation[0], is_causal[0], q.device)
    kn = k[:, idx]
    logits = torch.einsum("blhd,blkhd->blhk", qs, kn) * sc
    if valid is not None:
        logits = logits.masked_fill(~valid.view(1, -1, 1, kernel_size[0]), float("-inf"))
    attn = torch.softmax(logits, dim=-1)
    vn = v[:, idx]
    return torch.einsum("blhk,blkhd->blhd", attn, vn)


def na2d_forward(q, k, v, kernel_size, stride, dilation, is_causal, scale):
    _check_same(q, k, v, 5, "[B, H, W, heads, dim]")
    sc = float(_default_scale(q) if scale is None else scale)
    _, height, width, _, _ = q.shape
    ph = output_positions(height, stride[0], q.device)
    pw = output_positions(width, stride[1], q.device)
    qs = q.index_select(1, ph).index_select(2, pw)
    flat, valid = neighborhood_2d(ph, pw, height, width, kernel_size, dilation, is_causal, q.device)
    kf = k.reshape(k.shape[0], height * width, k.shape[3], k.shape[4])
    vf = v.reshape(v.shape[0], height * width, v.shape[3], v.shape[4])
    kn = kf[:, flat]
    logits = torch.einsum("bijhd,bijkhd->bijhk", qs, kn) * sc
    if valid is not None:
        logits = logits.masked_fill(~valid.view(1, valid.shape[0], valid.shape[1], 1, valid.shape[2]), float("-inf"))
    attn = torch.softmax(logits, dim=-1)
    vn = vf[:, flat]
    return torch.einsum("bijhk,bijkhd->bijhd", attn, vn)


def na3d_forward(q, k, v, kernel_size, stride, dilation, is_causal, scale):
    _check_same(q, k, v, 6, "[B, D, H, W, heads, dim]")
    sc = float(_default_scale(q) if scale is None else scale)
    _, depth, height, width, _, _ = q.shape
    pd = output_positions(depth, stride[0], q.device)
    ph = output_positions(height, stride[1], q.device)
    pw = output_positions(width, stride[2], q.device)
    qs = q.index_select(1, pd).index_select(2, ph).index_select(3, pw)
    flat, valid = neighborhood_3d(pd, ph, pw, depth, height, width, kernel_size, dilation, is_causal, q.device)
    kf = k.reshape(k.shape[0], depth * height * width, k.shape[4], k.shape[5])
    kn = kf[:, flat]
    logits = torch.einsum("bdijhf,bdijkhf->bdijhk", qs, kn) * sc
    if valid is not None:
        logits = logits.masked_fill(
            ~valid.view(1, valid.shape[0], valid.shape[1], valid.shape[2], 1, valid.shape[3]), float("-inf"))
    attn = torch.softmax(logits, dim=-1)
    vf = v.reshape(v.shape[0], depth * height * width, v.shape[4], v.shape[5])
    vn = vf[:, flat]
    return torch.einsum("bdijhk,bdijkhf->bdijhf", attn, vn)


# ---------------------------------------------------------------------------
# Split QK (pure.py:223-256, 302-332, 437-474)
# ---------------------------------------------------------------------------


def na1d_qk_forward(q, k, kernel_size, dilation, stride=(1,), is_causal=(False,), scale=None):
    if q.ndim != 4 or k.ndim != 4:
        raise ValueError("na1d_qk expects query/key shaped [B, L, H, D].")
    if q.shape != k.shape:
        raise ValueError("query and key must have identical shape for na1d_qk.")
    length = q.shape[1]
    pos = output_positions(length, stride[0], q.device)
    qs = q.index_select(1, pos) if stride[0] != 1 else q
    idx, valid = neighborhood_1d(pos, length, kernel_size[0], dilation[0], is_causal[0], q.device)
    logits = torch.einsum("blhd,blkhd->blhk", qs, k[:, idx])
    if valid is not None:
        logits = logits.masked_fill(~valid.view(1, -1, 1, kernel_size[0]), float("-inf"))
    if scale is not None:
        logits = logits * scale
    return logits


def na2d_qk_forward(q, k, kernel_size, dilation, stride=(1, 1), is_causal=(False, False), scale=None):
    if q.ndim != 5 or k.ndim != 5:
        raise ValueError("na2d_qk expects query/key shaped [B, H, W, heads, dim].")
    if q.shape != k.shape:
        raise ValueError("query and key must have identical shape for na2d_qk.")
    _, height, width, _, _ = q.shape
    ph = _split_positions(height, stride[0], height, q.device)
    pw = _split_positions(width, stride[1], width, q.device)
    qs = q.index_select(1, ph).index_select(2, pw) if stride[0] != 1 or stride[1] != 1 else q
    flat, valid = neighborhood_2d(ph, pw, height, width, kernel_size, dilation, is_causal, q.device)
    kf = k.reshape(k.shape[0], height * width, k.shape[3], k.shape[4])
    logits = torch.einsum("bijhd,bijkhd->bijhk", qs, kf[:, flat])
    if valid is not None:
        logits = logits.masked_fill(~valid.view(1, valid.shape[0], valid.shape[1], 1, valid.shape[2]), float("-inf"))
    if scale is not None:
        logits = logits * scale
    return logits


def na3d_qk_forward(q, k, kernel_size, dilation, stride=(1, 1, 1), is_causal=(False, False, False), scale=None):
    if q.ndim != 6 or k.ndim != 6:
        raise ValueError("na3d_qk expects query/key shaped [B, D, H, W, heads, dim].")
    if q.shape != k.shape:
        raise ValueError("query and key must have identical shape for na3d_qk.")
    _, depth, height, width, _, _ = q.shape
    pd = _split_positions(depth, stride[0], depth, q.device)
    ph = _split_positions(height, stride[1], height, q.device)
    pw = _split_positions(width, stride[2], width, q.device)
    strided = stride[0] != 1 or stride[1] != 1 or stride[2] != 1
    qs = q.index_select(1, pd).index_select(2, ph).index_select(3, pw) if strided else q
    flat, valid = neighborhood_3d(pd, ph, pw, depth, height, width, kernel_size, dilation, is_causal, q.device)
    kf = k.reshape(k.shape[0], depth * height * width, k.shape[4], k.shape[5])
    logits = torch.einsum("bdijhf,bdijkhf->bdijhk", qs, kf[:, flat])
    if valid is not None:
        logits = logits.masked_fill(
            ~valid.view(1, valid.shape[0], valid.shape[1], valid.shape[2], 1, valid.shape[3]), float("-inf"))
    if scale is not None:
        logits = logits * scale
    return logits


# ---------------------------------------------------------------------------
# Split AV (pure.py:259-296, 477-512, 515-565)
# ---------------------------------------------------------------------------


def na1d_av_forward(attn, v, kernel_size, dilation, stride=(1,), is_causal=(False,)):
    if attn.ndim != 4:
        raise ValueError("attn must have shape [B, L, H, K] for na1d_av.")
    if v.ndim != 4:
        raise ValueError("value must have shape [B, L, H, D] for na1d_av.")
    b1, l_out, h1, k_attn = attn.shape
    b2, length, h2, _ = v.shape
    if b1 != b2 or h1 != h2:
        raise ValueError("Batch and head dimensions of attn/value must match in na1d_av.")
    if k_attn != kernel_size[0]:
        raise ValueError(f"attn last dim ({k_attn}) must match kernel_size ({kernel_size[0]}).")
    if l_out > length:
        raise ValueError("attn sequence length cannot exceed value sequence length.")
    pos = _split_positions(length, stride[0], l_out, v.device)
    idx, valid = neighborhood_1d(pos, length, kernel_size[0], dilation[0], is_causal[0], v.device)
    vn = v[:, idx]
    if valid is not None:
        a = attn.masked_fill(~valid.view(1, -1, 1, kernel_size[0]), 0.0)
        return torch.einsum("blhk,blkhd->blhd", a, vn)
    return torch.einsum("blhk,blkhd->blhd", attn, vn)


def na2d_av_forward(attn, v, kernel_size, dilation, stride=(1, 1), is_causal=(False, False)):
    if attn.ndim != 5:
        raise ValueError("attn must have shape [B, H, W, heads, K] for na2d_av.")
    if v.ndim != 5:
        raise ValueError("value must have shape [B, H, W, heads, D] for na2d_av.")
    b1, h_out, w_out, heads1, k_attn = attn.shape
    b2, height, width, heads2, _ = v.shape
    if b1 != b2 or heads1 != heads2:
        raise ValueError("Batch and head dimensions of attn/value must match in na2d_av.")
    if k_attn != kernel_size[0] * kernel_size[1]:
        raise ValueError(f"attn last dim ({k_attn}) must match kernel area ({kernel_size[0] * kernel_size[1]}).")
    if h_out > height or w_out > width:
        raise ValueError("attn spatial dimensions cannot exceed value spatial dimensions.")
    ph = _split_positions(height, stride[0], h_out, v.device)
    pw = _split_positions(width, stride[1], w_out, v.device)
    flat, valid = neighborhood_2d(ph, pw, height, width, kernel_size, dilation, is_causal, v.device)
    vf = v.reshape(v.shape[0], height * width, v.shape[3], v.shape[4])
    vn = vf[:, flat]
    if valid is not None:
        a = attn.masked_fill(~valid.view(1, valid.shape[0], valid.shape[1], 1, valid.shape[2]), 0.0)
        return torch.einsum("bijhk,bijkhd->bijhd", a, vn)
    return torch.einsum("bijhk,bijkhd->bijhd", attn, vn)


def na3d_av_forward(attn, v, kernel_size, dilation, stride=(1, 1, 1), is_causal=(False, False, False)):
    if attn.ndim != 6:
        raise ValueError("attn must have shape [B, D, H, W, heads, K] for na3d_av.")
    if v.ndim != 6:
        raise ValueError("value must have shape [B, D, H, W, heads, D] for na3d_av.")
    b1, d_out, h_out, w_out, heads1, k_attn = attn.shape
    b2, depth, height, width, heads2, _ = v.shape
    if b1 != b2 or heads1 != heads2:
        raise ValueError("Batch and head dimensions of attn/value must match in na3d_av.")
    vol = kernel_size[0] * kernel_size[1] * kernel_size[2]
    if k_attn != vol:
        raise ValueError(f"attn last dim ({k_attn}) must match kernel volume ({vol}).")
    if d_out > depth or h_out > height or w_out > width:
        raise ValueError("attn spatial dimensions cannot exceed value spatial dimensions.")
    pd = _split_positions(depth, stride[0], d_out, v.device)
    ph = _split_positions(height, stride[1], h_out, v.device)
    pw = _split_positions(width, stride[2], w_out, v.device)
    flat, valid = neighborhood_3d(pd, ph, pw, depth, height, width, kernel_size, dilation, is_causal, v.device)
    vf = v.reshape(v.shape[0], depth * height * width, v.shape[4], v.shape[5])
    vn = vf[:, flat]
    if valid is not None:
        a = attn.masked_fill(
            ~valid.view(1, valid.shape[0], valid.shape[1], valid.shape[2], 1, valid.shape[3]), 0.0)
        return torch.einsum("bdijhk,bdijkhf->bdijhf", a, vn)
    return torch.einsum("bdijhk,bdijkhf->bdijhf", attn, vn)


# ---------------------------------------------------------------------------
# Backward hooks: none (pure.py:680-696) -- gradients via torch autograd.
# ---------------------------------------------------------------------------


def na1d_qk_backward(*args, **kwargs):
    return None


def na2d_qk_backward(*args, **kwargs):
    return None


def na3d_qk_backward(*args, **kwargs):
    return None


def na1d_av_backward(*args, **kwargs):
    return None


def na2d_av_backward(*args, **kwargs):
    return None


def na3d_av_backward(*args, **kwargs):
    return None


# ---------------------------------------------------------------------------
# Helpers used by the tests and the bench's CPU leg
# ---------------------------------------------------------------------------


# ---------------------------------------------------------------------------
# Variable-length forward (pure.py:573-673): the padded batch is processed
# per sample on the sample's own extent; padding stays zero.
# ---------------------------------------------------------------------------


def _varlen(rank, fwd, q, k, v, sizes, kernel_size, dilation, scale):
    out = torch.zeros_like(q)
    stride = (1,) * rank
    causal = (False,) * rank
    for b in range(q.shape[0]):
        ext = [int(x) for x in sizes[b].reshape(-1).tolist()]
        idx = (slice(b, b + 1),) + tuple(slice(0, n) for n in ext)
        out[idx] = fwd(q[idx], k[idx], v[idx], kernel_size, stride, dilation, causal, scale)
    return out


def na1d_varlen_forward(q, k, v, seq_lens, kernel_size, dilation, scale):
    """``pure.py:573-600``."""
    return _varlen(1, na1d_forward, q, k, v, seq_lens.reshape(-1, 1), kernel_size, dilation, scale)


def na2d_varlen_forward(q, k, v, spatial_sizes, kernel_size, dilation, scale):
    """``pure.py:608-636``."""
    return _varlen(2, na2d_forward, q, k, v, spatial_sizes, kernel_size, dilation, scale)


def na3d_varlen_forward(q, k, v, spatial_sizes, kernel_size, dilation, scale):
    """``pure.py:644-673``."""
    return _varlen(3, na3d_forward, q, k, v, spatial_sizes, kernel_size, dilation, scale)


def forward(rank: int, q, k, v, kernel_size: Sequence[int], stride: Sequence[int],
            dilation: Sequence[int], is_causal: Sequence[bool], scale):
    """Rank-dispatching fused forward with GQA by ``repeat_interleave``
    (``functional.py:27-31,273-274``)."""
    rep = q.shape[-2] // k.shape[-2]
    if rep != 1:
        k = k.repeat_interleave(rep, dim=-2)
        v = v.repeat_interleave(rep, dim=-2)
    fn = {1: na1d_forward, 2: na2d_forward, 3: na3d_forward}[rank]
    return fn(q, k, v, tuple(kernel_size), tuple(stride), tuple(dilation), tuple(is_causal), scale)


def neighborhood(rank: int, spatial, kernel_size, dilation, stride, is_causal):
    """Flattened neighbour map and validity for the fused op at ``spatial``."""
    dev = torch.device("cpu")
    pos = [output_positions(n, s, dev) for n, s in zip(spatial, stride)]
    if rank == 1:
        return neighborhood_1d(pos[0], spatial[0], kernel_size[0], dilation[0], is_causal[0], dev)
    if rank == 2:
        return neighborhood_2d(pos[0], pos[1], spatial[0], spatial[1], kernel_size, dilation, is_causal, dev)
    return neighborhood_3d(pos[0], pos[1], pos[2], *spatial, kernel_size, dilation, is_causal, dev)
