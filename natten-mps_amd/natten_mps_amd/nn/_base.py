"""Shared body of the NeighborhoodAttention{1,2,3}D modules (``nn/na{1,2,3}d.py``
of /root/reference/src/natten_mps): qkv projection (or q_proj + kv_proj for
GQA), neighbourhood attention, output projection.

Kept as in the reference: with ``attn_drop > 0`` the module takes the split
QK -> softmax -> dropout -> AV path, which uses neither stride nor is_causal
and applies only the ratio of a custom scale to the default one
(``nn/na2d.py:105-111``)."""
from __future__ import annotations

from typing import Optional, Tuple, Union

import torch

from natten_mps_amd import functional as F
from natten_mps_amd.utils.params import normalize_tuple_param

_SHAPES = {1: "[B, L, C]", 2: "[B, H, W, C]", 3: "[B, D, H, W, C]"}


class _NeighborhoodAttentionND(torch.nn.Module):
    rank = 0

    def __init__(self, embed_dim: int, num_heads: int, kernel_size: Union[int, Tuple[int, ...]],
                 stride: Union[int, Tuple[int, ...]] = 1, dilation: Union[int, Tuple[int, ...]] = 1,
                 is_causal: Union[bool, Tuple[bool, ...]] = False, num_kv_heads: Optional[int] = None,
                 qkv_bias: bool = True, qk_scale: Optional[float] = None, attn_drop: float = 0.0,
                 proj_drop: float = 0.0):
        super().__init__()
        r = self.rank
        if embed_dim % num_heads != 0:
            raise ValueError("embed_dim must be divisible by num_heads")
        self.embed_dim = int(embed_dim)
        self.num_heads = int(num_heads)
        self.head_dim = self.embed_dim // self.num_heads
        self.num_kv_heads = int(num_kv_heads) if num_kv_heads is not None else self.num_heads
        if self.num_heads % self.num_kv_heads != 0:
            raise ValueError(
                f"num_heads ({self.num_heads}) must be divisible by num_kv_heads ({self.num_kv_heads})"
            )
        self.kernel_size = normalize_tuple_param(kernel_size, r, "kernel_size")
        self.stride = normalize_tuple_param(stride, r, "stride")
        self.dilation = normalize_tuple_param(dilation, r, "dilation")
        self.is_causal = tuple(bool(v) for v in normalize_tuple_param(is_causal, r, "is_causal"))
        self.scale = float(qk_scale) if qk_scale is not None else self.head_dim ** -0.5
        self._use_gqa = self.num_kv_heads != self.num_heads
        if self._use_gqa:
            self.q_proj = torch.nn.Linear(self.embed_dim, self.num_heads * self.head_dim, bias=qkv_bias)
            self.kv_proj = torch.nn.Linear(self.embed_dim, 2 * self.num_kv_heads * self.head_dim, bias=qkv_bias)
        else:
            self.qkv = torch.nn.Linear(self.embed_dim, self.embed_dim * 3, bias=qkv_bias)
        self.attn_drop_p = float(attn_drop)
        self.attn_drop = torch.nn.Dropout(attn_drop)
        self.proj = torch.nn.Linear(self.embed_dim, self.embed_dim)
        self.proj_drop = torch.nn.Dropout(proj_drop)

    def forward(self, x, sizes=None):
        r = self.rank
        if x.ndim != r + 2:
            raise ValueError(f"NeighborhoodAttention{r}D expects input shape {_SHAPES[r]}.")
        bsz, *sp, channels = x.shape
        if channels != self.embed_dim:
            raise ValueError(f"Input channel dim ({channels}) must equal embed_dim ({self.embed_dim}).")
        # move the q/k/v selector axis to the front: [3 or 2, B, *sp, heads, dim]
        perm = (r + 1, 0, *range(1, r + 1), r + 2, r + 3)
        if self._use_gqa:
            q = self.q_proj(x).reshape(bsz, *sp, self.num_heads, self.head_dim)
            kv = self.kv_proj(x).reshape(bsz, *sp, 2, self.num_kv_heads, self.head_dim).permute(*perm)
            k, v = kv.unbind(0)
        else:
            qkv = self.qkv(x).reshape(bsz, *sp, 3, self.num_heads, self.head_dim).permute(*perm)
            q, k, v = qkv.unbind(0)

        if sizes is not None:
            out = getattr(F, f"na{r}d_varlen")(q, k, v, sizes, kernel_size=self.kernel_size,
                                               dilation=self.dilation, scale=self.scale)
        elif self.attn_drop_p > 0.0:
            logits = getattr(F, f"na{r}d_qk")(q, k, kernel_size=self.kernel_size, dilation=self.dilation)
            default_scale = self.head_dim ** -0.5
            if self.scale != default_scale:
                logits = logits * (self.scale / default_scale)
            attn = self.attn_drop(torch.softmax(logits, dim=-1))
            out = getattr(F, f"na{r}d_av")(attn, v, kernel_size=self.kernel_size, dilation=self.dilation)
        else:
            out = getattr(F, f"na{r}d")(q, k, v, kernel_size=self.kernel_size, stride=self.stride,
                                        dilation=self.dilation, is_causal=self.is_causal, scale=self.scale)
        out = out.reshape(bsz, *out.shape[1:1 + r], self.embed_dim)
        return self.proj_drop(self.proj(out))
