from natten_mps_amd.nn._base import _NeighborhoodAttentionND


class NeighborhoodAttention1D(_NeighborhoodAttentionND):
    """1-D neighbourhood attention module over [B, L, C] inputs (``nn/na1d.py`` of the reference).

    Args: embed_dim, num_heads, kernel_size, stride, dilation, is_causal,
    num_kv_heads (GQA/MQA when smaller than num_heads), qkv_bias, qk_scale,
    attn_drop, proj_drop.
    """

    rank = 1

    def forward(self, x, seq_lens=None):
        return super().forward(x, seq_lens)
