from natten_mps_amd.nn._base import _NeighborhoodAttentionND


class NeighborhoodAttention2D(_NeighborhoodAttentionND):
    """2-D neighbourhood attention module over [B, H, W, C] inputs (``nn/na2d.py`` of the reference).

    Args: embed_dim, num_heads, kernel_size, stride, dilation, is_causal,
    num_kv_heads (GQA/MQA when smaller than num_heads), qkv_bias, qk_scale,
    attn_drop, proj_drop.
    """

    rank = 2

    def forward(self, x, spatial_sizes=None):
        return super().forward(x, spatial_sizes)
