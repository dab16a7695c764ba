from natten_mps_amd.nn._base import _NeighborhoodAttentionND


class NeighborhoodAttention3D(_NeighborhoodAttentionND):
    """3-D neighbourhood attention module over [B, D, H, W, C] inputs (``nn/na3d.py`` of the reference).

    Args: embed_dim, num_heads, kernel_size, stride, dilation, is_causal,
    num_kv_heads (GQA/MQA when smaller than num_heads), qkv_bias, qk_scale,
    attn_drop, proj_drop.
    """

    rank = 3

    def forward(self, x, spatial_sizes=None):
        return super().forward(x, spatial_sizes)
