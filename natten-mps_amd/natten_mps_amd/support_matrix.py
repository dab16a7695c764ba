"""Backend capability matrix (``support_matrix.py`` of the reference, with the
``'hip'`` backend of this build)."""
from __future__ import annotations

from natten_mps_amd._core import hip, ops


def get_support_matrix() -> dict:
    out = {
        "hip": {
            "available": hip.is_available(),
            "forward": {"na1d": True, "na2d": True, "na3d": True, "split_qk_av": True},
            "backward": {"na1d": True, "na2d": True, "na3d": True, "split_qk_av": True},
            "varlen": {"na1d": True, "na2d": True, "na3d": True},
            "fusion": {"na1d": True, "na2d": True, "na3d": True},
            "extras_allin1": {"na1d_qk_rpb": True, "na1d_av_fused": True, "na2d_qk_rpb": True,
                              "na2d_av_fused": True},
            "constraints": [
                "Requires a ROCm GPU (gfx950 / MI355X) and the built libnatten_hip.so.",
                "float32, float16 and bfloat16; head dims up to 256 (q/k and v may differ).",
                "Causal, strided, causal+strided, dilated and non-uniform per-axis kernels.",
                "Native GQA/MQA (no K/V expansion); fused forward writes the LSE, fused backward "
                "accepts an LSE gradient (return_lse, additional_keys).",
                "An even kernel equal to a non-causal, undilated axis length is rejected.",
                "Variable-length (na{1,2,3}d_varlen): one launch per op for the whole padded batch, "
                "fused backward; padding positions are zero.",
            ],
        },
    }
    for name in ops.registered_backends():
        if name != "hip":
            out[name] = {"available": ops._backend_available(name), "registered": True}
    return out
