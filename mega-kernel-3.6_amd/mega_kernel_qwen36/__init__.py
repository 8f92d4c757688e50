"""mega_kernel_qwen36 -- Qwen3.6 single-token decode hot path on MI355X (gfx950).

Drop-in for the decode surface of the reference package of the same name
(reference ``mega_kernel_qwen36/__init__.py:1-89``): the decode dataclasses and
ops, ``extension_available`` and the text-config factories.  The vision
encoder and the MPK task-graph planner are not part of this package.
"""

from .config import (
    Qwen36TextConfig,
    qwen36_27b_config,
    qwen36_35b_a3b_config,
    qwen36_layer_type,
)
from .ops import (
    DecodeLayerResult,
    DenseFfnWeights,
    FullAttentionInputs,
    GatedMoeWeights,
    LinearAttentionInputs,
    MoeWeights,
    apply_partial_rope,
    causal_conv1d_update,
    decode_layer,
    dense_ffn_decode,
    extension_available,
    full_attention_decode,
    gated_rms_norm,
    linear_attention_decode,
    linear_attention_step,
    moe_decode,
    moe_decode_status,
)
from ._lib import library_path, load_library

__all__ = [
    "DecodeLayerResult",
    "DenseFfnWeights",
    "FullAttentionInputs",
    "GatedMoeWeights",
    "LinearAttentionInputs",
    "MoeWeights",
    "Qwen36TextConfig",
    "apply_partial_rope",
    "causal_conv1d_update",
    "decode_layer",
    "dense_ffn_decode",
    "extension_available",
    "full_attention_decode",
    "gated_rms_norm",
    "library_path",
    "linear_attention_decode",
    "linear_attention_step",
    "load_library",
    "moe_decode",
    "moe_decode_status",
    "qwen36_27b_config",
    "qwen36_35b_a3b_config",
    "qwen36_layer_type",
]
