"""mega_kernel_qwen36 -- Qwen3.6 single-token decode hot path on MI355X (gfx950).

Drop-in for the decode surface of the reference package of the same name
(reference ``mega_kernel_qwen36/__init__.py:1-89``): the decode dataclasses and
ops, ``extension_available`` and the text-config factories.  The vision
encoder is not part of this package.  The decode task-graph planner
(``mpk_graph``) builds the reference's plans, and ``executor`` runs them on
the HIP kernels.
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
from .mpk_graph import (
    CompiledPlan,
    EventSpec,
    LaunchStep,
    TaskGraph,
    TaskSpec,
    TensorSpec,
    WorkerConfig,
    build_batch_specialized_plans,
    build_qwen36_decode_tgraph,
)
from .executor import DecodeLayerWeights, DecodePlanExecutor, DecodeStepResult

__all__ = [
    "CompiledPlan",
    "DecodeLayerResult",
    "DecodeLayerWeights",
    "DecodePlanExecutor",
    "DecodeStepResult",
    "EventSpec",
    "LaunchStep",
    "TaskGraph",
    "TaskSpec",
    "TensorSpec",
    "WorkerConfig",
    "build_batch_specialized_plans",
    "build_qwen36_decode_tgraph",
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
