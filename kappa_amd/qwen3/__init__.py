"""Qwen3 MoE block API mirroring kappa.qwen3 (ffn_moe, quant, architecture, norms, block)."""

from .architecture import (
    MoEImpl,
    Qwen3Config,
    moe_layer_config,
    qwen3_235b_a22b_moe_config,
    qwen3_config_for_preset,
)
from .block import moe_block_ffn, rms_norm
from .ffn_moe import PackedExperts, moe_swiglu_ffn, moe_swiglu_ffn_legacy, prepack_moe_experts
from .quant import (
    Q8Weight,
    Weight,
    is_q8_weight,
    quantize_weight,
    quantize_weight_per_channel,
    to_compute_dtype,
    weight_param_dtype,
)

__all__ = [
    "MoEImpl",
    "PackedExperts",
    "Q8Weight",
    "Qwen3Config",
    "Weight",
    "is_q8_weight",
    "moe_block_ffn",
    "moe_layer_config",
    "moe_swiglu_ffn",
    "moe_swiglu_ffn_legacy",
    "prepack_moe_experts",
    "quantize_weight",
    "quantize_weight_per_channel",
    "qwen3_235b_a22b_moe_config",
    "qwen3_config_for_preset",
    "rms_norm",
    "to_compute_dtype",
    "weight_param_dtype",
]
