"""Qwen3 hyperparameters: the reference's ``Qwen3Config`` (kappa/qwen3/architecture.py:19-51).

Field names, order and defaults are kept so that a config built for the
reference works here unchanged. The MoE block reads ``use_moe``,
``num_experts``, ``num_experts_per_tok``, ``moe_impl``, ``moe_capacity_factor``,
``moe_fixed_capacity_slots`` and ``moe_ragged_decode_token_threshold``.
"""

from __future__ import annotations

from dataclasses import dataclass, replace
from typing import Literal

ModelPreset = Literal["qwen3-0.6b", "qwen3-4b", "qwen3-30b-a3b"]

# kappa/qwen3/architecture.py:14
MoEImpl = Literal["gather_einsum", "fixed_capacity", "ragged_jax", "ragged_tokamax"]

QuantMode = Literal["none", "w8"]


@dataclass(frozen=True, slots=True)
class Qwen3Config:
    """Dense or MoE decoder-only config (same fields as the reference)."""

    vocab_size: int
    num_layers: int
    num_heads: int
    num_kv_heads: int
    head_dim: int
    model_dim: int
    intermediate_size: int
    rope_theta: float
    rms_eps: float
    use_tied_embedding: bool
    attn_logits_soft_cap: float | None
    use_moe: bool
    num_experts: int
    num_experts_per_tok: int
    pad_token_id: int
    eos_token_id: int
    moe_impl: MoEImpl = "gather_einsum"
    moe_capacity_factor: float = 1.25
    moe_fixed_capacity_slots: int | None = None
    moe_ragged_decode_token_threshold: int = 64
    quantization: QuantMode = "none"


def qwen3_config_for_preset(preset: ModelPreset) -> Qwen3Config:
    """Public shapes (kappa/qwen3/architecture.py:54-113)."""
    common = dict(
        vocab_size=151_936,
        rope_theta=1_000_000.0,
        rms_eps=1e-6,
        attn_logits_soft_cap=None,
        pad_token_id=151_643,
        eos_token_id=151_645,
    )
    if preset == "qwen3-0.6b":
        return Qwen3Config(
            num_layers=28, num_heads=16, num_kv_heads=8, head_dim=128, model_dim=1024, intermediate_size=3072,
            use_tied_embedding=True, use_moe=False, num_experts=0, num_experts_per_tok=0, **common,
        )  # fmt: skip
    if preset == "qwen3-4b":
        return Qwen3Config(
            num_layers=36, num_heads=32, num_kv_heads=8, head_dim=128, model_dim=2560, intermediate_size=9728,
            use_tied_embedding=True, use_moe=False, num_experts=0, num_experts_per_tok=0, **common,
        )  # fmt: skip
    if preset == "qwen3-30b-a3b":
        return Qwen3Config(
            num_layers=48, num_heads=32, num_kv_heads=4, head_dim=128, model_dim=2048, intermediate_size=768,
            use_tied_embedding=False, use_moe=True, num_experts=128, num_experts_per_tok=8, **common,
        )  # fmt: skip
    raise ValueError(f"unknown preset: {preset!r}")


def qwen3_235b_a22b_moe_config() -> Qwen3Config:
    """The 235B-A22B MoE layer shape (D=4096, 128 experts, top-8, I=1536).

    The reference has no preset for it; this is the 30B preset with the MoE
    layer fields replaced, the way the reference derives configs
    (dataclasses.replace)."""
    return replace(
        qwen3_config_for_preset("qwen3-30b-a3b"),
        num_layers=94,
        num_heads=64,
        model_dim=4096,
        intermediate_size=1536,
    )


def moe_layer_config(*, hidden: int, experts: int, top_k: int, intermediate: int, **overrides) -> Qwen3Config:
    """A minimal MoE config for one layer of the given shape (tests and benchmarks)."""
    base = Qwen3Config(
        vocab_size=128, num_layers=1, num_heads=4, num_kv_heads=2, head_dim=8, model_dim=hidden,
        intermediate_size=intermediate, rope_theta=10_000.0, rms_eps=1e-6, use_tied_embedding=True,
        attn_logits_soft_cap=None, use_moe=True, num_experts=experts, num_experts_per_tok=top_k,
        pad_token_id=0, eos_token_id=1,
    )  # fmt: skip
    return replace(base, **overrides) if overrides else base
