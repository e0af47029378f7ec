"""The steps either side of the MoE block in a Qwen3 MoE layer.

``rms_norm`` mirrors kappa/qwen3/norms.py:10-16 and ``moe_block_ffn`` the MoE
half of the layer (kappa/qwen3/block.py:71-82, 153-164, 196-207)::

    h2 = rms_norm(h, params.pre_ffn_norm)
    out = moe_swiglu_ffn(h2, router, gate_proj, up_proj, down_proj, cfg=cfg)
    return h + out

``moe_block_ffn`` runs the three steps as one C-ABI call (kmoe_forward_block):
the norm writes h2 once into the workspace and the combine kernel adds the
block's output to h, so the separate add and its [T, D] round trip disappear.
"""

from __future__ import annotations

import torch

from .. import _lib
from .architecture import Qwen3Config
from .ffn_moe import PackedExperts, _desc, _impl_and_capacity, _moe_forward, _norm_scale, _stream
from .quant import Weight, kmoe_dtype


def rms_norm(
    x: torch.Tensor, scale: torch.Tensor, *, epsilon: float = 1e-6, out_dtype: torch.dtype | None = None
) -> torch.Tensor:
    """RMSNorm with a learnable ``scale`` (kappa/qwen3/norms.py:10-16): ``x * scale``
    after normalising by ``rsqrt(mean(x^2) + epsilon)``, computed in f32 and
    returned in ``x.dtype``."""
    if out_dtype is not None and out_dtype != x.dtype:
        raise ValueError(f"out_dtype must be x.dtype ({x.dtype}); got {out_dtype}")
    if x.device.type != "cuda":
        raise ValueError(f"x must be on a HIP device (got {x.device}); rms_norm has no CPU implementation")
    if x.dtype not in (torch.bfloat16, torch.float32):
        raise ValueError(f"x must be bfloat16 or float32 (got {x.dtype})")
    d = int(x.shape[-1])
    T = x.numel() // d if d else 0
    xf = x.reshape(T, d).contiguous()
    sc = _norm_scale(scale, d, x.device)
    out = torch.empty((T, d), dtype=x.dtype, device=x.device)
    desc = _desc(T, d, 1, 1, 1, x.dtype)
    _lib.check(
        _lib.lib().kmoe_rms_norm(
            desc, xf.data_ptr(), sc.data_ptr(), kmoe_dtype(sc.dtype), float(epsilon), out.data_ptr(), _stream(x.device)
        )
    )
    return out.reshape(x.shape)


def moe_block_ffn(
    h: torch.Tensor,
    pre_ffn_norm: torch.Tensor,
    router_w: Weight,
    ffn_gate: Weight,
    ffn_up: Weight,
    ffn_down: Weight,
    *,
    cfg: Qwen3Config,
    epsilon: float = 1e-6,
    packed: PackedExperts | None = None,
) -> torch.Tensor:
    """``h + moe_swiglu_ffn(rms_norm(h, pre_ffn_norm), ...)`` (kappa/qwen3/block.py:196-207).

    ``h`` is the residual stream ``[B, T, D]``; the result has its shape and dtype."""
    if not cfg.use_moe:
        raise ValueError("moe_swiglu_ffn requires cfg.use_moe")
    b, t = int(h.shape[0]), int(h.shape[1])
    impl, capacity = _impl_and_capacity(cfg, b * t)
    return _moe_forward(
        h, router_w, ffn_gate, ffn_up, ffn_down,
        num_experts=cfg.num_experts, num_experts_per_tok=cfg.num_experts_per_tok, impl=impl,
        decode_threshold=cfg.moe_ragged_decode_token_threshold, packed=packed, capacity=capacity,
        norm=(pre_ffn_norm, epsilon),
    )  # fmt: skip
