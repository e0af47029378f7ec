"""W8 weights: ``Q8Weight`` (int8 values + scale) and its helpers.

Mirrors kappa/qwen3/quant.py. ``Q8Weight.scale`` may be a scalar (the
reference's per-tensor scale, kappa/qwen3/quant.py:41-48) or one scale per
output channel (``[E, 1, N]`` for stacked ``[E, K, N]`` expert tensors,
``[1, E]`` or ``[E]`` for the ``[D, E]`` router). Dequantisation casts the
scale to the compute dtype before the multiply (kappa/qwen3/quant.py:37).
"""

from __future__ import annotations

from typing import NamedTuple, Union

import torch

from .. import _lib


class Q8Weight(NamedTuple):
    """Symmetric int8 weight: ``dequant = values * scale``."""

    values: torch.Tensor
    scale: torch.Tensor


Weight = Union[torch.Tensor, Q8Weight]


def is_q8_weight(w) -> bool:
    return isinstance(w, Q8Weight)


def weight_param_dtype(w: Weight) -> torch.dtype:
    """Dtype for activations (the Q8 scale dtype, or the array dtype) (kappa/qwen3/quant.py:28-31)."""
    return w.scale.dtype if is_q8_weight(w) else w.dtype


_TORCH_TO_KMOE = {torch.float32: _lib.DTYPE_F32, torch.bfloat16: _lib.DTYPE_BF16, torch.int8: _lib.DTYPE_I8}


def kmoe_dtype(t: torch.dtype) -> int:
    try:
        return _TORCH_TO_KMOE[t]
    except KeyError:
        raise ValueError(f"unsupported dtype {t}; expected float32, bfloat16 or int8") from None


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _require_cuda(t: torch.Tensor, name: str) -> None:
    if not isinstance(t, torch.Tensor) or t.device.type != "cuda":
        raise ValueError(f"{name} must be a torch tensor on a HIP device (got {getattr(t, 'device', type(t))})")


def scale_kind(w: Q8Weight, n_out: int, n_groups: int | None) -> int:
    """TENSOR for a one-element scale, CHANNEL for one scale per (group, output channel)."""
    s = w.scale
    if s.numel() == 1:
        return _lib.SCALE_TENSOR
    expect = n_out if n_groups is None else n_groups * n_out
    if s.numel() != expect or s.shape[-1] != n_out:
        raise ValueError(f"scale shape {tuple(s.shape)} is neither a scalar nor per output channel ({expect} values)")
    return _lib.SCALE_CHANNEL


def weight_struct(w: Weight, device: torch.device, *, n_out: int, n_groups: int | None, name: str):
    """Build the C ``kmoe_weight`` for ``w`` and return it with the tensors it points into."""
    if is_q8_weight(w):
        v = w.values
        _require_cuda(v, f"{name}.values")
        if v.dtype != torch.int8:
            raise ValueError(f"{name}.values must be int8 (got {v.dtype})")
        v = v.contiguous()
        s = w.scale
        if not isinstance(s, torch.Tensor):
            s = torch.tensor(s, dtype=torch.float32)
        if s.device != v.device:
            s = s.to(v.device)
        s = s.contiguous()
        kind = scale_kind(Q8Weight(v, s), n_out, n_groups)
        st = _lib.KmoeWeight(v.data_ptr(), _lib.DTYPE_I8, s.data_ptr(), kmoe_dtype(s.dtype), kind)
        return st, (v, s)
    _require_cuda(w, name)
    v = w.contiguous()
    if v.dtype not in (torch.float32, torch.bfloat16):
        raise ValueError(f"{name} must be float32, bfloat16 or a Q8Weight (got {v.dtype})")
    return _lib.KmoeWeight(v.data_ptr(), kmoe_dtype(v.dtype), None, _lib.DTYPE_F32, _lib.SCALE_NONE), (v,)


def to_compute_dtype(w: Weight, dtype: torch.dtype) -> torch.Tensor:
    """Dequantise a Q8 weight or cast a plain one (kappa/qwen3/quant.py:34-38), on the GPU."""
    if dtype not in (torch.float32, torch.bfloat16):
        raise ValueError(f"compute dtype must be float32 or bfloat16 (got {dtype})")
    v = w.values if is_q8_weight(w) else w
    shape = tuple(v.shape)
    channels = shape[-1] if len(shape) else 1
    outer = v.numel() // max(channels, 1)
    rows = shape[-2] if len(shape) >= 2 else 1
    n_groups = outer // rows if len(shape) >= 2 else None
    st, keep = weight_struct(w, v.device, n_out=channels, n_groups=n_groups, name="weight")
    out = torch.empty(shape, dtype=dtype, device=v.device)
    _lib.check(
        _lib.lib().kmoe_to_compute_dtype(
            st, outer, channels, rows, kmoe_dtype(dtype), out.data_ptr(), _stream(v.device)
        )
    )
    return out


def quantize_weight(w: torch.Tensor, *, scale_dtype: torch.dtype = torch.bfloat16) -> Q8Weight:
    """Per-tensor max-abs symmetric int8 (kappa/qwen3/quant.py:41-48).

    Offline post-training quantisation in the reference's own (per-tensor)
    format, written with plain tensor ops; it is not on the block's hot path."""
    w_f = w.to(torch.float32)
    amax = torch.max(torch.abs(w_f))
    scale = torch.clamp_min(amax / 127.0, torch.finfo(torch.float32).tiny)
    q = torch.clamp(torch.round(w_f / scale), -128.0, 127.0).to(torch.int8)
    return Q8Weight(values=q, scale=scale.to(scale_dtype))


def quantize_weight_per_channel(w: torch.Tensor, *, scale_dtype: torch.dtype = torch.float32) -> Q8Weight:
    """Per-output-channel symmetric int8 of a stacked ``[E, K, N]`` tensor, on the GPU.

    ``s[e, n] = max(max_k |w[e, k, n]| / 127, FLT_MIN)``, ``q = clip(rint(w / s), -128, 127)``:
    the reference's quantiser (kappa/qwen3/quant.py:41-48) with the max-abs taken
    per output channel. Returns ``Q8Weight(q [E,K,N] int8, scale [E,1,N])``."""
    _require_cuda(w, "w")
    if w.dim() == 2:  # [D, E] router: scale [1, E]
        q, s = quantize_weight_per_channel(w.unsqueeze(0), scale_dtype=scale_dtype)
        return Q8Weight(values=q[0], scale=s[0])
    if w.dim() != 3:
        raise ValueError(f"expected a stacked [E, K, N] tensor (got shape {tuple(w.shape)})")
    w = w.contiguous()
    E, K, N = w.shape
    q = torch.empty((E, K, N), dtype=torch.int8, device=w.device)
    s = torch.empty((E, 1, N), dtype=torch.float32, device=w.device)
    _lib.check(
        _lib.lib().kmoe_quantize_per_channel(
            E, K, N, w.data_ptr(), kmoe_dtype(w.dtype), q.data_ptr(), s.data_ptr(), _stream(w.device)
        )
    )
    return Q8Weight(values=q, scale=s.to(scale_dtype) if scale_dtype != torch.float32 else s)
