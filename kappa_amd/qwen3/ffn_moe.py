"""MoE SwiGLU feed-forward block on MI355X: the drop-in for kappa/qwen3/ffn_moe.py.

``moe_swiglu_ffn(x, router_w, ffn_gate, ffn_up, ffn_down, *, cfg)`` keeps the
reference signature (kappa/qwen3/ffn_moe.py:226-234) and its errors. Arrays are
torch tensors on a HIP device (bf16 or f32 activations ``[B, T, D]``); weights
are plain tensors or ``Q8Weight``. The block runs entirely in libkmoe.so:

  router logits -> top-k + softmax -> dispatch sort -> SwiGLU experts -> combine

W8 experts with bf16 activations are relaid out once (``prepack_moe_experts``)
for the MFMA kernels; the packed copy is cached per weight tensor so repeated
calls with the same weights do not repack. ``T <= cfg.moe_ragged_decode_token_threshold``
selects the decode kernels (the reference's decode switch, kappa/qwen3/ffn_moe.py:219-223);
every kernel family follows the same numerics, so the choice only affects speed.
"""

from __future__ import annotations

import math
import threading
from collections import OrderedDict
from dataclasses import dataclass

import numpy as np
import torch

from .. import _lib
from .architecture import Qwen3Config
from .quant import Q8Weight, Weight, is_q8_weight, kmoe_dtype, weight_struct

_MOE_IMPLS = ("gather_einsum", "fixed_capacity", "ragged_jax", "ragged_tokamax")

# Upper bound on B*T when deriving the static fixed_capacity buffer depth
# (kappa/qwen3/ffn_moe.py:20).
_MOE_FIXED_CAP_MAX_BT = 8192


def _fixed_capacity_buffer_slots(cfg: Qwen3Config) -> int:
    """Static per-expert buffer depth c_buf (kappa/qwen3/ffn_moe.py:23-31)."""
    if cfg.moe_fixed_capacity_slots is not None:
        return max(1, int(cfg.moe_fixed_capacity_slots))
    k, e = cfg.num_experts_per_tok, cfg.num_experts
    if e <= 0 or k <= 0:
        return 1
    cap = cfg.moe_capacity_factor * _MOE_FIXED_CAP_MAX_BT * k / e
    return max(1, int(math.ceil(cap)))


def _fixed_capacity(cfg: Qwen3Config, total_tokens: int) -> int:
    """Slot limit min(c_dyn, c_buf): c_dyn = max(1, round(f32(cf) * f32(B*T*K) / f32(E)))
    in float32 with round-half-even (kappa/qwen3/ffn_moe.py:136-141)."""
    k, e = cfg.num_experts_per_tok, cfg.num_experts
    prod = np.float32(cfg.moe_capacity_factor) * np.float32(total_tokens * k)
    c_dyn = max(1, int(np.round(np.float32(prod / np.float32(e)))))
    return min(c_dyn, _fixed_capacity_buffer_slots(cfg))


def _expert_count(w: Weight) -> int:
    """kappa/qwen3/ffn_moe.py:34-35."""
    return int(w.values.shape[0] if is_q8_weight(w) else w.shape[0])


def _effective_moe_impl(cfg: Qwen3Config, *, total_tokens: int) -> str:
    """kappa/qwen3/ffn_moe.py:219-223."""
    impl = cfg.moe_impl
    if impl in ("ragged_jax", "ragged_tokamax") and total_tokens <= cfg.moe_ragged_decode_token_threshold:
        return "gather_einsum"
    return impl


def _shape(w: Weight) -> tuple:
    return tuple((w.values if is_q8_weight(w) else w).shape)


@dataclass(frozen=True)
class PackedExperts:
    """W8 experts in the gfx950 layout (include/kmoe.h, kmoe_packed_experts)."""

    w13: torch.Tensor
    s13: torch.Tensor
    w2: torch.Tensor
    s2: torch.Tensor
    hidden: int
    intermediate: int
    num_experts: int

    def struct(self) -> _lib.KmoePacked:
        return _lib.KmoePacked(self.w13.data_ptr(), self.s13.data_ptr(), self.w2.data_ptr(), self.s2.data_ptr())


def _desc(
    T: int, D: int, E: int, K: int, I: int, act: torch.dtype, threshold: int, capacity: int = 0
) -> _lib.KmoeDesc:
    """kmoe_desc; capacity 0 is dropless, > 0 the fixed_capacity slot limit."""
    return _lib.KmoeDesc(T, D, E, K, I, kmoe_dtype(act), threshold, capacity)


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def packable(x_dtype: torch.dtype, gate: Weight, up: Weight, down: Weight) -> bool:
    """True when the MFMA kernels apply: bf16 activations, int8 experts, D and I multiples of 64."""
    if x_dtype != torch.bfloat16 or not all(is_q8_weight(w) for w in (gate, up, down)):
        return False
    E, D, I = _shape(gate)
    return D % 64 == 0 and I % 64 == 0


def prepack_moe_experts(ffn_gate: Q8Weight, ffn_up: Q8Weight, ffn_down: Q8Weight) -> PackedExperts:
    """One-time relayout of W8 experts ([E,D,I], [E,D,I], [E,I,D]) for the MFMA kernels."""
    E, D, I = _shape(ffn_gate)
    if _shape(ffn_up) != (E, D, I) or _shape(ffn_down) != (E, I, D):
        raise ValueError(
            f"expert shapes gate {_shape(ffn_gate)}, up {_shape(ffn_up)}, down {_shape(ffn_down)} "
            f"are not [E,D,I], [E,D,I], [E,I,D]"
        )
    dev = ffn_gate.values.device
    g, kg = weight_struct(ffn_gate, dev, n_out=I, n_groups=E, name="ffn_gate")
    u, ku = weight_struct(ffn_up, dev, n_out=I, n_groups=E, name="ffn_up")
    d, kd = weight_struct(ffn_down, dev, n_out=D, n_groups=E, name="ffn_down")
    desc = _desc(0, D, E, 1, I, torch.bfloat16, 0)
    sizes = _lib.KmoePackedSizes()
    L = _lib.lib()
    _lib.check(L.kmoe_prepack_bytes(desc, sizes))
    w13 = torch.empty(sizes.w13_bytes, dtype=torch.int8, device=dev)
    s13 = torch.empty(sizes.s13_bytes // 4, dtype=torch.float32, device=dev)
    w2 = torch.empty(sizes.w2_bytes, dtype=torch.int8, device=dev)
    s2 = torch.empty(sizes.s2_bytes // 4, dtype=torch.float32, device=dev)
    packed = PackedExperts(w13, s13, w2, s2, D, I, E)
    _lib.check(L.kmoe_prepack(desc, g, u, d, packed.struct(), _stream(dev)))
    return packed


class _PackCache:
    """Small LRU of packed experts keyed by the source tensors' storage and version."""

    def __init__(self, capacity: int = 4):
        self.capacity = capacity
        self._d: OrderedDict = OrderedDict()
        self._lock = threading.Lock()

    @staticmethod
    def key(*ws: Q8Weight) -> tuple:
        parts = []
        for w in ws:
            for t in (w.values, w.scale):
                if isinstance(t, torch.Tensor):
                    parts.append((t.data_ptr(), t._version, tuple(t.shape), t.dtype, t.device))
                else:
                    parts.append(("scalar", float(t)))
        return tuple(parts)

    def get(self, gate: Q8Weight, up: Q8Weight, down: Q8Weight) -> PackedExperts:
        k = self.key(gate, up, down)
        with self._lock:
            hit = self._d.get(k)
            if hit is not None:
                self._d.move_to_end(k)
                return hit
        packed = prepack_moe_experts(gate, up, down)
        with self._lock:
            self._d[k] = packed
            while len(self._d) > self.capacity:
                self._d.popitem(last=False)
        return packed

    def clear(self) -> None:
        with self._lock:
            self._d.clear()


PACK_CACHE = _PackCache()

_ws_lock = threading.Lock()
_workspaces: dict = {}


def _workspace(device: torch.device, stream: int, nbytes: int) -> torch.Tensor:
    """Per (device, stream) workspace that grows to the largest request (kernels are stream-ordered)."""
    key = (device.index, stream)
    with _ws_lock:
        ws = _workspaces.get(key)
        if ws is None or ws.numel() < nbytes:
            ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=device)
            _workspaces[key] = ws
        return ws


def _route_checks(x: torch.Tensor, router_w: Weight, num_experts: int) -> tuple[int, int, int]:
    """The validation in _route (kappa/qwen3/ffn_moe.py:45-49)."""
    if not isinstance(x, torch.Tensor) or x.dim() != 3:
        raise ValueError(f"x must be a [B, T, D] tensor (got {getattr(x, 'shape', type(x))})")
    b, t, d = x.shape
    rs = _shape(router_w)
    if rs != (d, num_experts):
        raise ValueError(f"router_w shape {rs} != ({d}, {num_experts})")
    return b, t, d


def _norm_scale(scale: torch.Tensor, d: int, dev: torch.device) -> torch.Tensor:
    """The RMSNorm scale as a contiguous [D] f32 or bf16 tensor on ``dev``."""
    if not isinstance(scale, torch.Tensor):
        raise ValueError("the norm scale must be a tensor")
    if scale.numel() != d:
        raise ValueError(f"norm scale has {scale.numel()} entries, hidden size is {d}")
    if scale.dtype not in (torch.bfloat16, torch.float32):
        scale = scale.to(torch.float32)
    return scale.reshape(d).to(dev).contiguous()


def _moe_forward(
    x: torch.Tensor,
    router_w: Weight,
    ffn_gate: Weight,
    ffn_up: Weight,
    ffn_down: Weight,
    *,
    num_experts: int,
    num_experts_per_tok: int,
    decode_threshold: int,
    packed: PackedExperts | None,
    return_routing: bool = False,
    capacity: int = 0,
    norm: tuple[torch.Tensor, float] | None = None,
):
    """The block through the C ABI. With ``norm = (scale, epsilon)``, ``x`` is the
    residual stream h and the call returns h + block(rms_norm(h)) (kmoe_forward_block)."""
    b, t, d = _route_checks(x, router_w, num_experts)
    if x.device.type != "cuda":
        raise ValueError(f"x must be on a HIP device (got {x.device}); the block has no CPU implementation")
    if x.dtype not in (torch.bfloat16, torch.float32):
        raise ValueError(f"x must be bfloat16 or float32 (got {x.dtype})")
    E, K = num_experts, num_experts_per_tok
    if _expert_count(ffn_gate) != E:
        raise ValueError(f"ffn_gate has {_expert_count(ffn_gate)} experts, cfg.num_experts is {E}")
    Eg, Dg, I = _shape(ffn_gate)
    if Dg != d or _shape(ffn_up) != (E, d, I) or _shape(ffn_down) != (E, I, d):
        raise ValueError(
            f"expert shapes gate {_shape(ffn_gate)}, up {_shape(ffn_up)}, down {_shape(ffn_down)} "
            f"do not match [E,D,I]/[E,I,D] with D={d}, E={E}"
        )
    dev = x.device
    T = b * t
    x_flat = x.reshape(T, d).contiguous()
    desc = _desc(T, d, E, K, I, x.dtype, decode_threshold, capacity)
    r, kr = weight_struct(router_w, dev, n_out=E, n_groups=None, name="router_w")
    if packed is None and packable(x.dtype, ffn_gate, ffn_up, ffn_down):
        packed = PACK_CACHE.get(ffn_gate, ffn_up, ffn_down)
    g, kg = weight_struct(ffn_gate, dev, n_out=I, n_groups=E, name="ffn_gate")
    u, ku = weight_struct(ffn_up, dev, n_out=I, n_groups=E, name="ffn_up")
    dn, kd = weight_struct(ffn_down, dev, n_out=d, n_groups=E, name="ffn_down")
    L = _lib.lib()
    nbytes = _lib.ctypes.c_size_t()
    _lib.check(L.kmoe_workspace_bytes(desc, _lib.ctypes.byref(nbytes)))
    stream = _stream(dev)
    ws = _workspace(dev, stream, nbytes.value)
    out = torch.empty((T, d), dtype=x.dtype, device=dev)
    idx = w_out = None
    if return_routing:
        idx = torch.empty((T, K), dtype=torch.int32, device=dev)
        w_out = torch.empty((T, K), dtype=x.dtype, device=dev)
    pk = packed.struct() if packed is not None else None
    idx_p = idx.data_ptr() if idx is not None else None
    w_p = w_out.data_ptr() if w_out is not None else None
    if norm is None:
        st = L.kmoe_forward(
            desc, x_flat.data_ptr(), r, g, u, dn, pk, out.data_ptr(), idx_p, w_p, ws.data_ptr(), ws.numel(), stream
        )
    else:
        scale, eps = norm
        scale = _norm_scale(scale, d, dev)
        st = L.kmoe_forward_block(
            desc, x_flat.data_ptr(), scale.data_ptr(), kmoe_dtype(scale.dtype), float(eps), r, g, u, dn, pk,
            out.data_ptr(), idx_p, w_p, ws.data_ptr(), ws.numel(), stream,
        )  # fmt: skip
    _lib.check(st)
    out = out.reshape(b, t, d)
    if return_routing:
        return out, idx, w_out
    return out


def moe_swiglu_ffn(
    x: torch.Tensor,
    router_w: Weight,
    ffn_gate: Weight,
    ffn_up: Weight,
    ffn_down: Weight,
    *,
    cfg: Qwen3Config,
    packed: PackedExperts | None = None,
) -> torch.Tensor:
    """MoE SwiGLU forward (kappa/qwen3/ffn_moe.py:226-299).

    Shapes: ``router_w`` ``[D, E]``; ``ffn_*`` ``[E, D, I]`` / ``[E, I, D]`` for
    gate/up/down. Returns ``[B, T, D]`` in ``x.dtype``. ``packed`` optionally
    supplies experts already relaid out by ``prepack_moe_experts``.
    """
    if not cfg.use_moe:
        raise ValueError("moe_swiglu_ffn requires cfg.use_moe")
    _route_checks(x, router_w, cfg.num_experts)
    b, t = int(x.shape[0]), int(x.shape[1])
    impl = _effective_moe_impl(cfg, total_tokens=b * t)
    if impl not in _MOE_IMPLS:
        raise ValueError(f"unknown moe_impl: {impl!r}")
    capacity = 0
    if impl == "fixed_capacity":
        if cfg.moe_capacity_factor <= 0:
            raise ValueError("fixed_capacity requires cfg.moe_capacity_factor > 0")
        # token dropping: the dropless kernels with each expert limited to its
        # first `capacity` assignments in the stable (expert, token) order
        capacity = _fixed_capacity(cfg, b * t)
    # gather_einsum, ragged_jax and ragged_tokamax are dropless and share one numerics contract here.
    return _moe_forward(
        x, router_w, ffn_gate, ffn_up, ffn_down,
        num_experts=cfg.num_experts, num_experts_per_tok=cfg.num_experts_per_tok,
        decode_threshold=cfg.moe_ragged_decode_token_threshold, packed=packed, capacity=capacity,
    )  # fmt: skip


def moe_swiglu_ffn_legacy(
    x: torch.Tensor,
    router_w: Weight,
    ffn_gate: Weight,
    ffn_up: Weight,
    ffn_down: Weight,
    *,
    num_experts: int,
    num_experts_per_tok: int,
) -> torch.Tensor:
    """Backward-compatible API with explicit expert counts (kappa/qwen3/ffn_moe.py:302-316)."""
    return _moe_forward(
        x, router_w, ffn_gate, ffn_up, ffn_down,
        num_experts=num_experts, num_experts_per_tok=num_experts_per_tok,
        decode_threshold=64, packed=None,
    )  # fmt: skip
