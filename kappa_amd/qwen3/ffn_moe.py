"""MoE SwiGLU feed-forward block on MI355X: the drop-in for kappa/qwen3/ffn_moe.py.

``moe_swiglu_ffn(x, router_w, ffn_gate, ffn_up, ffn_down, *, cfg)`` keeps the
reference signature (kappa/qwen3/ffn_moe.py:226-234) and its errors. Arrays are
torch tensors on a HIP device (bf16 or f32 activations ``[B, T, D]``); weights
are plain tensors or ``Q8Weight``. The block runs entirely in libkmoe.so:

  router logits -> top-k + softmax -> dispatch sort -> SwiGLU experts -> combine

Each ``cfg.moe_impl`` keeps its own rounding points, as the reference's array
programs write them: ``gather_einsum`` (the default, and what ``ragged_jax`` /
``ragged_tokamax`` run at ``T <= cfg.moe_ragged_decode_token_threshold``,
kappa/qwen3/ffn_moe.py:219-223) computes the expert products in x.dtype and sums
the rounded weighted terms in f32; ``ragged_*`` above the threshold computes
them in f32 and adds the rounded terms into an x.dtype buffer; ``fixed_capacity``
drops assignments beyond each expert's slot limit, computes in x.dtype and adds
like the ragged path. The gather program takes per-tensor scales only
(kappa/qwen3/quant.py:71-74), so per-output-channel W8 weights run with
``ragged_*`` (a threshold of 0 for decode batches) or ``fixed_capacity``.

The kernel family (GEMV-style up to 64 tokens, grouped GEMMs above) is chosen
by token count, independently of the impl; the families follow the same
rounding points but add the f32 products in different orders, so they agree
to rounding, not bit for bit. W8 experts with bf16 activations are relaid out
once for the MFMA kernels: ``prepack_moe_experts`` at load time (pass the result
as ``packed=``), or implicitly through a cache keyed by the weight tensors.
"""

from __future__ import annotations

import math
import threading
import warnings
import weakref
from collections import OrderedDict
from dataclasses import dataclass

import numpy as np
import torch

from .. import _lib
from .architecture import Qwen3Config
from .quant import Q8Weight, Weight, is_q8_weight, kmoe_dtype, scale_kind, weight_struct

_MOE_IMPLS = ("gather_einsum", "fixed_capacity", "ragged_jax", "ragged_tokamax")
# kmoe_impl of each MoEImpl (kappa/qwen3/architecture.py:14)
_IMPL_CODE = {
    "gather_einsum": _lib.IMPL_GATHER_EINSUM,
    "fixed_capacity": _lib.IMPL_FIXED_CAPACITY,
    "ragged_jax": _lib.IMPL_RAGGED,
    "ragged_tokamax": _lib.IMPL_RAGGED,
}

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
    source_scale_kind: int  # _lib.SCALE_TENSOR or _lib.SCALE_CHANNEL

    @property
    def nbytes(self) -> int:
        return sum(t.numel() * t.element_size() for t in (self.w13, self.s13, self.w2, self.s2))

    def struct(self) -> _lib.KmoePacked:
        return _lib.KmoePacked(
            self.w13.data_ptr(), self.s13.data_ptr(), self.w2.data_ptr(), self.s2.data_ptr(), self.num_experts,
            self.hidden, self.intermediate, self.source_scale_kind,
        )  # fmt: skip


def _desc(
    T: int, D: int, E: int, K: int, I: int, act: torch.dtype, *, impl: str = "gather_einsum", threshold: int = 64,
    capacity: int = 0, kernels: int = _lib.KERNELS_AUTO,
) -> _lib.KmoeDesc:
    """kmoe_desc for the MoEImpl ``impl`` (capacity: the fixed_capacity slot limit)."""
    return _lib.KmoeDesc(T, D, E, K, I, kmoe_dtype(act), _IMPL_CODE[impl], threshold, capacity, kernels)


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def packable(x_dtype: torch.dtype, gate: Weight, up: Weight, down: Weight) -> bool:
    """True when the MFMA kernels apply: bf16 activations, int8 experts, D and I multiples of 64."""
    if x_dtype != torch.bfloat16 or not all(is_q8_weight(w) for w in (gate, up, down)):
        return False
    E, D, I = _shape(gate)
    return D % 64 == 0 and I % 64 == 0


def _source_scale_kind(ws, n_outs, E) -> int:
    kinds = [scale_kind(w, n, E) for w, n in zip(ws, n_outs)]
    return _lib.SCALE_TENSOR if all(k == _lib.SCALE_TENSOR for k in kinds) else _lib.SCALE_CHANNEL


def prepack_moe_experts(ffn_gate: Q8Weight, ffn_up: Q8Weight, ffn_down: Q8Weight) -> PackedExperts:
    """One-time relayout of W8 experts ([E,D,I], [E,D,I], [E,I,D]) for the MFMA kernels.

    The load-time step: run it once per layer when the weights are loaded (next to
    the reference's quantize_qwen3_params, kappa/qwen3/weights.py:143-188) and pass
    the result to ``moe_swiglu_ffn(..., packed=)``. The packed copy holds the same
    int8 values and the scales as given; it does not follow later in-place writes
    to the source tensors."""
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
    desc = _desc(0, D, E, 1, I, torch.bfloat16)
    sizes = _lib.KmoePackedSizes()
    L = _lib.lib()
    _lib.check(L.kmoe_prepack_bytes(desc, sizes))
    w13 = torch.empty(sizes.w13_bytes, dtype=torch.int8, device=dev)
    s13 = torch.empty(sizes.s13_bytes // 4, dtype=torch.float32, device=dev)
    w2 = torch.empty(sizes.w2_bytes, dtype=torch.int8, device=dev)
    s2 = torch.empty(sizes.s2_bytes // 4, dtype=torch.float32, device=dev)
    kind = _source_scale_kind((ffn_gate, ffn_up, ffn_down), (I, I, D), E)
    packed = PackedExperts(w13, s13, w2, s2, D, I, E, kind)
    _lib.check(L.kmoe_prepack(desc, g, u, d, packed.struct(), _stream(dev)))
    return packed


class _PackCache:
    """Packed experts for weights passed without ``packed=``, keyed by the source tensors.

    An entry lives as long as all of its source tensors (values and scales of
    gate, up and down): it holds only weak references to them and is dropped when
    any of them is freed, so a new tensor that reuses a freed address can never
    hit an old entry. A hit also requires every source's ``_version`` to be
    unchanged (torch in-place ops).

    Each entry is a second copy of a layer's experts next to the caller's source
    tensors, so the cache is bounded twice, least recently used first out:
    ``max_entries`` entries, and ``max_bytes`` bytes of packed weights per device
    (default: ``max_fraction`` of the device's memory). A whole large model does
    not fit twice in one GPU (235B-A22B holds ~2.4 GB of W8 experts per layer, 94
    layers): such models should call ``prepack_moe_experts`` once per layer at load
    time, pass ``packed=`` and free the source int8 tensors. The first eviction
    for lack of room warns once."""

    def __init__(self, max_entries: int = 256, max_bytes: int | None = None, max_fraction: float = 0.4):
        self.max_entries = max_entries
        self.max_bytes = max_bytes
        self.max_fraction = max_fraction
        self._d: OrderedDict = OrderedDict()
        self._lock = threading.RLock()
        self.packs = 0  # prepack calls made (a miss)
        self.evicted_for_room = 0
        self._warned = False

    def _budget(self, device: torch.device) -> int:
        if self.max_bytes is not None:
            return self.max_bytes
        return int(self.max_fraction * torch.cuda.get_device_properties(device).total_memory)

    def _device_bytes(self, device: torch.device) -> int:
        return sum(p.nbytes for _, _, p in self._d.values() if p.w13.device == device)

    def _make_room(self, device: torch.device, keep) -> None:
        """Evict the least recently used entries of ``device`` beyond the byte budget."""
        budget = self._budget(device)
        while self._device_bytes(device) > budget:
            victim = next((k for k, (_, _, p) in self._d.items() if p.w13.device == device and k != keep), None)
            if victim is None:
                return
            del self._d[victim]
            self.evicted_for_room += 1
            if not self._warned:
                self._warned = True
                warnings.warn(
                    "kappa_amd: the implicit prepack cache exceeded its budget of "
                    f"{budget / 2**30:.1f} GiB on {device} and evicts layers, which are packed again on their next "
                    "call; call prepack_moe_experts() at load time, pass packed= and free the source int8 tensors",
                    ResourceWarning,
                    stacklevel=3,
                )

    @staticmethod
    def _sources(ws) -> tuple[list, tuple]:
        """The source tensors, and the values of scales given as Python numbers."""
        src, scalars = [], []
        for w in ws:
            for t in (w.values, w.scale):
                if isinstance(t, torch.Tensor):
                    src.append(t)
                else:
                    scalars.append(float(t))
        return src, tuple(scalars)

    def _evict(self, key) -> None:
        with self._lock:
            self._d.pop(key, None)

    def get(self, gate: Q8Weight, up: Q8Weight, down: Q8Weight) -> PackedExperts:
        src, scalars = self._sources((gate, up, down))
        key = tuple(id(t) for t in src) + scalars
        stamp = tuple((t._version, t.data_ptr()) for t in src)
        with self._lock:
            ent = self._d.get(key)
            if ent is not None:
                refs, st, packed = ent
                if all(r() is t for r, t in zip(refs, src)) and st == stamp:
                    self._d.move_to_end(key)
                    return packed
                del self._d[key]
        packed = prepack_moe_experts(gate, up, down)
        with self._lock:
            self.packs += 1
            self._d[key] = ([weakref.ref(t) for t in src], stamp, packed)
            for t in src:
                weakref.finalize(t, self._evict, key)
            while len(self._d) > self.max_entries:
                self._d.popitem(last=False)
            self._make_room(packed.w13.device, key)
        return packed

    def __len__(self) -> int:
        return len(self._d)

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


def _check_packed(packed: PackedExperts, E: int, d: int, I: int, dev: torch.device) -> None:
    """A packed copy must hold this layer's shapes, on x's device."""
    if not isinstance(packed, PackedExperts):
        raise ValueError(f"packed must be a PackedExperts from prepack_moe_experts (got {type(packed).__name__})")
    if (packed.num_experts, packed.hidden, packed.intermediate) != (E, d, I):
        raise ValueError(
            f"packed experts hold E={packed.num_experts}, D={packed.hidden}, I={packed.intermediate}; "
            f"the layer has E={E}, D={d}, I={I}"
        )
    for name in ("w13", "s13", "w2", "s2"):
        if getattr(packed, name).device != dev:
            raise ValueError(f"packed.{name} is on {getattr(packed, name).device}, x is on {dev}")


def _check_gather_scales(impl: str, ws, n_outs, E: int) -> None:
    """The gather program (moe_take_dequant, kappa/qwen3/quant.py:71-74) multiplies the
    gathered [T, K, D, I] values by the scale as stored: it takes a per-tensor scale
    (or one expert's [1, 1, N]), not per-expert per-channel scales."""
    if impl != "gather_einsum" or E <= 1:
        return
    for w, n in zip(ws, n_outs):
        if is_q8_weight(w) and scale_kind(w, n, E) == _lib.SCALE_CHANNEL:
            raise _gather_scale_error()


def _gather_scale_error() -> ValueError:
    return ValueError(
        "gather_einsum takes one scale per tensor (kappa/qwen3/quant.py:71-74); per-channel scales run "
        "with moe_impl='ragged_jax' / 'ragged_tokamax' (moe_ragged_decode_token_threshold=0 for decode "
        "batches) or 'fixed_capacity'"
    )


def _moe_forward(
    x: torch.Tensor,
    router_w: Weight,
    ffn_gate: Weight,
    ffn_up: Weight,
    ffn_down: Weight,
    *,
    num_experts: int,
    num_experts_per_tok: int,
    impl: str,
    decode_threshold: int,
    packed: PackedExperts | None,
    return_routing: bool = False,
    capacity: int = 0,
    norm: tuple[torch.Tensor, float] | None = None,
    kernels: int = _lib.KERNELS_AUTO,
):
    """The block through the C ABI for the MoEImpl ``impl`` (the configured one; the
    library applies the decode switch). With ``norm = (scale, epsilon)``, ``x`` is the
    residual stream h and the call returns h + block(rms_norm(h)) (kmoe_forward_block)."""
    b, t, d = _route_checks(x, router_w, num_experts)
    E, K = num_experts, num_experts_per_tok
    T = b * t
    effective = _effective_moe_impl(
        Qwen3ConfigView(impl, decode_threshold), total_tokens=T
    )  # the program that runs (kappa/qwen3/ffn_moe.py:219-223)
    sources = (ffn_gate, ffn_up, ffn_down)
    if any(w is None for w in sources):
        # the packed copy alone (the source int8 tensors freed after a load-time prepack)
        if packed is None or any(w is not None for w in sources):
            raise ValueError("ffn_gate, ffn_up and ffn_down may be None only all together, with packed=")
        if not isinstance(packed, PackedExperts):
            raise ValueError(f"packed must be a PackedExperts from prepack_moe_experts (got {type(packed).__name__})")
        I = packed.intermediate
        if effective == "gather_einsum" and E > 1 and packed.source_scale_kind == _lib.SCALE_CHANNEL:
            raise _gather_scale_error()
    else:
        if _expert_count(ffn_gate) != E:
            raise ValueError(f"ffn_gate has {_expert_count(ffn_gate)} experts, cfg.num_experts is {E}")
        Eg, Dg, I = _shape(ffn_gate)
        if Dg != d or _shape(ffn_up) != (E, d, I) or _shape(ffn_down) != (E, I, d):
            raise ValueError(
                f"expert shapes gate {_shape(ffn_gate)}, up {_shape(ffn_up)}, down {_shape(ffn_down)} "
                f"do not match [E,D,I]/[E,I,D] with D={d}, E={E}"
            )
        _check_gather_scales(effective, sources, (I, I, d), E)
    dev = x.device
    if packed is not None:
        _check_packed(packed, E, d, I, dev)
    if dev.type != "cuda":
        raise ValueError(f"x must be on a HIP device (got {dev}); the block has no CPU implementation")
    if x.dtype not in (torch.bfloat16, torch.float32):
        raise ValueError(f"x must be bfloat16 or float32 (got {x.dtype})")
    x_flat = x.reshape(T, d).contiguous()
    desc = _desc(T, d, E, K, I, x.dtype, impl=impl, threshold=decode_threshold, capacity=capacity, kernels=kernels)
    r, kr = weight_struct(router_w, dev, n_out=E, n_groups=None, name="router_w")
    if packed is None and packable(x.dtype, ffn_gate, ffn_up, ffn_down):
        packed = PACK_CACHE.get(ffn_gate, ffn_up, ffn_down)
    if ffn_gate is None:
        if x.dtype != torch.bfloat16:
            raise ValueError("packed experts alone run with bfloat16 activations")
        g = u = dn = None
    else:
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


@dataclass(frozen=True)
class Qwen3ConfigView:
    """The two Qwen3Config fields _effective_moe_impl reads."""

    moe_impl: str
    moe_ragged_decode_token_threshold: int


def _impl_and_capacity(cfg: Qwen3Config, total_tokens: int) -> tuple[str, int]:
    """The configured impl (validated, kappa/qwen3/ffn_moe.py:250-252, 299) and its slot limit."""
    impl = cfg.moe_impl
    if impl not in _MOE_IMPLS:
        raise ValueError(f"unknown moe_impl: {impl!r}")
    capacity = 0
    if _effective_moe_impl(cfg, total_tokens=total_tokens) == "fixed_capacity":
        if cfg.moe_capacity_factor <= 0:
            raise ValueError("fixed_capacity requires cfg.moe_capacity_factor > 0")
        # token dropping: each expert keeps its first `capacity` assignments in the
        # stable (expert, token) order
        capacity = _fixed_capacity(cfg, total_tokens)
    return impl, capacity


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
    """MoE SwiGLU forward (kappa/qwen3/ffn_moe.py:226-299); implementation selected by
    ``cfg.moe_impl`` (and the decode threshold).

    Shapes: ``router_w`` ``[D, E]``; ``ffn_*`` ``[E, D, I]`` / ``[E, I, D]`` for
    gate/up/down. Returns ``[B, T, D]`` in ``x.dtype``. ``packed`` optionally
    supplies experts already relaid out by ``prepack_moe_experts``; with it,
    ``ffn_gate``, ``ffn_up`` and ``ffn_down`` may all be None (a model that
    prepacked at load time and freed the int8 sources).
    """
    if not cfg.use_moe:
        raise ValueError("moe_swiglu_ffn requires cfg.use_moe")
    _route_checks(x, router_w, cfg.num_experts)
    b, t = int(x.shape[0]), int(x.shape[1])
    impl, capacity = _impl_and_capacity(cfg, b * t)
    return _moe_forward(
        x, router_w, ffn_gate, ffn_up, ffn_down,
        num_experts=cfg.num_experts, num_experts_per_tok=cfg.num_experts_per_tok, impl=impl,
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
    """Backward-compatible API: always the gather program, whatever a config says
    (kappa/qwen3/ffn_moe.py:302-316)."""
    return _moe_forward(
        x, router_w, ffn_gate, ffn_up, ffn_down,
        num_experts=num_experts, num_experts_per_tok=num_experts_per_tok, impl="gather_einsum",
        decode_threshold=64, packed=None,
    )  # fmt: skip
