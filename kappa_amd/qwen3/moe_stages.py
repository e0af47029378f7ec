"""The block's stages as separate calls (kmoe_route / kmoe_dispatch /
kmoe_expert_ffn / kmoe_combine), for per-stage parity checks and profiling.

``moe_swiglu_ffn`` chains exactly these stages inside one C call. The expert
and combine stages take the array program whose rounding points they follow
(``impl``: "gather_einsum", "ragged" or "fixed_capacity"; the program that runs
after the decode switch, kappa/qwen3/ffn_moe.py:219-223).
"""

from __future__ import annotations

import ctypes

import torch

from .. import _lib
from .ffn_moe import PACK_CACHE, PackedExperts, _desc, _shape, _stream, packable
from .quant import Weight, weight_struct


def route(x_flat: torch.Tensor, router_w: Weight, *, num_experts: int, k: int, logits: bool = True) -> dict:
    """Router logits [T,E] f32, top-k indices [T,K] int32, weights [T,K] f32 (rounded to x.dtype), block histogram.

    logits=False: no logits; the call brings kmoe_route's scratch, so a bf16 router
    takes the two-phase form (MFMA logits, the canonical order for the experts near
    the K-th); the selections and weights are the same."""
    T, D = x_flat.shape
    dev = x_flat.device
    x_flat = x_flat.contiguous()
    desc = _desc(T, D, num_experts, k, 1, x_flat.dtype)
    r, keep = weight_struct(router_w, dev, n_out=num_experts, n_groups=None, name="router_w")
    lg = torch.empty((T, num_experts), dtype=torch.float32, device=dev) if logits else None
    idx = torch.empty((T, k), dtype=torch.int32, device=dev)
    w = torch.empty((T, k), dtype=torch.float32, device=dev)
    hist = torch.empty(((T + 63) // 64, num_experts), dtype=torch.int32, device=dev)
    scratch = None
    if not logits:
        n = _lib.ctypes.c_size_t()
        _lib.check(_lib.lib().kmoe_route_scratch_bytes(desc, _lib.ctypes.byref(n)))
        scratch = torch.empty(max(n.value, 1), dtype=torch.uint8, device=dev)
    _lib.check(
        _lib.lib().kmoe_route(
            desc, x_flat.data_ptr(), r, lg.data_ptr() if lg is not None else None,
            scratch.data_ptr() if scratch is not None else None, scratch.numel() if scratch is not None else 0,
            idx.data_ptr(), w.data_ptr(), hist.data_ptr(), _stream(dev),
        )
    )  # fmt: skip
    out = {"idx": idx, "w": w, "hist": hist}
    if lg is not None:
        out["logits"] = lg
    return out


def dispatch(idx: torch.Tensor, hist: torch.Tensor, *, num_experts: int, capacity: int = 0) -> dict:
    """Stable sort of the (t, j) assignments by expert. capacity > 0
    (fixed_capacity): inv is -1 for an assignment whose slot within its expert
    is >= capacity."""
    T, k = idx.shape
    dev = idx.device
    M = T * k
    desc = _desc(T, 1, num_experts, k, 1, torch.float32, impl="fixed_capacity" if capacity else "gather_einsum",
                 capacity=capacity)  # fmt: skip
    out = {
        "group_sizes": torch.empty(num_experts, dtype=torch.int32, device=dev),
        "offsets": torch.empty(num_experts + 1, dtype=torch.int32, device=dev),
        "active": torch.empty(num_experts + 1, dtype=torch.int32, device=dev),
        "sorted_token": torch.empty(M, dtype=torch.int32, device=dev),
        "sorted_expert": torch.empty(M, dtype=torch.int32, device=dev),
        "inv": torch.empty(M, dtype=torch.int32, device=dev),
    }
    _lib.check(
        _lib.lib().kmoe_dispatch(
            desc, idx.contiguous().data_ptr(), hist.contiguous().data_ptr(),
            *(out[n].data_ptr() for n in ("group_sizes", "offsets", "active", "sorted_token", "sorted_expert", "inv")),
            _stream(dev),
        )
    )  # fmt: skip
    return out


def _program(impl: str) -> str:
    """The MoEImpl name of an array program (ragged: ragged_jax, whose rounding points
    ragged_tokamax shares)."""
    names = {"gather_einsum": "gather_einsum", "ragged": "ragged_jax", "ragged_jax": "ragged_jax",
             "ragged_tokamax": "ragged_jax", "fixed_capacity": "fixed_capacity"}  # fmt: skip
    if impl not in names:
        raise ValueError(f"unknown impl {impl!r}")
    return names[impl]


def _stage_desc(T, D, E, k, I, act, impl, capacity=0, kernels=_lib.KERNELS_AUTO):
    # threshold -1: the named program runs at every token count
    return _desc(T, D, E, k, I, act, impl=_program(impl), threshold=-1, capacity=capacity, kernels=kernels)


def h_columns(impl: str, act: torch.dtype, I: int) -> int:
    """Columns of h_sorted: the ragged program's f32 h is two bf16 planes (hi, lo) per row."""
    return 2 * I if _program(impl) == "ragged_jax" and act == torch.bfloat16 else I


def expert_ffn(
    x_flat: torch.Tensor,
    disp: dict,
    ffn_gate: Weight,
    ffn_up: Weight,
    ffn_down: Weight,
    *,
    k: int,
    impl: str,
    packed: PackedExperts | None = None,
    layout_native: bool = False,
    capacity: int = 0,
    kernels: int = _lib.KERNELS_AUTO,
) -> tuple[torch.Tensor, torch.Tensor]:
    """SwiGLU experts over the sorted rows with ``impl``'s rounding points:
    (h_sorted, y_sorted [M, D] in x.dtype). h_sorted is [M, I] in x.dtype, or for
    the ragged program with bf16 activations [M, 2I] bf16 holding hi = bf16(h) and
    lo = bf16(h - hi) of its f32 h.

    ``layout_native=True`` runs the kernels that read the reference layout
    directly (one fmaf chain per output) instead of the packed MFMA kernels;
    ``kernels`` picks the packed family (``_lib.KERNELS_*``).
    ``capacity > 0``: the packed kernels compute only each expert's first
    ``capacity`` rows (the others are left as they were)."""
    T, D = x_flat.shape
    E, _, I = _shape(ffn_gate)
    dev = x_flat.device
    M = T * k
    if capacity:
        impl = "fixed_capacity"
    desc = _stage_desc(T, D, E, k, I, x_flat.dtype, impl, capacity, kernels)
    if not layout_native and packed is None and packable(x_flat.dtype, ffn_gate, ffn_up, ffn_down):
        packed = PACK_CACHE.get(ffn_gate, ffn_up, ffn_down)
    if layout_native:
        packed = None
    g, kg = weight_struct(ffn_gate, dev, n_out=I, n_groups=E, name="ffn_gate")
    u, ku = weight_struct(ffn_up, dev, n_out=I, n_groups=E, name="ffn_up")
    d, kd = weight_struct(ffn_down, dev, n_out=D, n_groups=E, name="ffn_down")
    h = torch.empty((M, h_columns(impl, x_flat.dtype, I)), dtype=x_flat.dtype, device=dev)
    y = torch.empty((M, D), dtype=x_flat.dtype, device=dev)
    _lib.check(
        _lib.lib().kmoe_expert_ffn(
            desc, x_flat.contiguous().data_ptr(), disp["offsets"].data_ptr(), disp["active"].data_ptr(),
            disp["sorted_token"].data_ptr(), disp["sorted_expert"].data_ptr(), g, u, d,
            packed.struct() if packed is not None else None, h.data_ptr(), y.data_ptr(), _stream(dev),
        )
    )  # fmt: skip
    return h, y


def h_float(h_sorted: torch.Tensor, I: int) -> torch.Tensor:
    """h_sorted as f32 [M, I] (hi + lo for the two-plane form)."""
    if h_sorted.shape[1] == 2 * I:
        return h_sorted[:, :I].float() + h_sorted[:, I:].float()
    return h_sorted.float()


def combine(y_sorted: torch.Tensor, inv: torch.Tensor, w: torch.Tensor, *, k: int, impl: str) -> torch.Tensor:
    """out[t] from the terms round(w[t,j] * y_sorted[inv[t*K+j]]): summed in f32 and
    rounded once (gather_einsum) or added into an x.dtype buffer (ragged, fixed_capacity)."""
    M, D = y_sorted.shape
    T = M // k
    dev = y_sorted.device
    desc = _stage_desc(T, D, max(k, 1), k, 1, y_sorted.dtype, impl, 1 if _program(impl) == "fixed_capacity" else 0)
    out = torch.empty((T, D), dtype=y_sorted.dtype, device=dev)
    _lib.check(
        _lib.lib().kmoe_combine(
            desc, y_sorted.contiguous().data_ptr(), inv.contiguous().data_ptr(),
            w.to(torch.float32).contiguous().data_ptr(), out.data_ptr(), _stream(dev),
        )
    )  # fmt: skip
    return out


def workspace_bytes(T: int, D: int, E: int, k: int, I: int, act: torch.dtype, impl: str = "ragged") -> int:
    n = ctypes.c_size_t()
    _lib.check(_lib.lib().kmoe_workspace_bytes(_stage_desc(T, D, E, k, I, act, impl), ctypes.byref(n)))
    return int(n.value)
