"""CPU oracle for the Qwen3 MoE feed-forward block -- TEST INFRASTRUCTURE ONLY.

This package is the checker the HIP library is compared against. Only
``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` import it; the product package ``kappa_amd`` never does.

It wraps ``liboracle_moe.so`` (built from ``moe_oracle.c`` by ``make`` in this
directory) with numpy. Every floating array is float32; bf16 values are carried
as float32 numbers that are exactly representable in bfloat16.

Weights are passed either as a plain float32 array or as a ``(q, s)`` pair of
int8 values and a float32 scale that broadcasts against the values with the
input axis reduced (per tensor: a scalar; per output channel: ``[E, 1, N]``),
mirroring ``Q8Weight`` (kappa/qwen3/quant.py:15-19).

Function -> reference it restates:
  router_logits   kappa/qwen3/ffn_moe.py:46-50   (_route logits)
  topk_softmax    kappa/qwen3/ffn_moe.py:51-55   (lax.top_k + softmax)
  dispatch        kappa/qwen3/ffn_moe.py:189-200, 212 (argsort stable, bincount, inv)
  expert_ffn      impl "gather_einsum": kappa/qwen3/ffn_moe.py:87-102 with
                  kappa/qwen3/quant.py:60-76; "fixed_capacity": :146-152;
                  "ragged": :202-213 (ragged_jax and ragged_tokamax)
  combine         "gather_einsum": :103; "ragged": :212-215; "fixed_capacity": :153-157
  forward         kappa/qwen3/ffn_moe.py:226-299 (moe_swiglu_ffn for one impl,
                  the one _effective_moe_impl, :219-223, selects; capacity= gives
                  the fixed_capacity drops, :107-158)
  effective_impl  kappa/qwen3/ffn_moe.py:219-223
  capacity_slots  kappa/qwen3/ffn_moe.py:23-31, 136-141 (c_buf and c_dyn)
  drop_over_capacity  kappa/qwen3/ffn_moe.py:59-71, 141, 153 (slot within expert, mask)
  quantize_*      kappa/qwen3/quant.py:41-48
  rms_norm        kappa/qwen3/norms.py:10-16 (squares summed in the router's slice order)
  residual_add    kappa/qwen3/block.py:207 (h + out)
  forward_block   kappa/qwen3/block.py:196-207 (rms_norm -> moe_swiglu_ffn -> residual)
"""

from __future__ import annotations

import ctypes
import math
import os
import subprocess
from typing import Any

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_SO = os.path.join(_HERE, "liboracle_moe.so")
_lib: ctypes.CDLL | None = None

_f32p = ctypes.POINTER(ctypes.c_float)
_i32p = ctypes.POINTER(ctypes.c_int32)
_i8p = ctypes.POINTER(ctypes.c_int8)
_i64 = ctypes.c_int64


def build() -> str:
    """Compile liboracle_moe.so with make (gcc). Returns the library path."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _SO


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_SO):
            build()
        L = ctypes.CDLL(_SO)
        L.orc_bf16_round.restype = ctypes.c_float
        L.orc_bf16_round.argtypes = [ctypes.c_float]
        L.orc_bf16_round_array.argtypes = [_i64, _f32p, _f32p]
        L.orc_set_threads.argtypes = [ctypes.c_int]
        L.orc_get_threads.restype = ctypes.c_int
        L.orc_router_logits.argtypes = [_i64, _i64, _i64, _f32p, _f32p, _i8p, _f32p, _f32p]
        L.orc_topk_softmax.argtypes = [_i64, _i64, _i64, ctypes.c_int, _f32p, _i32p, _f32p]
        L.orc_dispatch.argtypes = [_i64, _i64, _i64, _i32p, _i32p, _i32p, _i32p, _i32p, _i32p]
        L.orc_expert_ffn.argtypes = [_i64, _i64, _i64, _i64, _i64, ctypes.c_int, ctypes.c_int, _f32p, _i32p, _i32p] + [
            _f32p,
            _i8p,
            _f32p,
        ] * 3 + [_f32p, _f32p]
        L.orc_combine.argtypes = [_i64, _i64, _i64, ctypes.c_int, ctypes.c_int, _f32p, _i32p, _f32p, _f32p]
        L.orc_rms_norm.argtypes = [_i64, _i64, ctypes.c_int, _f32p, _f32p, ctypes.c_float, _f32p]
        L.orc_quantize_per_channel.argtypes = [_i64, _i64, _i64, _f32p, _i8p, _f32p]
        L.orc_quantize_per_tensor.restype = ctypes.c_float
        L.orc_quantize_per_tensor.argtypes = [_i64, _f32p, _i8p]
        _lib = L
    return _lib


def _p(a: np.ndarray | None, t):
    if a is None:
        return ctypes.cast(None, t)
    return a.ctypes.data_as(t)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def set_threads(n: int) -> None:
    lib().orc_set_threads(int(n))


def get_threads() -> int:
    return int(lib().orc_get_threads())


def bf16_round(a) -> np.ndarray:
    a = _f32(a)
    out = np.empty_like(a)
    lib().orc_bf16_round_array(a.size, _p(a, _f32p), _p(out, _f32p))
    return out


def _weight_parts(w: Any, n_out: int, n_exp: int | None):
    """Return (f, q, s_expanded) for a plain array or a (q, s) pair.

    ``s_expanded`` is float32 [n_exp, n_out] (or [n_out] for the router when n_exp is None)."""
    if isinstance(w, tuple):
        q, s = w
        q = np.ascontiguousarray(q, dtype=np.int8)
        s = np.asarray(s, dtype=np.float32)
        if n_exp is None:
            s_full = np.broadcast_to(s.reshape(-1) if s.ndim else s, (n_out,))
        else:
            s_full = np.broadcast_to(s.reshape(s.shape[0], s.shape[-1]) if s.ndim >= 2 else s, (n_exp, n_out))
        return None, q, np.ascontiguousarray(s_full, dtype=np.float32)
    return _f32(w), None, None


def router_logits(x, router) -> np.ndarray:
    """N0: canonical-order fp32 logits [T, E] (kappa/qwen3/ffn_moe.py:46-50)."""
    x = _f32(x)
    T, D = x.shape
    f, q, s = _weight_parts(router, (router[0] if isinstance(router, tuple) else router).shape[1], None)
    E = (q if f is None else f).shape[1]
    out = np.empty((T, E), np.float32)
    lib().orc_router_logits(T, D, E, _p(x, _f32p), _p(f, _f32p), _p(q, _i8p), _p(s, _f32p), _p(out, _f32p))
    return out


def topk_softmax(logits, k: int, act_bf16: bool):
    """N1/N2: (idx [T,K] int32, w [T,K] float32 rounded to the activation dtype)."""
    logits = _f32(logits)
    T, E = logits.shape
    idx = np.empty((T, k), np.int32)
    w = np.empty((T, k), np.float32)
    lib().orc_topk_softmax(T, E, k, int(act_bf16), _p(logits, _f32p), _p(idx, _i32p), _p(w, _f32p))
    return idx, w


def dispatch(idx, num_experts: int) -> dict:
    """N3: stable counting sort of assignments by expert."""
    idx = np.ascontiguousarray(idx, dtype=np.int32)
    T, K = idx.shape
    M = T * K
    gs = np.empty(num_experts, np.int32)
    off = np.empty(num_experts + 1, np.int32)
    order = np.empty(M, np.int32)
    st = np.empty(M, np.int32)
    inv = np.empty(M, np.int32)
    lib().orc_dispatch(
        T, K, num_experts, _p(idx, _i32p), _p(gs, _i32p), _p(off, _i32p), _p(order, _i32p), _p(st, _i32p), _p(inv, _i32p)
    )
    return {"group_sizes": gs, "offsets": off, "order": order, "sorted_token": st, "inv": inv}


# The three array programs of the reference's MoE layer (kappa/qwen3/ffn_moe.py):
# which rounding chain the expert products follow and how the combine adds.
IMPLS = ("gather_einsum", "ragged", "fixed_capacity")
_CHAIN = {"gather_einsum": 0, "fixed_capacity": 0, "ragged": 1}  # ORC_CHAIN_ACT / ORC_CHAIN_F32
_COMBINE = {"gather_einsum": 0, "fixed_capacity": 1, "ragged": 1}  # ORC_COMBINE_SUM / ORC_COMBINE_SCATTER


def _impl(impl: str) -> str:
    if impl in ("ragged_jax", "ragged_tokamax"):
        return "ragged"
    if impl not in IMPLS:
        raise ValueError(f"unknown impl {impl!r}; expected one of {IMPLS}")
    return impl


def effective_impl(moe_impl: str, total_tokens: int, threshold: int = 64) -> str:
    """_effective_moe_impl (kappa/qwen3/ffn_moe.py:219-223), in the oracle's names."""
    if moe_impl in ("ragged_jax", "ragged_tokamax"):
        return "gather_einsum" if total_tokens <= threshold else "ragged"
    return _impl(moe_impl)


def expert_ffn(x, offsets, sorted_token, gate, up, down, act_bf16: bool, *, impl: str):
    """(h_sorted [M, I], y_sorted [M, D]) for the sorted assignment rows, with the
    rounding points of ``impl``'s expert products (h is f32 under "ragged")."""
    chain = _CHAIN[_impl(impl)]
    x = _f32(x)
    T, D = x.shape
    offsets = np.ascontiguousarray(offsets, np.int32)
    sorted_token = np.ascontiguousarray(sorted_token, np.int32)
    E = offsets.shape[0] - 1
    gshape = (gate[0] if isinstance(gate, tuple) else gate).shape
    I = gshape[2]
    M = int(offsets[-1])
    gf, gq, gs = _weight_parts(gate, I, E)
    uf, uq, us = _weight_parts(up, I, E)
    df, dq, ds = _weight_parts(down, D, E)
    h = np.empty((M, I), np.float32)
    y = np.empty((M, D), np.float32)
    lib().orc_expert_ffn(
        T, D, E, 0, I, int(act_bf16), chain, _p(x, _f32p), _p(offsets, _i32p), _p(sorted_token, _i32p),
        _p(gf, _f32p), _p(gq, _i8p), _p(gs, _f32p),
        _p(uf, _f32p), _p(uq, _i8p), _p(us, _f32p),
        _p(df, _f32p), _p(dq, _i8p), _p(ds, _f32p),
        _p(h, _f32p), _p(y, _f32p),
    )  # fmt: skip
    return h, y


def combine(y_sorted, inv, w, act_bf16: bool, *, impl: str) -> np.ndarray:
    """out [T, D] from y_sorted rows inv[t*K+j] and weights w [T, K] (inv < 0: dropped):
    "gather_einsum" rounds each product and sums in f32 (:103); "ragged" and
    "fixed_capacity" add the rounded products into a zero buffer of x.dtype (:156-157, :214-215)."""
    mode = _COMBINE[_impl(impl)]
    y_sorted = _f32(y_sorted)
    w = _f32(w)
    inv = np.ascontiguousarray(inv, np.int32)
    T, K = w.shape
    D = y_sorted.shape[1]
    out = np.empty((T, D), np.float32)
    lib().orc_combine(T, K, D, int(act_bf16), mode, _p(y_sorted, _f32p), _p(inv, _i32p), _p(w, _f32p), _p(out, _f32p))
    return out


def capacity_slots(T: int, K: int, E: int, capacity_factor: float, fixed_slots: int | None = None) -> int:
    """fixed_capacity slot limit min(c_dyn, c_buf) for T flattened tokens.

    c_buf is the static buffer depth (kappa/qwen3/ffn_moe.py:23-31, with the
    8192-token bound of :20); c_dyn = max(1, round_half_even(f32(cf) *
    f32(T*K) / f32(E))) in float32 arithmetic (:136-139)."""
    if fixed_slots is not None:
        c_buf = max(1, int(fixed_slots))
    elif E <= 0 or K <= 0:
        c_buf = 1
    else:
        c_buf = max(1, int(math.ceil(capacity_factor * 8192 * K / E)))
    prod = np.float32(capacity_factor) * np.float32(T * K)
    c_dyn = max(1, int(np.round(np.float32(prod / np.float32(E)))))
    return min(c_dyn, c_buf)


def drop_over_capacity(idx, disp: dict, capacity: int) -> np.ndarray:
    """inv with -1 for each assignment whose slot within its expert (position in
    the stable order minus the expert's offset) is >= capacity."""
    idx = np.asarray(idx, np.int32).reshape(-1)
    inv = np.asarray(disp["inv"], np.int32).copy()
    slot = inv - np.asarray(disp["offsets"], np.int32)[idx]
    inv[slot >= capacity] = -1
    return inv


def forward(x, router, gate, up, down, *, k: int, act_bf16: bool, impl: str, capacity: int | None = None) -> dict:
    """Whole block on flattened tokens x [T, D] with the array program ``impl``
    ("gather_einsum", "ragged" or "fixed_capacity"); returns every intermediate.

    capacity: the fixed_capacity slot limit (impl "fixed_capacity" requires it)."""
    impl = _impl(impl)
    if (impl == "fixed_capacity") != (capacity is not None):
        raise ValueError("capacity is given exactly when impl is fixed_capacity")
    logits = router_logits(x, router)
    E = logits.shape[1]
    idx, w = topk_softmax(logits, k, act_bf16)
    disp = dispatch(idx, E)
    if capacity is not None:
        disp["inv"] = drop_over_capacity(idx, disp, capacity)
    h, y = expert_ffn(x, disp["offsets"], disp["sorted_token"], gate, up, down, act_bf16, impl=impl)
    out = combine(y, disp["inv"], w, act_bf16, impl=impl)
    return {"logits": logits, "idx": idx, "w": w, **disp, "h_sorted": h, "y_sorted": y, "out": out}


def rms_norm(h, scale, eps: float, act_bf16: bool) -> np.ndarray:
    """R1: rms_norm(h, scale, epsilon=eps) (kappa/qwen3/norms.py:10-16) in the
    canonical order, rounded to the activation dtype."""
    h = _f32(h)
    scale = _f32(scale).reshape(-1)
    T, D = h.shape
    if scale.shape[0] != D:
        raise ValueError(f"scale has {scale.shape[0]} entries, hidden size is {D}")
    out = np.empty((T, D), np.float32)
    lib().orc_rms_norm(T, D, int(act_bf16), _p(h, _f32p), _p(scale, _f32p), float(eps), _p(out, _f32p))
    return out


def residual_add(h, moe_out, act_bf16: bool) -> np.ndarray:
    """R2: round_act(f32(h) + f32(moe_out)) (the ``h + out`` of kappa/qwen3/block.py:207)."""
    s = (_f32(h) + _f32(moe_out)).astype(np.float32)
    return bf16_round(s) if act_bf16 else s


def forward_block(h, norm_scale, router, gate, up, down, *, k: int, act_bf16: bool, impl: str, eps: float = 1e-6,
                  capacity: int | None = None) -> dict:
    """h + moe_swiglu_ffn(rms_norm(h, norm_scale)) (kappa/qwen3/block.py:196-207)."""
    h2 = rms_norm(h, norm_scale, eps, act_bf16)
    moe = forward(h2, router, gate, up, down, k=k, act_bf16=act_bf16, impl=impl, capacity=capacity)
    return {**moe, "h2": h2, "moe_out": moe["out"], "out": residual_add(h, moe["out"], act_bf16)}


def quantize_per_channel(w):
    """A7 per output channel over [E, Kd, N]: (q int8, s float32 [E, 1, N])."""
    w = _f32(w)
    E, Kd, N = w.shape
    q = np.empty(w.shape, np.int8)
    s = np.empty((E, N), np.float32)
    lib().orc_quantize_per_channel(E, Kd, N, _p(w, _f32p), _p(q, _i8p), _p(s, _f32p))
    return q, s.reshape(E, 1, N)


def quantize_per_tensor(w):
    """A7 as in the reference (one scale): (q int8, s float32 scalar)."""
    w = _f32(w)
    q = np.empty(w.shape, np.int8)
    s = lib().orc_quantize_per_tensor(w.size, _p(w, _f32p), _p(q, _i8p))
    return q, np.float32(s)
