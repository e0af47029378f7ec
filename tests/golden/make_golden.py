#!/usr/bin/env python3
"""Write the golden vectors in this directory.

The expected values come from a literal numpy/torch-CPU transliteration of the
reference layer's array programs -- not from the C oracle -- so the oracle is
checked against an independent restatement. Each program is restated one jnp
operation at a time, each operation rounding its result to its array dtype:

  _route               kappa/qwen3/ffn_moe.py:38-56  (einsum -> lax.top_k -> softmax)
  to_compute_dtype     kappa/qwen3/quant.py:34-38    (values.astype(dt) * scale.astype(dt))
  moe_take_dequant     kappa/qwen3/quant.py:60-76
  _moe_gather_einsum   kappa/qwen3/ffn_moe.py:74-104 (bf16 weights, g, u, silu, h, y_k,
                       the bf16 product y_k * w and jnp.sum over k, which accumulates
                       a bf16 array in float32 and rounds once)
  _moe_ragged          kappa/qwen3/ffn_moe.py:174-216 (float32 weights with the float32
                       scale, float32 g, u, h and y; y.astype(bf16); the bf16 product
                       y * w; .at[token].add into a bf16 zero buffer, one rounding per
                       update, the updates of a token in j order)
  _moe_fixed_capacity  kappa/qwen3/ffn_moe.py:107-158 with _slot_within_expert :59-71
                       and _fixed_capacity_buffer_slots :23-31 (bf16 weights, the
                       [E, C, D] buffer, the same bf16 scatter-add combine as ragged)
  rms_norm             kappa/qwen3/norms.py:10-16
  block MoE half       kappa/qwen3/block.py:196-207 (h2 = rms_norm(h); h + moe(h2))

Dot products (einsum, ragged_dot) accumulate in float64 and are rounded to their
array dtype (through float32 for bf16, as an f32 accumulator would be); the
elementwise operations run on torch CPU tensors of the array dtype, which round
every result (bfloat16 round-to-nearest-even). ``jax`` is not installed here,
so the reference itself cannot be executed; this restatement stands in for it.

Usage: python tests/golden/make_golden.py   (rewrites *.npz and golden.json)
"""

from __future__ import annotations

import json
import math
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
from inputs import BLOCK_SPECS, CAPACITY_SPECS, GOLDEN_SPECS, Spec, digest, make_inputs, make_norm_scale  # noqa: E402


def tdt(act: str) -> torch.dtype:
    return torch.bfloat16 if act == "bf16" else torch.float32


def as_t(a, dt: torch.dtype) -> torch.Tensor:
    """``.astype(dt)`` of a float array: float32 rounding first, then bf16 RNE for bf16."""
    return torch.from_numpy(np.ascontiguousarray(np.asarray(a, dtype=np.float32))).to(dt)


def dot64(a: torch.Tensor, b: torch.Tensor, dt: torch.dtype) -> torch.Tensor:
    """A matmul whose operands and result carry dtype dt: exact products summed in
    float64, rounded to float32 and then to dt."""
    return (a.double() @ b.double()).float().to(dt)


def to_compute_dtype(w, dt: torch.dtype) -> torch.Tensor:
    """kappa/qwen3/quant.py:34-38: values.astype(dt) * scale.astype(dt), or w.astype(dt)."""
    if isinstance(w, tuple):
        q, s = w
        qv = torch.from_numpy(np.ascontiguousarray(q)).to(dt)
        sv = as_t(np.asarray(s, np.float32), dt)
        return qv * sv  # a dt multiply, broadcasting a scalar or [E, 1, N]
    return as_t(w, dt)


def silu_mul(g: torch.Tensor, u: torch.Tensor) -> torch.Tensor:
    """jax.nn.silu(g) * u with silu(g) = g * sigmoid(g): three dt operations."""
    return (g * torch.sigmoid(g)) * u


def route(spec: Spec, inp: dict) -> dict:
    """_route (kappa/qwen3/ffn_moe.py:38-56): float64 logits (the fp32 einsum up to its
    summation order), top-k with ties to the lower index, softmax, .astype(x.dtype)."""
    x = inp["x"]
    T = x.shape[0]
    E, K = spec.E, spec.K
    r = inp["router"]
    rw = (r[0].astype(np.float32) * np.asarray(r[1], np.float32)) if isinstance(r, tuple) else np.asarray(r, np.float32)
    logits = x.astype(np.float64) @ rw.astype(np.float64)
    order_e = np.lexsort((np.broadcast_to(np.arange(E), (T, E)), -logits), axis=-1)
    top_idx = order_e[:, :K].astype(np.int32)
    top_l = np.take_along_axis(logits, top_idx.astype(np.int64), axis=-1)
    ex = np.exp(top_l - top_l[:, :1])
    w = as_t(ex / ex.sum(axis=-1, keepdims=True), tdt(spec.act))
    srt = np.take_along_axis(logits, order_e.astype(np.int64), axis=-1)
    gap = (srt[:, K - 1] - srt[:, K]) if K < E else np.full(T, np.inf)
    return {"logits64": logits, "idx": top_idx, "w": w, "gap": gap}


def sort_assignments(idx: np.ndarray, E: int) -> dict:
    """The stable order of :196-200, 212 (argsort(stable), bincount, inv)."""
    M = idx.size
    expert_flat = idx.reshape(M)
    order = np.argsort(expert_flat, kind="stable").astype(np.int32)
    inv = np.zeros(M, np.int32)
    inv[order] = np.arange(M, dtype=np.int32)
    return {"order": order, "group_sizes": np.bincount(expert_flat, minlength=E).astype(np.int32), "inv": inv}


def gather_einsum(spec: Spec, inp: dict, rt: dict) -> dict:
    """_moe_gather_einsum (kappa/qwen3/ffn_moe.py:74-104), one (token, k) pair at a time."""
    dt = tdt(spec.act)
    x = as_t(inp["x"], dt)
    T, K = rt["idx"].shape
    for n in ("gate", "up", "down"):
        w = inp[n]
        if isinstance(w, tuple) and np.asarray(w[1]).size != 1:
            raise ValueError("the gather path takes a per-tensor scale (kappa/qwen3/quant.py:71-74)")
    wg, wu, wd = (to_compute_dtype(inp[n], dt) for n in ("gate", "up", "down"))
    h = torch.empty((T, K, spec.I), dtype=dt)
    y_k = torch.empty((T, K, spec.D), dtype=dt)
    for t in range(T):
        for k in range(K):
            e = int(rt["idx"][t, k])
            g = dot64(x[t : t + 1], wg[e], dt)
            u = dot64(x[t : t + 1], wu[e], dt)
            h[t, k] = silu_mul(g, u)[0]
            y_k[t, k] = dot64(h[t, k : k + 1], wd[e], dt)[0]
    p = y_k * rt["w"][:, :, None]  # y_k * w[..., None] in dt
    out = p.float().sum(dim=1).to(dt)  # jnp.sum: float32 accumulation, one rounding
    return {"h": h, "y_k": y_k, "out": out}


def scatter_add_combine(y_assign: torch.Tensor, w: torch.Tensor, T: int, K: int) -> torch.Tensor:
    """out_flat = zeros(dt).at[token_flat].add(y_assign * w_flat[:, None]) with
    token_flat = m // K: the update of assignment m = t*K + j is added to row t in m
    order, each add rounded to dt."""
    p = y_assign.reshape(T, K, -1) * w[:, :, None]
    out = torch.zeros((T, y_assign.shape[-1]), dtype=y_assign.dtype)
    for j in range(K):
        out = out + p[:, j]
    return out


def ragged(spec: Spec, inp: dict, rt: dict, srt: dict) -> dict:
    """_moe_ragged (kappa/qwen3/ffn_moe.py:174-216)."""
    dt = tdt(spec.act)
    T, K = rt["idx"].shape
    M = T * K
    expert_flat = rt["idx"].reshape(M)
    token_flat = np.repeat(np.arange(T, dtype=np.int32), K)
    order = srt["order"]
    sorted_e = expert_flat[order]
    lhs_f = as_t(inp["x"], dt)[torch.from_numpy(token_flat[order].astype(np.int64))].float()  # sorted_x.astype(f32)
    wg, wu, wd = (to_compute_dtype(inp[n], torch.float32) for n in ("gate", "up", "down"))
    g_out = torch.empty((M, spec.I), dtype=torch.float32)
    u_out = torch.empty((M, spec.I), dtype=torch.float32)
    bounds = np.concatenate([[0], np.cumsum(srt["group_sizes"])])
    for e in range(spec.E):  # ragged_dot: row group e times expert e's matrix
        a, b = int(bounds[e]), int(bounds[e + 1])
        if b > a:
            g_out[a:b] = dot64(lhs_f[a:b], wg[e], torch.float32)
            u_out[a:b] = dot64(lhs_f[a:b], wu[e], torch.float32)
    h = silu_mul(g_out, u_out)  # float32
    y_sorted = torch.zeros((M, spec.D), dtype=torch.float32)
    for e in range(spec.E):
        a, b = int(bounds[e]), int(bounds[e + 1])
        if b > a:
            y_sorted[a:b] = dot64(h[a:b], wd[e], torch.float32)
    assert np.array_equal(sorted_e, np.repeat(np.arange(spec.E), srt["group_sizes"]))
    y_orig = y_sorted[torch.from_numpy(srt["inv"].astype(np.int64))].to(dt)  # y_sorted[inv].astype(x.dtype)
    out = scatter_add_combine(y_orig, rt["w"], T, K)
    return {"h_sorted": h, "y_k": y_orig.reshape(T, K, -1), "out": out}


def fixed_capacity_slots(T: int, K: int, E: int, cf: float, fixed_slots) -> tuple:
    """(c_dyn, c_buf): c_buf as kappa/qwen3/ffn_moe.py:23-31 (8192-token bound, :20);
    c_dyn = max(1, round(f32(cf) * f32(T*K) / f32(E))) in float32 (:136-139)."""
    if fixed_slots is not None:
        c_buf = max(1, int(fixed_slots))
    else:
        c_buf = max(1, int(math.ceil(cf * 8192 * K / E)))
    c_dyn = max(1, int(np.round(np.float32(np.float32(cf) * np.float32(T * K)) / np.float32(E))))
    return c_dyn, c_buf


def fixed_capacity(spec: Spec, inp: dict, rt: dict, cf: float, fixed_slots) -> dict:
    """_moe_fixed_capacity (kappa/qwen3/ffn_moe.py:107-158) on the routing of route()."""
    dt = tdt(spec.act)
    x = as_t(inp["x"], dt)
    T, K = rt["idx"].shape
    E, D = spec.E, spec.D
    M = T * K
    expert_flat = rt["idx"].reshape(M)
    token_flat = np.repeat(np.arange(T, dtype=np.int32), K)
    order = np.lexsort((token_flat, expert_flat))  # sort by expert, then token (:130)
    sorted_e = expert_flat[order]
    sorted_x = x[torch.from_numpy(token_flat[order].astype(np.int64))]
    # _slot_within_expert: 0, 1, ... along each run of equal experts (:59-71)
    slot = np.zeros(M, np.int32)
    for i in range(1, M):
        slot[i] = slot[i - 1] + 1 if sorted_e[i] == sorted_e[i - 1] else 0
    c_dyn, c_buf = fixed_capacity_slots(T, K, E, cf, fixed_slots)
    valid = (slot < c_dyn) & (slot < c_buf)
    safe_s = np.where(valid, slot, 0)
    buf = torch.zeros((E, c_buf, D), dtype=dt)
    for i in range(M):  # .at[sorted_e, safe_s].add(where(valid, sorted_x, 0)) in dt
        buf[sorted_e[i], safe_s[i]] = buf[sorted_e[i], safe_s[i]] + (sorted_x[i] if valid[i] else 0 * sorted_x[i])
    wg, wu, wd = (to_compute_dtype(inp[n], dt) for n in ("gate", "up", "down"))
    g = torch.stack([dot64(buf[e], wg[e], dt) for e in range(E)])  # einsum ecd,edi->eci
    u = torch.stack([dot64(buf[e], wu[e], dt) for e in range(E)])
    h = silu_mul(g, u)
    y_b = torch.stack([dot64(h[e], wd[e], dt) for e in range(E)])  # einsum eci,eid->ecd
    y_pick = torch.where(
        torch.from_numpy(valid)[:, None], y_b[torch.from_numpy(sorted_e.astype(np.int64)), torch.from_numpy(safe_s)],
        torch.zeros((M, D), dtype=dt),
    )  # fmt: skip
    inv = np.zeros(M, np.int32)
    inv[order] = np.arange(M, dtype=np.int32)
    y_assign = y_pick[torch.from_numpy(inv.astype(np.int64))]
    out = scatter_add_combine(y_assign, rt["w"], T, K)
    inv_cap = np.where(valid[inv], inv, -1).astype(np.int32)  # -1 for dropped assignments
    return {"capacity": np.int32(min(c_dyn, c_buf)), "inv_cap": inv_cap, "y_assign": y_assign.reshape(T, K, D),
            "out": out}  # fmt: skip


def f32np(t) -> np.ndarray:
    return t.float().numpy() if isinstance(t, torch.Tensor) else np.asarray(t, np.float32)


def reference_block(spec: Spec, inp: dict) -> dict:
    """moe_swiglu_ffn (kappa/qwen3/ffn_moe.py:226-299) with the spec's array program."""
    rt = route(spec, inp)
    srt = sort_assignments(rt["idx"], spec.E)
    if spec.impl == "gather_einsum":
        ex = gather_einsum(spec, inp, rt)
    elif spec.impl == "ragged":
        ex = ragged(spec, inp, rt, srt)
    else:
        raise ValueError(spec.impl)
    res = {"logits64": rt["logits64"], "idx": rt["idx"], "w": f32np(rt["w"]), "gap": rt["gap"], **srt}
    res.update({k: f32np(v) for k, v in ex.items()})
    return res


def reference_rms_norm(h: np.ndarray, scale: np.ndarray, eps: float, act: str) -> np.ndarray:
    """kappa/qwen3/norms.py:10-16: xf = f32(h); var = mean(xf^2); (xf * rsqrt(var + eps)) * f32(scale),
    cast to the activation dtype (float64 arithmetic)."""
    xf = h.astype(np.float64)
    var = np.mean(xf * xf, axis=-1, keepdims=True)
    normed = xf / np.sqrt(var + eps)
    return f32np(as_t(normed * scale.astype(np.float64), tdt(act)))


def reference_block_residual(spec: Spec, inp: dict, scale: np.ndarray, eps: float) -> dict:
    """h2 = rms_norm(h); out = h + moe_swiglu_ffn(h2) in the activation dtype (kappa/qwen3/block.py:196-207)."""
    h = inp["x"]
    h2 = reference_rms_norm(h, scale, eps, spec.act)
    moe = reference_block(spec, {**inp, "x": h2})
    dt = tdt(spec.act)
    out = as_t(h, dt) + as_t(moe["out"], dt)
    return {"h2": h2, "idx": moe["idx"], "w": moe["w"], "gap": moe["gap"], "moe_out": moe["out"], "out": f32np(out)}


def main() -> None:
    torch.set_num_threads(min(8, os.cpu_count() or 1))
    meta = {}
    for spec in GOLDEN_SPECS:
        inp = make_inputs(spec)
        ref = reference_block(spec, inp)
        np.savez_compressed(os.path.join(HERE, f"{spec.name}.npz"), **ref)
        meta[spec.name] = {"spec": spec.as_dict(), "input_sha256": digest(inp), "min_gap": float(np.min(ref["gap"]))}
        print(f"{spec.name}: {spec.impl} T={spec.T} D={spec.D} E={spec.E} K={spec.K} I={spec.I} "
              f"min_gap={np.min(ref['gap']):.3e}")  # fmt: skip
    for spec, cf, slots in CAPACITY_SPECS:
        inp = make_inputs(spec)
        rt = route(spec, inp)
        ref = fixed_capacity(spec, inp, rt, cf, slots)
        ref = {"idx": rt["idx"], "w": f32np(rt["w"]), **{k: (f32np(v) if isinstance(v, torch.Tensor) else v)
                                                        for k, v in ref.items()}}  # fmt: skip
        np.savez_compressed(os.path.join(HERE, f"{spec.name}.npz"), **ref)
        dropped = int(np.sum(ref["inv_cap"] < 0))
        meta[spec.name] = {
            "spec": spec.as_dict(),
            "input_sha256": digest(inp),
            "min_gap": float(np.min(rt["gap"])),
            "capacity_factor": cf,
            "fixed_slots": slots,
            "capacity": int(ref["capacity"]),
            "dropped": dropped,
        }
        print(f"{spec.name}: capacity {int(ref['capacity'])}, {dropped} of {spec.T * spec.K} assignments dropped")
    for spec, eps in BLOCK_SPECS:
        inp = make_inputs(spec)
        scale = make_norm_scale(spec)
        ref = reference_block_residual(spec, inp, scale, eps)
        np.savez_compressed(os.path.join(HERE, f"{spec.name}.npz"), norm_scale=scale, **ref)
        meta[spec.name] = {
            "spec": spec.as_dict(),
            "input_sha256": digest({**inp, "norm_scale": scale}),
            "min_gap": float(np.min(ref["gap"])),
            "epsilon": eps,
        }
        print(f"{spec.name}: {spec.impl} T={spec.T} D={spec.D} eps={eps} min_gap={np.min(ref['gap']):.3e}")
    with open(os.path.join(HERE, "golden.json"), "w") as f:
        json.dump(meta, f, indent=1, sort_keys=True)


if __name__ == "__main__":
    main()
