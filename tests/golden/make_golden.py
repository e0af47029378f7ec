#!/usr/bin/env python3
"""Write the golden vectors in this directory.

The expected values come from a direct numpy/torch-CPU transliteration of the
reference layer's array program -- not from the C oracle -- so the oracle is
checked against an independent restatement:

  _route            kappa/qwen3/ffn_moe.py:38-56  (einsum -> lax.top_k -> softmax)
  to_compute_dtype  kappa/qwen3/quant.py:34-38    (values.astype(dt) * scale.astype(dt))
  moe_take_dequant  kappa/qwen3/quant.py:60-76
  _moe_gather_einsum kappa/qwen3/ffn_moe.py:74-104 (the default path)
  _moe_ragged order  kappa/qwen3/ffn_moe.py:189-200, 212 (argsort stable, bincount, inv)
  _moe_fixed_capacity kappa/qwen3/ffn_moe.py:107-158 with _slot_within_expert :59-71
                     and _fixed_capacity_buffer_slots :23-31 (token dropping)
  rms_norm           kappa/qwen3/norms.py:10-16
  block MoE half     kappa/qwen3/block.py:196-207 (h2 = rms_norm(h); h + moe(h2))

Accumulations run in float64 and are rounded to the activation dtype at the
points where the reference's arrays carry ``x.dtype``; bf16 rounding uses
torch's CPU bfloat16 conversion. ``jax`` is not installed here, so the
reference itself cannot be executed; this restatement stands in for it.

Usage: python tests/golden/make_golden.py   (rewrites *.npz and golden.json)
"""

from __future__ import annotations

import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
from inputs import BLOCK_SPECS, CAPACITY_SPECS, GOLDEN_SPECS, Spec, digest, make_inputs, make_norm_scale  # noqa: E402


def as_act(a, act: str) -> np.ndarray:
    """``.astype(x.dtype)``: float32 rounding, then bf16 rounding through torch when act is bf16."""
    a32 = np.asarray(a, dtype=np.float32)
    if act == "f32":
        return a32
    return torch.from_numpy(np.ascontiguousarray(a32)).to(torch.bfloat16).to(torch.float32).numpy()


def to_compute_dtype(w, act: str) -> np.ndarray:
    """kappa/qwen3/quant.py:34-38 with dt = x.dtype."""
    if isinstance(w, tuple):
        q, s = w
        qv = as_act(q.astype(np.float32), act)
        sv = as_act(np.asarray(s, np.float32), act)
        if act == "f32":
            return (qv * sv).astype(np.float32)
        prod = torch.from_numpy(np.ascontiguousarray(qv)).to(torch.bfloat16) * torch.from_numpy(
            np.ascontiguousarray(np.broadcast_to(sv, qv.shape))
        ).to(torch.bfloat16)
        return prod.to(torch.float32).numpy()
    return as_act(w, act)


def router_f32(r) -> np.ndarray:
    """to_compute_dtype(router_w, float32) (kappa/qwen3/ffn_moe.py:46)."""
    if isinstance(r, tuple):
        q, s = r
        return (q.astype(np.float32) * np.asarray(s, np.float32)).astype(np.float32)
    return np.asarray(r, np.float32)


def silu64(g: np.ndarray) -> np.ndarray:
    return g / (1.0 + np.exp(-g))


def reference_block(spec: Spec, inp: dict) -> dict:
    act = spec.act
    x = inp["x"]
    T, D = x.shape
    E, K = spec.E, spec.K
    # _route
    rw = router_f32(inp["router"])
    logits = x.astype(np.float64) @ rw.astype(np.float64)
    order_e = np.lexsort((np.broadcast_to(np.arange(E), (T, E)), -logits), axis=-1)
    top_idx = order_e[:, :K].astype(np.int32)
    top_l = np.take_along_axis(logits, top_idx.astype(np.int64), axis=-1)
    ex = np.exp(top_l - top_l[:, :1])
    w = as_act(ex / ex.sum(axis=-1, keepdims=True), act)
    # K-th vs (K+1)-th gap (near ties can flip selection under a different fp32 order)
    srt = np.take_along_axis(logits, order_e.astype(np.int64), axis=-1)
    gap = (srt[:, K - 1] - srt[:, K]) if K < E else np.full(T, np.inf)
    # dispatch as in _moe_ragged
    expert_flat = top_idx.reshape(-1)
    order = np.argsort(expert_flat, kind="stable").astype(np.int32)
    group_sizes = np.bincount(expert_flat, minlength=E).astype(np.int32)
    inv = np.zeros(T * K, np.int32)
    inv[order] = np.arange(T * K, dtype=np.int32)
    # _moe_gather_einsum
    wg = to_compute_dtype(inp["gate"], act)
    wu = to_compute_dtype(inp["up"], act)
    wd = to_compute_dtype(inp["down"], act)
    w0 = wg[top_idx].astype(np.float64)  # [T,K,D,I]
    w1 = wu[top_idx].astype(np.float64)
    w2 = wd[top_idx].astype(np.float64)  # [T,K,I,D]
    xd = x.astype(np.float64)
    g = as_act(np.einsum("bd,bkdi->bki", xd, w0), act)
    u = as_act(np.einsum("bd,bkdi->bki", xd, w1), act)
    h = as_act(silu64(g.astype(np.float64)) * u.astype(np.float64), act)
    y_k = as_act(np.einsum("bki,bkid->bkd", h.astype(np.float64), w2), act)
    out = as_act(np.sum(y_k.astype(np.float64) * w.astype(np.float64)[..., None], axis=1), act)
    return {
        "logits64": logits,
        "idx": top_idx,
        "w": w,
        "gap": gap,
        "order": order,
        "group_sizes": group_sizes,
        "inv": inv,
        "h": h.astype(np.float32),
        "y_k": y_k.astype(np.float32),
        "out": out.astype(np.float32),
    }


def fixed_capacity_slots(T: int, K: int, E: int, cf: float, fixed_slots) -> tuple:
    """(c_dyn, c_buf): c_buf as kappa/qwen3/ffn_moe.py:23-31 (8192-token bound, :20);
    c_dyn = max(1, round(f32(cf) * f32(T*K) / f32(E))) in float32 (:136-139)."""
    import math

    if fixed_slots is not None:
        c_buf = max(1, int(fixed_slots))
    else:
        c_buf = max(1, int(math.ceil(cf * 8192 * K / E)))
    c_dyn = max(1, int(np.round(np.float32(np.float32(cf) * np.float32(T * K)) / np.float32(E))))
    return c_dyn, c_buf


def reference_fixed_capacity(spec: Spec, inp: dict, blk: dict, cf: float, fixed_slots) -> dict:
    """_moe_fixed_capacity (kappa/qwen3/ffn_moe.py:107-158) on the routing of reference_block."""
    act = spec.act
    x = inp["x"]
    T, D = x.shape
    E, K = spec.E, spec.K
    M = T * K
    idx, w = blk["idx"], blk["w"]
    expert_flat = idx.reshape(M)
    token_flat = np.repeat(np.arange(T, dtype=np.int32), K)
    w_flat = w.reshape(M)
    order = np.lexsort((token_flat, expert_flat))  # sort by expert, then token (:130)
    sorted_e = expert_flat[order]
    sorted_x = x[token_flat[order]]
    # _slot_within_expert: 0, 1, ... along each run of equal experts (:59-71)
    slot = np.zeros(M, np.int32)
    for i in range(1, M):
        slot[i] = slot[i - 1] + 1 if sorted_e[i] == sorted_e[i - 1] else 0
    c_dyn, c_buf = fixed_capacity_slots(T, K, E, cf, fixed_slots)
    valid = (slot < c_dyn) & (slot < c_buf)
    buf = np.zeros((E, c_buf, D), np.float64)
    safe_s = np.where(valid, slot, 0)
    for i in range(M):
        if valid[i]:
            buf[sorted_e[i], safe_s[i]] += sorted_x[i]
    wg = to_compute_dtype(inp["gate"], act).astype(np.float64)
    wu = to_compute_dtype(inp["up"], act).astype(np.float64)
    wd = to_compute_dtype(inp["down"], act).astype(np.float64)
    g = as_act(np.einsum("ecd,edi->eci", buf, wg), act)
    u = as_act(np.einsum("ecd,edi->eci", buf, wu), act)
    h = as_act(silu64(g.astype(np.float64)) * u.astype(np.float64), act)
    y_b = as_act(np.einsum("eci,eid->ecd", h.astype(np.float64), wd), act)
    y_pick = np.where(valid[:, None], y_b[sorted_e, safe_s], 0.0)
    inv = np.zeros(M, np.int32)
    inv[order] = np.arange(M, dtype=np.int32)
    y_assign = y_pick[inv]  # gather order (t, j)
    out = as_act(np.sum((y_assign * w_flat[:, None].astype(np.float64)).reshape(T, K, D), axis=1), act)
    # inv with -1 for dropped assignments (position in the stable order otherwise)
    inv_cap = np.where(valid[inv], inv, -1).astype(np.int32)
    return {
        "idx": idx,
        "w": w,
        "capacity": np.int32(min(c_dyn, c_buf)),
        "inv_cap": inv_cap,
        "y_assign": y_assign.astype(np.float32).reshape(T, K, D),
        "out": out.astype(np.float32),
    }


def reference_rms_norm(h: np.ndarray, scale: np.ndarray, eps: float, act: str) -> np.ndarray:
    """kappa/qwen3/norms.py:10-16: xf = f32(h); var = mean(xf^2); (xf * rsqrt(var + eps)) * f32(scale),
    cast to the activation dtype (float64 arithmetic)."""
    xf = h.astype(np.float64)
    var = np.mean(xf * xf, axis=-1, keepdims=True)
    normed = xf / np.sqrt(var + eps)
    return as_act(normed * scale.astype(np.float64), act)


def reference_block_residual(spec: Spec, inp: dict, scale: np.ndarray, eps: float) -> dict:
    """h2 = rms_norm(h); out = h + moe_swiglu_ffn(h2) in the activation dtype (kappa/qwen3/block.py:196-207)."""
    h = inp["x"]
    h2 = reference_rms_norm(h, scale, eps, spec.act)
    moe = reference_block(spec, {**inp, "x": h2})
    out = as_act(h.astype(np.float64) + moe["out"].astype(np.float64), spec.act)
    return {"h2": h2.astype(np.float32), "idx": moe["idx"], "w": moe["w"], "gap": moe["gap"],
            "moe_out": moe["out"], "out": out.astype(np.float32)}  # fmt: skip


def main() -> None:
    meta = {}
    for spec in GOLDEN_SPECS:
        inp = make_inputs(spec)
        ref = reference_block(spec, inp)
        np.savez_compressed(os.path.join(HERE, f"{spec.name}.npz"), **ref)
        meta[spec.name] = {"spec": spec.as_dict(), "input_sha256": digest(inp), "min_gap": float(np.min(ref["gap"]))}
        print(f"{spec.name}: T={spec.T} D={spec.D} E={spec.E} K={spec.K} I={spec.I} min_gap={np.min(ref['gap']):.3e}")
    for spec, cf, slots in CAPACITY_SPECS:
        inp = make_inputs(spec)
        blk = reference_block(spec, inp)
        ref = reference_fixed_capacity(spec, inp, blk, cf, slots)
        np.savez_compressed(os.path.join(HERE, f"{spec.name}.npz"), **ref)
        dropped = int(np.sum(ref["inv_cap"] < 0))
        meta[spec.name] = {
            "spec": spec.as_dict(),
            "input_sha256": digest(inp),
            "min_gap": float(np.min(blk["gap"])),
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
        print(f"{spec.name}: T={spec.T} D={spec.D} eps={eps} min_gap={np.min(ref['gap']):.3e}")
    with open(os.path.join(HERE, "golden.json"), "w") as f:
        json.dump(meta, f, indent=1, sort_keys=True)


if __name__ == "__main__":
    main()
