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
from inputs import GOLDEN_SPECS, Spec, digest, make_inputs  # noqa: E402


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


def main() -> None:
    meta = {}
    for spec in GOLDEN_SPECS:
        inp = make_inputs(spec)
        ref = reference_block(spec, inp)
        np.savez_compressed(os.path.join(HERE, f"{spec.name}.npz"), **ref)
        meta[spec.name] = {"spec": spec.as_dict(), "input_sha256": digest(inp), "min_gap": float(np.min(ref["gap"]))}
        print(f"{spec.name}: T={spec.T} D={spec.D} E={spec.E} K={spec.K} I={spec.I} min_gap={np.min(ref['gap']):.3e}")
    with open(os.path.join(HERE, "golden.json"), "w") as f:
        json.dump(meta, f, indent=1, sort_keys=True)


if __name__ == "__main__":
    main()
