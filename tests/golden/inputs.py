"""Seeded synthetic inputs for the MoE block (numpy PCG64, one seed per tensor).

Seeds: x=1, router=2, gate=3, up=4, down=5, skew=6 (plus ``base_seed`` offset).
bf16 tensors are produced by round-to-nearest-even from float32 and returned
as float32 arrays holding bf16-representable values.

Weight kinds:
  "f32"      plain float32 weights (the CPU-runnable toy config, no quantisation)
  "bf16"     plain weights rounded to bf16
  "w8c"      int8 values + per-output-channel float32 scales [E, 1, N]
  "w8t"      int8 values + one per-tensor scale (reference default), rounded
             to ``scale_dtype`` ("bf16" as in kappa/qwen3/quant.py:41, or "f32")
"""

from __future__ import annotations

import hashlib
from dataclasses import asdict, dataclass, field

import numpy as np


def bf16_rne(a: np.ndarray) -> np.ndarray:
    """float32 -> bf16 (round to nearest even) -> float32, via integer bit arithmetic."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)
    return r.view(np.float32)


@dataclass(frozen=True)
class Spec:
    name: str
    T: int
    D: int
    E: int
    K: int
    I: int
    act: str = "bf16"  # "bf16" | "f32"
    weights: str = "w8c"  # "f32" | "bf16" | "w8c" | "w8t"
    router: str = "bf16"  # "f32" | "bf16" | "w8t"
    x_std: float = 1.0
    w_std: float = 0.02
    r_std: float = 0.02
    scale_dtype: str = "f32"
    base_seed: int = 0
    x_zero: bool = False  # KAT: x = 0 gives all-equal logits
    tie_router: bool = False  # KAT: duplicated router columns give exact logit ties
    skew_lambda: float = 0.0  # Zipf(1.2) routing bias injected through x[:,0] and router[0,:]
    # the reference array program the case follows: "gather_einsum"
    # (kappa/qwen3/ffn_moe.py:74-104), "ragged" (:174-216, moe_impl ragged_jax /
    # ragged_tokamax above the decode threshold) or "fixed_capacity" (:107-158)
    impl: str = "gather_einsum"
    extra: dict = field(default_factory=dict)

    def as_dict(self) -> dict:
        return asdict(self)


def _normal(seed: int, shape, std: float) -> np.ndarray:
    rng = np.random.default_rng(seed)
    return (rng.standard_normal(shape, dtype=np.float32) * np.float32(std)).astype(np.float32)


def quantize_per_channel_np(w: np.ndarray):
    """Per-output-channel symmetric int8 (kappa/qwen3/quant.py:41-48, reduced over axis -2)."""
    amax = np.max(np.abs(w), axis=-2, keepdims=True).astype(np.float32)
    s = np.maximum(amax / np.float32(127.0), np.finfo(np.float32).tiny).astype(np.float32)
    q = np.clip(np.rint(w / s), -128, 127).astype(np.int8)
    return q, s


def quantize_per_tensor_np(w: np.ndarray):
    amax = np.float32(np.max(np.abs(w)))
    s = np.float32(max(amax / np.float32(127.0), np.finfo(np.float32).tiny))
    q = np.clip(np.rint(w / s), -128, 127).astype(np.int8)
    return q, s


def make_inputs(spec: Spec) -> dict:
    """Return x [T,D], router (array or (q,s)), gate/up [E,D,I], down [E,I,D] (arrays or (q,s))."""
    b = spec.base_seed
    x = _normal(1 + b, (spec.T, spec.D), spec.x_std)
    if spec.x_zero:
        x[:] = 0.0
    r = _normal(2 + b, (spec.D, spec.E), spec.r_std)
    if spec.tie_router:
        # expert e copies expert e % 4's column: logits tie exactly within each class
        for e in range(4, spec.E):
            r[:, e] = r[:, e % 4]
    if spec.skew_lambda:
        rng = np.random.default_rng(6 + b)
        rank = rng.permutation(spec.E) + 1
        bias = spec.skew_lambda * np.log(rank.astype(np.float64) ** -1.2)
        x[:, 0] = 1.0
        r[0, :] = bias.astype(np.float32)
    gate = _normal(3 + b, (spec.E, spec.D, spec.I), spec.w_std)
    up = _normal(4 + b, (spec.E, spec.D, spec.I), spec.w_std)
    down = _normal(5 + b, (spec.E, spec.I, spec.D), spec.w_std)
    if spec.act == "bf16":
        x = bf16_rne(x)
    out = {"x": x}
    if spec.router == "bf16":
        out["router"] = bf16_rne(r)
    elif spec.router == "f32":
        out["router"] = r
    elif spec.router == "w8t":
        q, s = quantize_per_tensor_np(r)
        out["router"] = (q, bf16_rne(np.array([s]))[0] if spec.scale_dtype == "bf16" else s)
    else:
        raise ValueError(spec.router)
    for name, w in (("gate", gate), ("up", up), ("down", down)):
        if spec.weights == "f32":
            out[name] = w
        elif spec.weights == "bf16":
            out[name] = bf16_rne(w)
        elif spec.weights == "w8c":
            out[name] = quantize_per_channel_np(w)
        elif spec.weights == "w8t":
            q, s = quantize_per_tensor_np(w)
            out[name] = (q, bf16_rne(np.array([s]))[0] if spec.scale_dtype == "bf16" else s)
        else:
            raise ValueError(spec.weights)
    return out


def digest(inputs: dict) -> str:
    """SHA-256 over every input array (detects generator drift)."""
    h = hashlib.sha256()
    for k in sorted(inputs):
        v = inputs[k]
        parts = v if isinstance(v, tuple) else (v,)
        for p in parts:
            a = np.ascontiguousarray(np.asarray(p))
            h.update(k.encode())
            h.update(str(a.dtype).encode())
            h.update(str(a.shape).encode())
            h.update(a.tobytes())
    return h.hexdigest()


# Golden cases. Shapes follow the reference's own checks and the benchmark workloads.
# The gather path (moe_take_dequant, kappa/qwen3/quant.py:71-74) multiplies the
# gathered [T, K, D, I] values by the scale as stored, so it takes a per-tensor
# scale or plain weights; per-output-channel scales ([E, 1, N]) run on the
# ragged path, whose to_compute_dtype broadcasts them (:203-205).
#   verify_f32:   scripts/verify_qwen3_moe_impls.py:23 (b=2,t=3,d=16,e=8,k=2,i=32, fp32)
#   toy_f32:      the CPU-runnable toy block (T=64, D=256, E=8, K=2, I=128, fp32, N(0,0.02))
#   w8t_bf16:     the reference's per-tensor Q8 with a bf16 scale (kappa/qwen3/quant.py:41)
#   g30_w8t:      the 30B-A3B per-token shape (D 2048, I 768, top-8) with per-tensor
#                 bf16 scales, 16 experts, 8 tokens: the default decode program
#   w8c_*:        small W8 per-channel bf16 blocks on the ragged path
#   r30_w8c:      the 30B-A3B per-token shape with per-channel f32 scales, ragged
#   r_*:          the ragged program on the other weight kinds (f32, per-tensor, bf16)
#   tie_*:        known-answer tests for the top-k tie rule
GOLDEN_SPECS = [
    Spec("verify_f32", T=6, D=16, E=8, K=2, I=32, act="f32", weights="f32", router="f32", x_std=1.0),
    Spec("toy_f32", T=64, D=256, E=8, K=2, I=128, act="f32", weights="f32", router="f32", x_std=0.02),
    Spec("w8t_bf16", T=16, D=128, E=8, K=2, I=64, weights="w8t", scale_dtype="bf16", base_seed=20),
    Spec("bf16_plain", T=16, D=128, E=8, K=2, I=64, weights="bf16", base_seed=40),
    Spec("g30_w8t", T=8, D=2048, E=16, K=8, I=768, weights="w8t", scale_dtype="bf16", base_seed=200),
    Spec("tie_router", T=8, D=64, E=8, K=3, I=32, weights="w8t", scale_dtype="bf16", tie_router=True, base_seed=60),
    Spec("w8c_bf16", T=32, D=128, E=16, K=4, I=64, impl="ragged"),
    Spec("w8c_bf16_k8", T=24, D=192, E=32, K=8, I=96, base_seed=10, impl="ragged"),
    Spec("w8c_qrouter", T=16, D=128, E=8, K=2, I=64, router="w8t", scale_dtype="bf16", base_seed=30, impl="ragged"),
    Spec("r30_w8c", T=16, D=2048, E=16, K=8, I=768, base_seed=210, impl="ragged"),
    Spec("r_toy_f32", T=64, D=256, E=8, K=2, I=128, act="f32", weights="f32", router="f32", x_std=0.02,
         base_seed=220, impl="ragged"),  # fmt: skip
    Spec("r_w8t_bf16", T=16, D=128, E=8, K=2, I=64, weights="w8t", scale_dtype="bf16", base_seed=230, impl="ragged"),
    Spec("r_bf16_plain", T=16, D=128, E=8, K=2, I=64, weights="bf16", base_seed=240, impl="ragged"),
    Spec("tie_zero_x", T=4, D=64, E=8, K=3, I=32, x_zero=True, base_seed=50, impl="ragged"),
]

# fixed_capacity cases (kappa/qwen3/ffn_moe.py:107-158): (spec, capacity_factor, moe_fixed_capacity_slots)
#   cap_w8c_bf16:   c_dyn = round(0.5 * 128 / 16) = 4 slots for ~8 assignments per expert
#   cap_f32_slots:  c_dyn = round(1.25 * 48 / 8) = 8, capped by 3 static slots (c_buf)
#   cap_skew_bf16:  Zipf-skewed routing, c_dyn = 6: the hot experts overflow
#   cap30_w8c:      the 30B-A3B per-token shape, c_dyn = round(0.5 * 128 / 16) = 4
CAPACITY_SPECS = [
    (Spec("cap_w8c_bf16", T=32, D=128, E=16, K=4, I=64, base_seed=70, impl="fixed_capacity"), 0.5, None),
    (Spec("cap_f32_slots", T=24, D=64, E=8, K=2, I=32, act="f32", weights="f32", router="f32", base_seed=80,
          impl="fixed_capacity"), 1.25, 3),  # fmt: skip
    (Spec("cap_skew_bf16", T=48, D=128, E=16, K=2, I=64, skew_lambda=1.0, base_seed=90, impl="fixed_capacity"), 1.0,
     None),  # fmt: skip
    (Spec("cap30_w8c", T=16, D=2048, E=16, K=8, I=768, base_seed=250, impl="fixed_capacity"), 0.5, None),
]


# The MoE block with the steps either side of it (kappa/qwen3/block.py:196-207):
# (spec, epsilon). The spec's x is the residual stream h; the RMSNorm scale
# (pre_ffn_norm, seed 7) is N(1, 0.1), rounded to bf16 for bf16 activations.
#   blk_w8c_bf16:  the 30B numerics at toy size (ragged)
#   blk_d192_k8:   hidden 192 (three slices: a zero-padded sum tree), top-8 (ragged)
#   blk_w8t_bf16:  per-tensor scales on the gather path
#   blk_toy_f32:   the fp32 toy block (gather)
BLOCK_SPECS = [
    (Spec("blk_w8c_bf16", T=32, D=128, E=16, K=4, I=64, base_seed=100, impl="ragged"), 1e-6),
    (Spec("blk_d192_k8", T=24, D=192, E=32, K=8, I=96, base_seed=110, impl="ragged"), 1e-5),
    (Spec("blk_w8t_bf16", T=16, D=128, E=8, K=2, I=64, weights="w8t", scale_dtype="bf16", base_seed=130), 1e-6),
    (Spec("blk_toy_f32", T=16, D=256, E=8, K=2, I=128, act="f32", weights="f32", router="f32", base_seed=120), 1e-6),
]


def make_norm_scale(spec: Spec) -> np.ndarray:
    """pre_ffn_norm [D]: N(1, 0.1) from seed 7 (+ base_seed), bf16 for bf16 activations."""
    s = (_normal(7 + spec.base_seed, (spec.D,), 0.1) + np.float32(1.0)).astype(np.float32)
    return bf16_rne(s) if spec.act == "bf16" else s
