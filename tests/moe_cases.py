"""Layer builders and oracle helpers shared by the GPU tests and the benchmark.

Big layers (the 30B-A3B and 235B-A22B shapes) are generated on the device:
weights ~ N(0, 0.02) from a seeded torch generator, quantised per output
channel by the library's quantiser (or per tensor with a bf16 scale, the
reference's own quantize_weight, kappa/qwen3/quant.py:41-48), activations bf16
~ N(0, 1), router bf16 ~ N(0, 0.02). Host copies (numpy) feed the oracle.

Each layer call names the reference array program it is checked against:
per-channel layers run the ragged program (moe_impl ragged_jax with a decode
threshold of 0 at every token count, as scripts/verify_qwen3_moe_impls.py:51
configures it, or the default threshold above 64 tokens) or fixed_capacity;
per-tensor layers also run the gather program (the default impl).
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

SHAPES = {
    "30b": dict(D=2048, E=128, K=8, I=768),
    "235b": dict(D=4096, E=128, K=8, I=1536),
    # shapes outside the Qwen3 presets (GPU tests only): load batches that do
    # not divide a wave's chunks (D / 64 = 40, I / 64 = 16), 64 experts, top-6;
    # and 256 experts
    "odd": dict(D=2560, E=64, K=6, I=1024),
    "e256": dict(D=2048, E=256, K=8, I=768),
    # I not a multiple of 128 (fifteen 64-wide chunks): the grouped GEMM for
    # such shapes (k_prefill) and decode GEMVs whose waves take unequal chunks
    "i960": dict(D=2048, E=32, K=4, I=960),
}


@dataclass
class Layer:
    D: int
    E: int
    K: int
    I: int
    router: torch.Tensor  # [D, E] bf16
    gate: object  # Q8Weight
    up: object
    down: object

    def host(self) -> dict:
        """numpy copies for the oracle: router float32, experts (q int8, s float32 [E,1,N])."""
        if not hasattr(self, "_host"):
            self._host = {
                "router": self.router.float().cpu().numpy(),
                **{
                    n: (w.values.cpu().numpy(), w.scale.float().cpu().numpy())
                    for n, w in (("gate", self.gate), ("up", self.up), ("down", self.down))
                },
            }
        return self._host


def make_layer(shape: str, seed: int = 0, device: str = "cuda", per_tensor: bool = False) -> Layer:
    from kappa_amd.qwen3 import quantize_weight, quantize_weight_per_channel

    s = SHAPES[shape]
    D, E, K, I = s["D"], s["E"], s["K"], s["I"]
    g = torch.Generator(device=device)
    g.manual_seed(1000 + seed)
    router = (torch.randn(D, E, generator=g, device=device) * 0.02).to(torch.bfloat16)
    ws = []
    for shp in ((E, D, I), (E, D, I), (E, I, D)):
        w = torch.randn(*shp, generator=g, device=device) * 0.02
        ws.append(quantize_weight(w) if per_tensor else quantize_weight_per_channel(w))
        del w
    return Layer(D, E, K, I, router, *ws)


def layer_cfg(layer: Layer, impl: str, **kw):
    """A config that runs ``impl``'s array program at every token count: "ragged" is
    ragged_jax with threshold 0; "gather_einsum" and "fixed_capacity" as named."""
    from kappa_amd.qwen3 import moe_layer_config

    if impl == "ragged":
        kw = {"moe_impl": "ragged_jax", "moe_ragged_decode_token_threshold": 0, **kw}
    else:
        kw = {"moe_impl": impl, **kw}
    return moe_layer_config(hidden=layer.D, experts=layer.E, top_k=layer.K, intermediate=layer.I, **kw)


def forward_args(impl: str) -> dict:
    """_moe_forward keywords that run ``impl``'s program at every token count."""
    if impl == "ragged":
        return {"impl": "ragged_jax", "decode_threshold": 0}
    return {"impl": impl, "decode_threshold": 64}


def make_x(T: int, D: int, seed: int = 0, device: str = "cuda", skew_router: torch.Tensor | None = None):
    g = torch.Generator(device=device)
    g.manual_seed(2000 + seed)
    x = torch.randn(T, D, generator=g, device=device).to(torch.bfloat16)
    return x


def skew_router(router: torch.Tensor, lam: float, seed: int = 6) -> torch.Tensor:
    """Zipf(1.2) routing bias through the inputs: router[0, e] = lam * log(rank_e^-1.2); pair with x[:, 0] = 1."""
    E = router.shape[1]
    rng = np.random.default_rng(seed)
    rank = rng.permutation(E) + 1
    bias = lam * np.log(rank.astype(np.float64) ** -1.2)
    r = router.clone()
    r[0, :] = torch.from_numpy(bias.astype(np.float32)).to(r.device, r.dtype)
    return r


def oracle_rows(oracle, x_np, tokens, experts, host, act_bf16=True, *, impl):
    """Oracle h, y of ``impl``'s program for the assignment rows (tokens[i], experts[i]),
    in input order."""
    tokens = np.asarray(tokens, np.int32)
    experts = np.asarray(experts, np.int32)
    E = host["gate"][0].shape[0]
    order = np.argsort(experts, kind="stable")
    st = tokens[order]
    counts = np.bincount(experts, minlength=E)
    off = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    h, y = oracle.expert_ffn(x_np, off, st, host["gate"], host["up"], host["down"], act_bf16, impl=impl)
    inv = np.empty_like(order)
    inv[order] = np.arange(len(order))
    return h[inv], y[inv]


def mean_rel(a: np.ndarray, b: np.ndarray) -> float:
    return float(np.mean(np.abs(a - b)) / max(float(np.mean(np.abs(b))), 1e-30))


def bf16_np(t: torch.Tensor) -> np.ndarray:
    return t.float().cpu().numpy()
