"""The MoE half of a Qwen3 MoE layer on the GPU: rms_norm in, residual add out
(kappa/qwen3/block.py:196-207, kappa/qwen3/norms.py:10-16).

Bar: rms_norm bit-exact against the oracle (the kernel and the oracle sum the
squares in the same canonical order); top-k indices bit-exact; block outputs
within max-abs 2e-2 / mean-rel 1e-3 in bf16 and 1e-5 of the output scale in
f32 against the oracle; the fused call bit-identical to the composition of
the separate GPU calls (rms_norm, moe_swiglu_ffn, then the add).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from inputs import BLOCK_SPECS, make_inputs, make_norm_scale
from moe_cases import bf16_np, forward_args, layer_cfg, make_layer, make_x, mean_rel

pytestmark = pytest.mark.gpu

BF16_MAX_ABS = 2e-2
BF16_MEAN_REL = 1e-3
F32_REL = 1e-5


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    return torch.device("cuda:0")


def check_out(out: np.ndarray, ref: np.ndarray, bf16: bool, what: str = "out"):
    if bf16:
        d = np.abs(out - ref)
        assert d.max() <= BF16_MAX_ABS, f"{what}: max-abs {d.max():.3e}"
        assert mean_rel(out, ref) <= BF16_MEAN_REL, f"{what}: mean-rel {mean_rel(out, ref):.3e}"
    else:
        scale = max(float(np.abs(ref).max()), 1e-30)
        assert np.abs(out - ref).max() <= F32_REL * scale, f"{what}: {np.abs(out - ref).max() / scale:.3e}"


@pytest.mark.parametrize("act", ["bf16", "f32"])
@pytest.mark.parametrize("scale_dtype", ["bf16", "f32"])
@pytest.mark.parametrize("D", [16, 100, 192, 2048, 2560, 4096])
def test_rms_norm_bit_exact(dev, act, scale_dtype, D):
    from kappa_amd.qwen3 import rms_norm

    rng = np.random.default_rng(D)
    for T, eps in ((1, 1e-6), (7, 1e-5), (300, 1e-6)):
        h = (rng.standard_normal((T, D)) * rng.uniform(0.01, 30.0, (T, 1))).astype(np.float32)
        h[T // 2] = 0.0  # a zero row: r = 1 / sqrt(eps)
        s = (1.0 + 0.1 * rng.standard_normal(D)).astype(np.float32)
        if act == "bf16":
            h = oracle.bf16_round(h)
        if scale_dtype == "bf16":
            s = oracle.bf16_round(s)
        td = torch.bfloat16 if act == "bf16" else torch.float32
        sd = torch.bfloat16 if scale_dtype == "bf16" else torch.float32
        got = rms_norm(torch.from_numpy(h).to(dev).to(td), torch.from_numpy(s).to(dev).to(sd), epsilon=eps)
        want = oracle.rms_norm(h, s, eps, act == "bf16")
        np.testing.assert_array_equal(got.float().cpu().numpy(), want, err_msg=f"T={T} eps={eps}")


@pytest.mark.parametrize("case", BLOCK_SPECS, ids=[c[0].name for c in BLOCK_SPECS])
def test_block_golden(dev, case):
    from kappa_amd.qwen3.ffn_moe import _moe_forward
    from test_gpu_parity import spec_to_dev

    spec, eps = case
    inp = make_inputs(spec)
    scale = make_norm_scale(spec)
    bf16 = spec.act == "bf16"
    h, r, (g, u, d) = spec_to_dev(spec, inp, dev)
    sc = torch.from_numpy(scale).to(dev).to(torch.bfloat16 if bf16 else torch.float32)
    out, idx, w = _moe_forward(
        h.reshape(1, spec.T, spec.D), r, g, u, d, num_experts=spec.E, num_experts_per_tok=spec.K,
        packed=None, return_routing=True, norm=(sc, eps), **forward_args(spec.impl),
    )  # fmt: skip
    ref = oracle.forward_block(inp["x"], scale, inp["router"], inp["gate"], inp["up"], inp["down"], k=spec.K,
                               act_bf16=bf16, impl=spec.impl, eps=eps)  # fmt: skip
    np.testing.assert_array_equal(idx.cpu().numpy(), ref["idx"])
    check_out(out.reshape(spec.T, spec.D).float().cpu().numpy(), ref["out"], bf16)
    gold = np.load(f"tests/golden/{spec.name}.npz")
    np.testing.assert_array_equal(idx.cpu().numpy(), gold["idx"])
    check_out(out.reshape(spec.T, spec.D).float().cpu().numpy(), gold["out"], bf16, "vs golden")


@pytest.fixture(scope="module")
def l30(dev):
    return make_layer("30b", seed=0)


def _norm_scale(D, seed, dev):
    rng = np.random.default_rng(seed)
    return torch.from_numpy((1.0 + 0.1 * rng.standard_normal(D)).astype(np.float32)).to(dev).to(torch.bfloat16)


@pytest.mark.parametrize("T", [1, 2, 8, 17, 64, 65, 128, 129, 240, 241, 4096])
def test_30b_fused_block_equals_separate_calls(dev, l30, T):
    """moe_block_ffn == h + moe_swiglu_ffn(rms_norm(h)), bit for bit; the norm is
    checked against the oracle on every row, the MoE half against the oracle
    by the block tests of test_gpu_parity."""
    from kappa_amd.qwen3 import moe_block_ffn, moe_swiglu_ffn, rms_norm

    cfg = layer_cfg(l30, "ragged")
    h = make_x(T, l30.D, seed=900 + T).reshape(1, T, l30.D) * 4.0
    sc = _norm_scale(l30.D, T, dev)
    h2 = rms_norm(h, sc)
    want_h2 = oracle.rms_norm(bf16_np(h.reshape(T, l30.D)), sc.float().cpu().numpy(), 1e-6, True)
    np.testing.assert_array_equal(bf16_np(h2.reshape(T, l30.D)), want_h2)
    composed = h + moe_swiglu_ffn(h2, l30.router, l30.gate, l30.up, l30.down, cfg=cfg)
    for _ in range(2):
        fused = moe_block_ffn(h, sc, l30.router, l30.gate, l30.up, l30.down, cfg=cfg)
        assert fused.dtype == h.dtype and fused.shape == h.shape
        assert torch.equal(fused, composed)


@pytest.mark.parametrize("T", [8, 100, 241])
def test_other_shape_fused_block_equals_separate_calls(dev, T):
    """The block call on a layer outside the Qwen3 presets (D = 2560: 40 router
    slices, the split router normalising its rows at T <= 240, the norm kernel
    above), bit for bit against its composition."""
    from kappa_amd.qwen3 import moe_block_ffn, moe_swiglu_ffn, rms_norm

    layer = make_layer("odd", seed=5)
    cfg = layer_cfg(layer, "ragged")
    h = make_x(T, layer.D, seed=950 + T).reshape(1, T, layer.D) * 4.0
    sc = _norm_scale(layer.D, T, dev)
    h2 = rms_norm(h, sc)
    want_h2 = oracle.rms_norm(bf16_np(h.reshape(T, layer.D)), sc.float().cpu().numpy(), 1e-6, True)
    np.testing.assert_array_equal(bf16_np(h2.reshape(T, layer.D)), want_h2)
    composed = h + moe_swiglu_ffn(h2, layer.router, layer.gate, layer.up, layer.down, cfg=cfg)
    fused = moe_block_ffn(h, sc, layer.router, layer.gate, layer.up, layer.down, cfg=cfg)
    assert torch.equal(fused, composed)


def test_30b_fused_block_fixed_capacity(dev, l30):
    from kappa_amd.qwen3 import moe_block_ffn, moe_swiglu_ffn, rms_norm

    cfg = layer_cfg(l30, "fixed_capacity", moe_capacity_factor=0.5)
    for T in (3, 64, 100, 1024):
        h = make_x(T, l30.D, seed=950 + T).reshape(1, T, l30.D)
        sc = _norm_scale(l30.D, 7 + T, dev)
        composed = h + moe_swiglu_ffn(rms_norm(h, sc), l30.router, l30.gate, l30.up, l30.down, cfg=cfg)
        assert torch.equal(moe_block_ffn(h, sc, l30.router, l30.gate, l30.up, l30.down, cfg=cfg), composed)


def test_zero_norm_scale_returns_the_residual(dev, l30):
    # rms_norm(h) * 0 = 0 and the block maps 0 to exactly 0: out == h
    from kappa_amd.qwen3 import moe_block_ffn

    cfg = layer_cfg(l30, "ragged")
    for T in (3, 300):
        h = make_x(T, l30.D, seed=990 + T).reshape(1, T, l30.D)
        z = torch.zeros(l30.D, dtype=torch.bfloat16, device=dev)
        assert torch.equal(moe_block_ffn(h, z, l30.router, l30.gate, l30.up, l30.down, cfg=cfg), h)
