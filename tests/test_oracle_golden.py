"""The oracle against the golden vectors (CPU).

The golden vectors in tests/golden/ were written by make_golden.py, a literal
numpy / torch-CPU transliteration of the reference's array programs (one per
case: _moe_gather_einsum kappa/qwen3/ffn_moe.py:74-104, _moe_ragged :174-216,
_moe_fixed_capacity :107-158; kappa/qwen3/quant.py:34-38, 60-76) with float64
accumulation. The C oracle accumulates in float32 in its own order, so floating
results agree to rounding, and integer results exactly. The last tests plant
the rounding schemes of the other programs (and of an earlier contract of this
build) in the oracle's place and check that the goldens reject them.
"""

import json
import os

import numpy as np
import pytest

import oracle
from inputs import BLOCK_SPECS, GOLDEN_SPECS, digest, make_inputs, make_norm_scale

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
META = json.load(open(os.path.join(HERE, "golden.json")))


@pytest.mark.parametrize("spec", GOLDEN_SPECS, ids=[s.name for s in GOLDEN_SPECS])
def test_oracle_matches_golden(spec):
    inp = make_inputs(spec)
    assert digest(inp) == META[spec.name]["input_sha256"], "input generator drifted from the golden vectors"
    g = np.load(os.path.join(HERE, f"{spec.name}.npz"))
    bf16 = spec.act == "bf16"
    r = oracle.forward(inp["x"], inp["router"], inp["gate"], inp["up"], inp["down"], k=spec.K, act_bf16=bf16,
                       impl=spec.impl)  # fmt: skip
    # logits: fp32 canonical order vs fp64 within the fp32 summation error bound
    rw = inp["router"]
    rf = (rw[0].astype(np.float64) * np.float64(rw[1])) if isinstance(rw, tuple) else rw.astype(np.float64)
    bound = 2.0 * spec.D * np.finfo(np.float32).eps * (np.abs(inp["x"]).astype(np.float64) @ np.abs(rf)) + 1e-30
    assert np.all(np.abs(r["logits"] - g["logits64"]) <= bound)
    # top-k indices and dispatch are integer results: exact
    np.testing.assert_array_equal(r["idx"], g["idx"])
    np.testing.assert_array_equal(r["order"], g["order"])
    np.testing.assert_array_equal(r["group_sizes"], g["group_sizes"])
    np.testing.assert_array_equal(r["inv"], g["inv"])
    np.testing.assert_array_equal(r["sorted_token"], g["order"] // spec.K)
    # routing weights: within one ulp of the activation dtype
    ulp = 2.0**-8 if bf16 else 2.0**-23
    assert np.all(np.abs(r["w"] - g["w"]) <= ulp * np.abs(g["w"]) + 1e-30)
    # expert outputs in gather order [T, K, D]
    y_g = r["y_sorted"][r["inv"]].reshape(spec.T, spec.K, -1)
    out = r["out"]
    if spec.impl == "ragged":
        # h is f32 on the ragged path: f32 sums in another order than float64
        hs = g["h_sorted"]
        assert np.max(np.abs(r["h_sorted"] - hs)) <= 1e-5 * max(float(np.abs(hs).max()), 1e-30)
        pairs = ((y_g, g["y_k"]), (out, g["out"]))
    else:
        h_g = r["h_sorted"][r["inv"]].reshape(spec.T, spec.K, -1)
        pairs = ((h_g, g["h"]), (y_g, g["y_k"]), (out, g["out"]))
    if bf16:
        # identical except rare one-ulp flips from fp32 vs fp64 accumulation (a flip of
        # g, u or h moves y by a few ulps of the row's scale where y cancels to ~0)
        for a, b in pairs:
            diff = np.abs(a - b)
            assert np.mean(diff > 0) < 2e-2
            assert np.all(diff <= 2.0**-7 * np.abs(b) + 2.0**-9 * np.abs(b).max())
            assert np.mean(diff) <= 1e-4 * np.mean(np.abs(b))
    else:
        for a, b in pairs:
            assert np.max(np.abs(a - b)) <= 1e-5 * max(float(np.abs(b).max()), 1e-30)


def test_golden_cases_have_no_near_ties_except_the_tie_kats():
    for spec in GOLDEN_SPECS:
        gap = META[spec.name]["min_gap"]
        if spec.name.startswith("tie_"):
            assert gap == 0.0
        else:
            # far above the fp32 error of the logits (~1e-9 at these magnitudes)
            assert gap > 1e-5, spec.name


def test_tie_kats():
    # x = 0: every logit is +0.0, so top-k is [0..K-1] and each weight is round(1/K)
    spec = next(s for s in GOLDEN_SPECS if s.name == "tie_zero_x")
    inp = make_inputs(spec)
    r = oracle.forward(inp["x"], inp["router"], inp["gate"], inp["up"], inp["down"], k=spec.K, act_bf16=True,
                       impl=spec.impl)  # fmt: skip
    np.testing.assert_array_equal(r["idx"], np.tile(np.arange(spec.K, dtype=np.int32), (spec.T, 1)))
    np.testing.assert_array_equal(r["w"], oracle.bf16_round(np.full((spec.T, spec.K), 1.0 / spec.K, np.float32)))
    assert np.all(r["out"] == 0.0)
    # duplicated router columns: experts e and e+4 tie exactly; the lower index comes first
    spec = next(s for s in GOLDEN_SPECS if s.name == "tie_router")
    inp = make_inputs(spec)
    r = oracle.forward(inp["x"], inp["router"], inp["gate"], inp["up"], inp["down"], k=spec.K, act_bf16=True,
                       impl=spec.impl)  # fmt: skip
    lg = r["logits"]
    np.testing.assert_array_equal(lg[:, :4], lg[:, 4:])
    for t in range(spec.T):
        best = int(np.argmax(lg[t, :4]))
        assert r["idx"][t, 0] == best and r["idx"][t, 1] == best + 4
        assert r["w"][t, 0] == r["w"][t, 1]


from inputs import CAPACITY_SPECS  # noqa: E402


@pytest.mark.parametrize("case", CAPACITY_SPECS, ids=[c[0].name for c in CAPACITY_SPECS])
def test_oracle_fixed_capacity_matches_golden(case):
    """fixed_capacity (kappa/qwen3/ffn_moe.py:107-158): the slot limit, which
    assignments are dropped (exact), and the outputs of the kept ones."""
    spec, cf, slots = case
    inp = make_inputs(spec)
    assert digest(inp) == META[spec.name]["input_sha256"], "input generator drifted from the golden vectors"
    g = np.load(os.path.join(HERE, f"{spec.name}.npz"))
    cap = oracle.capacity_slots(spec.T, spec.K, spec.E, cf, slots)
    assert cap == int(g["capacity"])
    bf16 = spec.act == "bf16"
    r = oracle.forward(
        inp["x"], inp["router"], inp["gate"], inp["up"], inp["down"], k=spec.K, act_bf16=bf16, impl="fixed_capacity",
        capacity=cap,
    )  # fmt: skip
    np.testing.assert_array_equal(r["idx"], g["idx"])
    np.testing.assert_array_equal(r["inv"], g["inv_cap"])
    assert np.any(r["inv"] < 0), "the case must drop something"
    kept = r["inv"].reshape(spec.T, spec.K) >= 0
    y_g = np.where(kept[..., None], r["y_sorted"][np.maximum(r["inv"], 0)].reshape(spec.T, spec.K, -1), 0.0)
    if bf16:
        for a, b in ((y_g, g["y_assign"]), (r["out"], g["out"])):
            diff = np.abs(a - b)
            assert np.mean(diff > 0) < 2e-2
            assert np.all(diff <= 2.0**-7 * np.abs(b) + 2.0**-9 * np.abs(b).max())
            assert np.mean(diff) <= 1e-4 * np.mean(np.abs(b))
    else:
        scale = max(float(np.abs(g["out"]).max()), 1e-30)
        assert np.max(np.abs(r["out"] - g["out"])) <= 1e-5 * scale


@pytest.mark.parametrize("case", BLOCK_SPECS, ids=[c[0].name for c in BLOCK_SPECS])
def test_oracle_block_with_norm_and_residual_matches_golden(case):
    """h + moe_swiglu_ffn(rms_norm(h)) (kappa/qwen3/block.py:196-207, norms.py:10-16)."""
    spec, eps = case
    inp = make_inputs(spec)
    scale = make_norm_scale(spec)
    assert digest({**inp, "norm_scale": scale}) == META[spec.name]["input_sha256"]
    g = np.load(os.path.join(HERE, f"{spec.name}.npz"))
    bf16 = spec.act == "bf16"
    r = oracle.forward_block(inp["x"], scale, inp["router"], inp["gate"], inp["up"], inp["down"], k=spec.K,
                             act_bf16=bf16, impl=spec.impl, eps=eps)  # fmt: skip
    # the normalised input: fp32 in the canonical order vs fp64, so a rare one-ulp
    # flip of the final rounding (bf16: 2^-8 relative; fp32: a few ulps)
    d = np.abs(r["h2"] - g["h2"])
    if bf16:
        assert np.mean(d > 0) < 2e-3
        assert np.all(d <= 2.0**-8 * np.abs(g["h2"]) + 1e-30)
    else:
        assert np.all(d <= 4 * np.finfo(np.float32).eps * np.abs(g["h2"]) + 1e-30)
    np.testing.assert_array_equal(r["idx"], g["idx"])
    for a, b in ((r["moe_out"], g["moe_out"]), (r["out"], g["out"])):
        if bf16:
            diff = np.abs(a - b)
            assert np.mean(diff > 0) < 2e-2
            assert np.all(diff <= 2.0**-7 * np.abs(b) + 2.0**-9 * np.abs(b).max())
            assert np.mean(diff) <= 1e-4 * np.mean(np.abs(b))
        else:
            assert np.max(np.abs(a - b)) <= 1e-5 * max(float(np.abs(b).max()), 1e-30)


# --- the goldens pin the rounding points ---------------------------------------


def _mean_rel(a, b):
    return float(np.mean(np.abs(a - b)) / np.mean(np.abs(b)))


def _old_contract(inp, spec):
    """The numerics an earlier contract of this build applied to every impl: the x.dtype
    expert chain with a single-rounding silu, then out = round(sum_j fma(w_j, y_j)) with
    one rounding (no bf16 product, no bf16 running add)."""
    r = oracle.forward(inp["x"], inp["router"], inp["gate"], inp["up"], inp["down"], k=spec.K, act_bf16=True,
                       impl="gather_einsum")  # fmt: skip
    y = r["y_sorted"][r["inv"]].reshape(spec.T, spec.K, -1).astype(np.float64)
    return oracle.bf16_round(np.sum(y * r["w"].astype(np.float64)[..., None], axis=1).astype(np.float32))


@pytest.mark.parametrize("name", ["r30_w8c", "w8c_bf16_k8", "w8c_bf16"])
def test_ragged_golden_rejects_other_rounding_schemes(name):
    """On the ragged program's goldens (f32 weights and intermediates, bf16 y, bf16
    product, bf16 scatter-add) the oracle passes the 1e-3 bar, and each plausible
    mistake fails it: the gather program's bf16 chain, the old single-rounding contract,
    a one-rounding combine, and h rounded to bf16 before the down product."""
    spec = next(s for s in GOLDEN_SPECS if s.name == name)
    inp = make_inputs(spec)
    g = np.load(os.path.join(HERE, f"{spec.name}.npz"))
    args = (inp["x"], inp["router"], inp["gate"], inp["up"], inp["down"])
    right = oracle.forward(*args, k=spec.K, act_bf16=True, impl="ragged")
    assert _mean_rel(right["out"], g["out"]) < 1e-4
    wrong = {}
    wrong["gather chain"] = oracle.forward(*args, k=spec.K, act_bf16=True, impl="gather_einsum")["out"]
    wrong["old contract"] = _old_contract(inp, spec)
    y = right["y_sorted"][right["inv"]].reshape(spec.T, spec.K, -1).astype(np.float64)
    wrong["one-rounding combine"] = oracle.bf16_round(np.sum(y * right["w"][..., None], axis=1).astype(np.float32))
    # h rounded to bf16 before the down product (a bf16-only MFMA feed)
    hb = oracle.bf16_round(right["h_sorted"])
    qd, sd = inp["down"]
    yb = np.empty_like(right["y_sorted"])
    for e in range(spec.E):
        a, b = right["offsets"][e], right["offsets"][e + 1]
        wd = qd[e].astype(np.float64) * sd[e].astype(np.float64)
        yb[a:b] = oracle.bf16_round((hb[a:b].astype(np.float64) @ wd).astype(np.float32))
    wrong["bf16 h"] = oracle.combine(yb, right["inv"], right["w"], True, impl="ragged")
    for what, out in wrong.items():
        assert _mean_rel(out, g["out"]) > 1e-3, f"{what}: {_mean_rel(out, g['out']):.2e}"


@pytest.mark.parametrize("name", ["g30_w8t", "w8t_bf16", "bf16_plain"])
def test_gather_golden_rejects_other_rounding_schemes(name):
    """The gather program's goldens reject the ragged program's f32 chain."""
    spec = next(s for s in GOLDEN_SPECS if s.name == name)
    inp = make_inputs(spec)
    g = np.load(os.path.join(HERE, f"{spec.name}.npz"))
    args = (inp["x"], inp["router"], inp["gate"], inp["up"], inp["down"])
    assert _mean_rel(oracle.forward(*args, k=spec.K, act_bf16=True, impl="gather_einsum")["out"], g["out"]) < 1e-4
    assert _mean_rel(oracle.forward(*args, k=spec.K, act_bf16=True, impl="ragged")["out"], g["out"]) > 1e-3


def test_fixed_capacity_golden_rejects_a_one_rounding_combine():
    """_moe_fixed_capacity adds bf16 products into a bf16 buffer (:155-157); a combine
    that sums in f32 and rounds once misses the bar on the 30B-shaped case."""
    spec, cf, slots = next(c for c in CAPACITY_SPECS if c[0].name == "cap30_w8c")
    inp = make_inputs(spec)
    g = np.load(os.path.join(HERE, f"{spec.name}.npz"))
    cap = oracle.capacity_slots(spec.T, spec.K, spec.E, cf, slots)
    r = oracle.forward(inp["x"], inp["router"], inp["gate"], inp["up"], inp["down"], k=spec.K, act_bf16=True,
                       impl="fixed_capacity", capacity=cap)  # fmt: skip
    assert _mean_rel(r["out"], g["out"]) < 1e-4
    one = oracle.combine(r["y_sorted"], r["inv"], r["w"], True, impl="gather_einsum")
    assert _mean_rel(one, g["out"]) > 1e-3
