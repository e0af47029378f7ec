"""HIP kernels against the oracle (GPU).

Every layer call names the reference array program it is checked against
(``impl``): the gather program (_moe_gather_einsum, kappa/qwen3/ffn_moe.py:74-104,
the default impl and what ragged_* run at T <= the decode threshold), the ragged
program (_moe_ragged, :174-216) or fixed_capacity (:107-158). The oracle restates
each program's rounding points (oracle/moe_oracle.c) and is pinned by the golden
vectors and property tests of the CPU suite.

Bar: top-k indices and the dispatch arrays bit-exact; router logits bit-exact
(the kernels and the oracle share the canonical summation order); layer outputs
within max-abs 2e-2 and mean-rel 1e-3 in bf16, 1e-5 (relative to the output scale)
in f32. mean-rel = mean|a - b| / mean|b|.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from inputs import CAPACITY_SPECS, GOLDEN_SPECS, Spec, make_inputs
from moe_cases import bf16_np, forward_args, layer_cfg, make_layer, make_x, mean_rel, oracle_rows, skew_router

pytestmark = pytest.mark.gpu

BF16_MAX_ABS = 2e-2
BF16_MEAN_REL = 1e-3
F32_REL = 1e-5


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    return torch.device("cuda:0")


def to_dev_weight(w, dev, act_bf16):
    from kappa_amd.qwen3 import Q8Weight

    if isinstance(w, tuple):
        q, s = w
        return Q8Weight(torch.from_numpy(np.ascontiguousarray(q)).to(dev), torch.as_tensor(np.asarray(s, np.float32)).to(dev))
    t = torch.from_numpy(np.ascontiguousarray(w, np.float32)).to(dev)
    return t.to(torch.bfloat16) if act_bf16 else t


def spec_to_dev(spec: Spec, inp: dict, dev):
    bf16 = spec.act == "bf16"
    x = torch.from_numpy(inp["x"]).to(dev)
    x = x.to(torch.bfloat16) if bf16 else x
    r = inp["router"]
    if isinstance(r, tuple):
        rd = to_dev_weight(r, dev, bf16)
    else:
        rd = torch.from_numpy(r).to(dev)
        rd = rd.to(torch.bfloat16) if spec.router == "bf16" else rd
    ws = [to_dev_weight(inp[n], dev, spec.weights == "bf16") for n in ("gate", "up", "down")]
    if spec.weights == "f32":
        ws = [torch.from_numpy(inp[n]).to(dev) for n in ("gate", "up", "down")]
    return x, rd, ws


def check_out(out: np.ndarray, ref: np.ndarray, bf16: bool, what: str = "out"):
    if bf16:
        d = np.abs(out - ref)
        print(f"{what}: max-abs {d.max():.2e} mean-rel {mean_rel(out, ref):.2e}")
        assert d.max() <= BF16_MAX_ABS, f"{what}: max-abs {d.max():.3e}"
        assert mean_rel(out, ref) <= BF16_MEAN_REL, f"{what}: mean-rel {mean_rel(out, ref):.3e}"
    else:
        scale = max(float(np.abs(ref).max()), 1e-30)
        assert np.abs(out - ref).max() <= F32_REL * scale, f"{what}: {np.abs(out - ref).max() / scale:.3e}"


def check_inter(out: np.ndarray, ref: np.ndarray, what: str):
    """bf16 intermediates (h of the gather program, y).

    The MFMA kernels and the oracle add the same products in different fp32 orders, so
    g, u and y may round to a neighbouring bf16 number; silu amplifies a flip in g (up to
    ~4x near g = -5) and y has cancellation near zero, so an elementwise ulp bound does not
    apply. The bar: mean-rel <= 1e-3, every difference within 4 bf16 ulps of the tensor's
    largest magnitude, and at most 10% of elements not bit-identical (a wrong rounding
    point or scale changes most elements)."""
    d = np.abs(out - ref)
    top = float(np.abs(ref).max())
    diff_frac = float(np.mean(d > 0))
    print(f"{what}: mean-rel {mean_rel(out, ref):.2e} max-abs {d.max():.2e} (max|ref| {top:.2e}) "
          f"not-identical {diff_frac:.4f}")  # fmt: skip
    assert mean_rel(out, ref) <= BF16_MEAN_REL, f"{what}: mean-rel {mean_rel(out, ref):.3e}"
    assert d.max() <= 2.0**-6 * top, f"{what}: max-abs {d.max():.3e} vs max|ref| {top:.3e}"
    assert diff_frac <= 0.10, f"{what}: {diff_frac:.3f} of elements differ"


def check_h32(h_dev: torch.Tensor, ref: np.ndarray, I: int, what: str = "h"):
    """The ragged program's f32 h: the kernels keep it as bf16 hi + lo (~2^-17 relative)
    and sum in another f32 order than the oracle; a bf16-rounded h would miss by 2^-9."""
    from kappa_amd.qwen3.moe_stages import h_float

    h = h_float(h_dev, I).cpu().numpy()
    d = np.abs(h - ref)
    top = float(np.abs(ref).max())
    print(f"{what}: max-abs {d.max():.2e} (max|ref| {top:.2e}) mean-rel {mean_rel(h, ref):.2e}")
    assert d.max() <= 3e-5 * top, f"{what}: {d.max():.3e} vs max|ref| {top:.3e}"
    assert mean_rel(h, ref) <= 2e-5


# --- golden cases: the whole block through the C ABI --------------------------


def _spec_forward(spec, inp, dev, kernels):
    from kappa_amd.qwen3.ffn_moe import _moe_forward

    x, r, (g, u, d) = spec_to_dev(spec, inp, dev)
    return _moe_forward(
        x.reshape(1, spec.T, spec.D), r, g, u, d, num_experts=spec.E, num_experts_per_tok=spec.K,
        packed=None, return_routing=True, kernels=kernels, **forward_args(spec.impl),
    )  # fmt: skip


@pytest.mark.parametrize("kernels", ["auto", "grouped"])
@pytest.mark.parametrize("spec", GOLDEN_SPECS, ids=[s.name for s in GOLDEN_SPECS])
def test_golden_block(dev, spec, kernels):
    """Each golden case through the program it restates, on the token-count kernel
    family and on the grouped GEMMs."""
    from kappa_amd import _lib

    inp = make_inputs(spec)
    bf16 = spec.act == "bf16"
    fam = _lib.KERNELS_AUTO if kernels == "auto" else _lib.KERNELS_GROUPED
    out, idx, w = _spec_forward(spec, inp, dev, fam)
    ref = oracle.forward(inp["x"], inp["router"], inp["gate"], inp["up"], inp["down"], k=spec.K, act_bf16=bf16,
                         impl=spec.impl)  # fmt: skip
    np.testing.assert_array_equal(idx.cpu().numpy(), ref["idx"])
    wg = w.float().cpu().numpy()
    assert np.all(np.abs(wg - ref["w"]) <= (2.0**-8 if bf16 else 2.0**-22) * np.abs(ref["w"]))
    got = out.reshape(spec.T, spec.D).float().cpu().numpy()
    check_out(got, ref["out"], bf16)
    # and against the golden vectors written from the literal restatement
    gold = np.load(f"tests/golden/{spec.name}.npz")
    np.testing.assert_array_equal(idx.cpu().numpy(), gold["idx"])
    check_out(got, gold["out"], bf16, "vs golden")


# --- the 30B-A3B and 235B-A22B layers ----------------------------------------


@pytest.fixture(scope="module")
def l30(dev):
    """Per-output-channel scales (the benchmark layer)."""
    return make_layer("30b", seed=0)


@pytest.fixture(scope="module")
def l30t(dev):
    """Per-tensor bf16 scales (the reference's quantize_weight): runs every program."""
    return make_layer("30b", seed=5, per_tensor=True)


def _route_and_dispatch(x, layer_router, E, K):
    from kappa_amd.qwen3 import moe_stages

    r = moe_stages.route(x, layer_router, num_experts=E, k=K)
    d = moe_stages.dispatch(r["idx"], r["hist"], num_experts=E)
    return r, d


def _check_routing(x, router, E, K, r, d):
    xn = bf16_np(x)
    rn = router.float().cpu().numpy()
    lg = oracle.router_logits(xn, rn)
    np.testing.assert_array_equal(r["logits"].cpu().numpy(), lg)  # canonical order: bit-exact
    idx, w = oracle.topk_softmax(lg, K, act_bf16=True)
    np.testing.assert_array_equal(r["idx"].cpu().numpy(), idx)
    wd = r["w"].cpu().numpy()
    assert np.mean(wd != w) < 1e-3 and np.all(np.abs(wd - w) <= 2.0**-8 * w)
    od = oracle.dispatch(idx, E)
    for n in ("group_sizes", "offsets", "sorted_token", "inv"):
        np.testing.assert_array_equal(d[n].cpu().numpy(), od[n], err_msg=n)
    np.testing.assert_array_equal(d["sorted_expert"].cpu().numpy(), idx.reshape(-1)[od["order"]])
    act = np.nonzero(od["group_sizes"])[0]
    a = d["active"].cpu().numpy()
    assert a[E] == len(act)
    np.testing.assert_array_equal(a[: len(act)], act)
    return xn, idx, w, od


def _decode_full(layer, T, impl, seed):
    """Whole decode call and its stages against the oracle of ``impl``'s program."""
    from kappa_amd.qwen3 import moe_stages, moe_swiglu_ffn

    x = make_x(T, layer.D, seed=seed)
    r, d = _route_and_dispatch(x, layer.router, layer.E, layer.K)
    xn, idx, w, od = _check_routing(x, layer.router, layer.E, layer.K, r, d)
    host = layer.host()
    h, y = moe_stages.expert_ffn(x, d, layer.gate, layer.up, layer.down, k=layer.K, impl=impl)
    ho, yo = oracle.expert_ffn(xn, od["offsets"], od["sorted_token"], host["gate"], host["up"], host["down"], True,
                               impl=impl)  # fmt: skip
    if impl == "ragged":
        check_h32(h, ho, layer.I)
    else:
        check_inter(bf16_np(h), ho, "h")
    check_inter(bf16_np(y), yo, "y")
    out = moe_swiglu_ffn(x.reshape(1, T, layer.D), layer.router, layer.gate, layer.up, layer.down,
                         cfg=layer_cfg(layer, impl))  # fmt: skip
    ref = oracle.combine(yo, od["inv"], w, True, impl=impl)
    check_out(bf16_np(out.reshape(T, layer.D)), ref, True)
    # the staged combine follows the same program
    staged = moe_stages.combine(y, d["inv"], r["w"], k=layer.K, impl=impl)
    check_out(bf16_np(staged), ref, True, "staged combine")


@pytest.mark.parametrize("T", [1, 8, 32, 64])
def test_30b_decode_ragged_per_channel(dev, l30, T):
    """The benchmark decode configuration: per-channel W8 on the ragged program
    (ragged_jax, decode threshold 0)."""
    _decode_full(l30, T, "ragged", seed=T)


@pytest.mark.parametrize("T", [1, 8, 32, 64])
def test_30b_decode_gather_per_tensor(dev, l30t, T):
    """The reference's default decode program (gather_einsum) on per-tensor W8."""
    _decode_full(l30t, T, "gather_einsum", seed=40 + T)


@pytest.mark.parametrize("T", [8, 64])
def test_30b_decode_ragged_per_tensor(dev, l30t, T):
    _decode_full(l30t, T, "ragged", seed=80 + T)


def _prefill_sampled(layer, T, seed, router=None, x=None, n_tok=48, impl="ragged", cfg=None, kernels=None):
    """kernels: a kernel-family pin for the expert stage and the block (None:
    the block through moe_swiglu_ffn, which chooses by T)."""
    from kappa_amd.qwen3 import moe_stages, moe_swiglu_ffn
    from kappa_amd.qwen3.ffn_moe import _moe_forward

    router = layer.router if router is None else router
    x = make_x(T, layer.D, seed=seed) if x is None else x
    r, d = _route_and_dispatch(x, router, layer.E, layer.K)
    xn, idx, w, od = _check_routing(x, router, layer.E, layer.K, r, d)
    pin = {} if kernels is None else {"kernels": kernels}
    h, y = moe_stages.expert_ffn(x, d, layer.gate, layer.up, layer.down, k=layer.K, impl=impl, **pin)
    if kernels is None:
        out = moe_swiglu_ffn(x.reshape(1, T, layer.D), router, layer.gate, layer.up, layer.down,
                             cfg=cfg or layer_cfg(layer, impl))  # fmt: skip
    else:
        out = _moe_forward(
            x.reshape(1, T, layer.D), router, layer.gate, layer.up, layer.down, num_experts=layer.E,
            num_experts_per_tok=layer.K, packed=None, kernels=kernels, **forward_args(impl),
        )  # fmt: skip
    rng = np.random.default_rng(seed)
    toks = np.sort(rng.choice(T, size=min(n_tok, T), replace=False))
    toks = np.unique(np.concatenate([toks, [0, T - 1]]))
    rows_t = np.repeat(toks, layer.K)
    rows_e = idx[toks].reshape(-1)
    ho, yo = oracle_rows(oracle, xn, rows_t, rows_e, layer.host(), impl=impl)
    pos = od["inv"].reshape(T, layer.K)[toks].reshape(-1)
    if impl == "ragged":
        check_h32(h[torch.from_numpy(pos).to(h.device).long()], ho, layer.I, "h rows")
    else:
        check_inter(bf16_np(h)[pos], ho, "h rows")
    check_inter(bf16_np(y)[pos], yo, "y rows")
    ref = oracle.combine(yo, np.arange(len(rows_t), dtype=np.int32), w[toks], True, impl=impl)
    check_out(bf16_np(out.reshape(T, layer.D))[toks], ref, True, "out rows")
    return od


@pytest.mark.parametrize("T", [240, 512, 704, 1024, 1280, 1535, 1536, 2048, 2049, 3001, 4096])
def test_30b_prefill_ragged(dev, l30, T):
    """The prefill chunks under the reference's ragged program (ragged_jax with its
    default threshold of 64: these sizes run _moe_ragged). Every grouped-GEMM tile
    form is reached: 64-row tiles (T=240, 512, 704), 128-row tiles with
    nontemporal weights (T=1024, 64 rows per expert) and without (T=1280, 80),
    160-row tiles with (T=2048) and without (T=3001, 4096). From T=1536 (96 rows
    per expert) the down product takes h as int8 planes; T=1535 is the last size
    with the bf16 hi and lo planes. T=2049 and 3001 leave the two-phase router
    a last block of one and of nine tokens and the dispatch a partial 64-token
    chunk."""
    from kappa_amd.qwen3 import moe_layer_config

    cfg = moe_layer_config(hidden=l30.D, experts=l30.E, top_k=l30.K, intermediate=l30.I, moe_impl="ragged_jax")
    _prefill_sampled(l30, T, seed=100 + T, cfg=cfg)


@pytest.mark.parametrize("shape", ["odd", "e256", "i960"])
def test_other_layer_shapes(dev, shape):
    """Layers outside the Qwen3 presets through every size class of the packed
    kernels, against the oracle: D = 2560, I = 1024, E = 64, top-6 (the decode
    GEMVs' guarded load batches, whose chunks a wave's batches do not divide;
    the all-VALU router at every size, D / 64 = 40 slices padded to 64; the
    int8-plane down product at T = 2048, 192 rows per expert); 256 experts
    (D = 2048, I = 768, top-8); and I = 960 with 32 experts, top-4 (fifteen
    64-wide chunks: the grouped GEMM for I % 128 != 0, unequal chunk counts
    per wave in the decode down GEMV and the fused down + combine)."""
    layer = make_layer(shape, seed=3)
    for T in (1, 4, 8, 40, 64, 200, 1000, 2048):
        _prefill_sampled(layer, T, seed=2700 + T, n_tok=12)


def test_other_layer_shape_gather_per_tensor(dev):
    """The D = 2560, I = 1024, 64-expert, top-6 layer with per-tensor W8 under
    the gather program (the x.dtype chain of the same kernels)."""
    layer = make_layer("odd", seed=4, per_tensor=True)
    for T in (1, 8, 64, 1000):
        _prefill_sampled(layer, T, seed=2800 + T, n_tok=12, impl="gather_einsum")


@pytest.mark.parametrize("K", [1, 2, 4])
def test_30b_other_top_k(dev, l30, K):
    """The reference takes any num_experts_per_tok: the 30B-A3B layer with top-1,
    top-2 and top-4 routing on the packed kernels of each size class (the
    whole-block decode call with its fused down + combine at T = 1 and 4, the
    decode kernels at T = 64, the grouped GEMMs at T = 1024 and 4096), under
    the ragged program."""
    import dataclasses

    layer = dataclasses.replace(l30, K=K)
    for T in (1, 4, 64, 1024, 4096):
        _prefill_sampled(layer, T, seed=2600 + 10 * K + T, n_tok=16)


@pytest.mark.parametrize("T", [8192, 16384, 32768])
def test_30b_prefill_whole_prompts(dev, l30, T):
    """Prefill without chunking (the reference's default, prefill_chunk_size=None,
    kappa/qwen3/generate.py:48-65, passes a whole prompt to the layer): up to
    32768 tokens (262144 assignment rows, ~2000 rows per expert) under the
    ragged program, routing in full and sampled rows against the oracle."""
    from kappa_amd.qwen3 import moe_layer_config

    cfg = moe_layer_config(hidden=l30.D, experts=l30.E, top_k=l30.K, intermediate=l30.I, moe_impl="ragged_jax")
    _prefill_sampled(l30, T, seed=3000 + T, cfg=cfg, n_tok=16)


@pytest.mark.parametrize("T", [512, 1024, 4096])
def test_30b_prefill_gather_per_tensor(dev, l30t, T):
    """The gather program (the default impl) at prefill sizes on the grouped GEMMs
    (64-, 128- and 160-row tiles)."""
    _prefill_sampled(l30t, T, seed=150 + T, impl="gather_einsum", n_tok=24)


@pytest.mark.parametrize("T", [65, 100, 128])
def test_30b_rows_path(dev, l30, T):
    """65..128 tokens with the decode kernels asked for run them over all of an
    expert's rows in groups of 64 (the skewed router puts more than 64 rows on
    its hot experts, so those take several groups); left to choose, the same
    sizes run the grouped GEMMs. Routing bit-exact, sampled rows and h/y
    against the oracle."""
    from kappa_amd import _lib

    for kernels in (_lib.KERNELS_DECODE, None):
        _prefill_sampled(l30, T, seed=500 + T, n_tok=24, kernels=kernels)
    x = make_x(T, l30.D, seed=600 + T)
    x[:, 0] = 1.0
    router = skew_router(l30.router, lam=1.5)
    for kernels in (_lib.KERNELS_DECODE, None):
        od = _prefill_sampled(l30, T, seed=600 + T, router=router, x=x, n_tok=24, kernels=kernels)
        assert int(np.max(od["group_sizes"])) > 64 or T < 100


def test_30b_skewed_routing(dev, l30):
    """Hot experts at T=512 hold several 64-row GEMM tiles (their rows split
    evenly over them); at T=4096 several 160-row tiles."""
    for T, seed in ((4096, 7), (512, 9), (64, 8)):
        x = make_x(T, l30.D, seed=seed)
        x[:, 0] = 1.0
        router = skew_router(l30.router, lam=1.5)
        od = _prefill_sampled(l30, T, seed, router=router, x=x)
        share = np.sort(od["group_sizes"])[::-1][:8].sum() / (T * l30.K)
        assert share > 0.5, f"hot-expert share {share:.2f}"
        if T == 512:
            assert int(np.max(od["group_sizes"])) > 128


@pytest.mark.parametrize("T", [512, 1000, 1536])
def test_235b_prefill_tile_forms(dev, T):
    """The 235B-A22B layer (D = 4096, I = 1536) on the grouped GEMMs' other
    tile forms: 64-row tiles (T = 512, 32 rows per expert), 128-row tiles with
    nontemporal weights (T = 1000, ~62 rows), and 160-row tiles with the down
    product on int8 planes of h (T = 1536, 96 rows)."""
    layer = make_layer("235b", seed=1)
    _prefill_sampled(layer, T, seed=2300 + T, n_tok=16)


def test_235b_layer(dev):
    from kappa_amd import _lib
    from kappa_amd.qwen3 import moe_block_ffn, moe_stages, moe_swiglu_ffn, rms_norm

    layer = make_layer("235b", seed=1)
    cfg = layer_cfg(layer, "ragged")
    _prefill_sampled(layer, 16, seed=16, n_tok=16)
    # 16 < T <= 64 at D = 4096: the gate/up kernel's 16-row groups spread over
    # blocks, a skewed router putting more than 16 rows on its hot experts
    x40 = make_x(40, layer.D, seed=40)
    x40[:, 0] = 1.0
    od = _prefill_sampled(layer, 40, seed=40, n_tok=16, router=skew_router(layer.router, lam=1.5), x=x40)
    assert int(np.max(od["group_sizes"])) > 16
    _prefill_sampled(layer, 100, seed=100, n_tok=16, kernels=_lib.KERNELS_DECODE)  # the row-group kernels
    _prefill_sampled(layer, 2048, seed=2048, n_tok=24)
    # the block call at T = 100: the split router normalising 4096-wide rows
    # (four tokens per block)
    h = make_x(100, layer.D, seed=101).reshape(1, 100, layer.D)
    sc = (1.0 + 0.1 * torch.randn(layer.D, device=dev)).to(torch.bfloat16)
    composed = h + moe_swiglu_ffn(rms_norm(h, sc), layer.router, layer.gate, layer.up, layer.down, cfg=cfg)
    assert torch.equal(moe_block_ffn(h, sc, layer.router, layer.gate, layer.up, layer.down, cfg=cfg), composed)
    # T = 1, 2 and 4: the whole layer (the gate/up kernel finishing the routing
    # itself, its dense token tile in two load batches per wave; fused down +
    # combine, each wave holding 12 of the 24 chunks of the reduction) against
    # the staged calls
    for T in (1, 2, 4):
        _prefill_sampled(layer, T, seed=T, n_tok=T)
        x = make_x(T, layer.D, seed=T)
        r, d = _route_and_dispatch(x, layer.router, layer.E, layer.K)
        h, y = moe_stages.expert_ffn(x, d, layer.gate, layer.up, layer.down, k=layer.K, impl="ragged")
        staged = moe_stages.combine(y, d["inv"], r["w"], k=layer.K, impl="ragged")
        out = moe_swiglu_ffn(x.reshape(1, T, layer.D), layer.router, layer.gate, layer.up, layer.down, cfg=cfg)
        assert torch.equal(out.reshape(T, layer.D), staged.reshape(T, layer.D))
    # a token's output does not depend on its batch across the D = 4096 shape
    # switches: dense tile / gathered rows (T = 4/5), eight / four gate/up waves
    # (T = 16/17)
    for T in (4, 16):
        x = make_x(T + 1, layer.D, seed=900 + T)
        a = moe_swiglu_ffn(x[:T].reshape(1, T, layer.D), layer.router, layer.gate, layer.up, layer.down, cfg=cfg)
        b = moe_swiglu_ffn(x.reshape(1, T + 1, layer.D), layer.router, layer.gate, layer.up, layer.down, cfg=cfg)
        assert torch.equal(a.reshape(T, layer.D), b.reshape(T + 1, layer.D)[:T]), f"T={T}"
    del layer
    torch.cuda.empty_cache()


# --- cross-checks between kernel families, determinism, edge cases -----------


@pytest.mark.parametrize("impl", ["ragged", "gather_einsum"])
def test_decode_and_grouped_kernels_agree(dev, l30, l30t, impl):
    """The GEMV-style kernels and the grouped GEMMs follow the same program: they agree
    within the bar (scripts/verify_qwen3_moe_impls.py:61-70 cross-checks the
    reference's own paths the same way)."""
    from kappa_amd import _lib
    from kappa_amd.qwen3.ffn_moe import _moe_forward

    layer = l30 if impl == "ragged" else l30t
    for T in (1, 16, 64, 65, 128):
        x = make_x(T, layer.D, seed=300 + T).reshape(1, T, layer.D)
        outs = [
            bf16_np(_moe_forward(x, layer.router, layer.gate, layer.up, layer.down, num_experts=layer.E,
                                 num_experts_per_tok=layer.K, packed=None, kernels=k, **forward_args(impl)))
            for k in (_lib.KERNELS_AUTO, _lib.KERNELS_GROUPED)
        ]  # fmt: skip
        check_out(outs[0], outs[1], True, f"T={T}")


@pytest.mark.parametrize("impl", ["ragged", "gather_einsum"])
@pytest.mark.parametrize("T", [1, 2, 8, 16, 17, 40, 64, 65, 100, 128])
def test_whole_block_matches_staged_path(dev, l30, l30t, T, impl):
    """At T <= 128 the whole-block call routes with the split router (many
    blocks per token); the staged calls use the one-block-per-token router.
    Both follow the canonical summation order, so selections, weights and
    outputs are bit-identical. The skewed router puts up to T rows on an
    expert (above 64 tokens: two dispatch chunks, and row groups in the
    expert kernels)."""
    from kappa_amd.qwen3 import moe_stages
    from kappa_amd.qwen3.ffn_moe import PACK_CACHE, _moe_forward

    layer = l30 if impl == "ragged" else l30t
    for router in (layer.router, skew_router(layer.router, lam=1.5)):
        x = make_x(T, layer.D, seed=700 + T)
        x[:, 0] = 1.0
        r, d = _route_and_dispatch(x, router, layer.E, layer.K)
        h, y = moe_stages.expert_ffn(x, d, layer.gate, layer.up, layer.down, k=layer.K, impl=impl)
        staged = moe_stages.combine(y, d["inv"], r["w"], k=layer.K, impl=impl)
        packed = PACK_CACHE.get(layer.gate, layer.up, layer.down)
        for _ in range(2):
            out, idx, w = _moe_forward(
                x.reshape(1, T, layer.D), router, layer.gate, layer.up, layer.down, num_experts=layer.E,
                num_experts_per_tok=layer.K, packed=packed, return_routing=True, **forward_args(impl),
            )  # fmt: skip
            assert torch.equal(idx, r["idx"])
            assert torch.equal(w.float(), r["w"])
            assert torch.equal(out.reshape(T, layer.D), staged.reshape(T, layer.D))


@pytest.mark.parametrize("impl", ["ragged", "gather_einsum"])
def test_large_chunks_feed_h_as_int8_planes(dev, l30, l30t, impl):
    """From 96 rows per expert on average (30B-A3B: 1536 tokens) the whole-block
    call's f32-chain down product takes h as two int8 planes with a per-row scale
    (15 bits relative to the row's largest |h|) instead of bf16 hi and lo planes;
    the staged calls keep hi and lo. So the ragged program's outputs differ from
    the staged ones by the feed's rounding alone: a few 1e-4 mean-rel, inside the
    1e-3 bar, and not bit for bit (the planes path ran). The gather program's
    x.dtype chain has no f32 h: bit-identical."""
    from kappa_amd.qwen3 import moe_stages
    from kappa_amd.qwen3.ffn_moe import PACK_CACHE, _moe_forward

    layer = l30 if impl == "ragged" else l30t
    T = 2048
    x = make_x(T, layer.D, seed=1700)
    r, d = _route_and_dispatch(x, layer.router, layer.E, layer.K)
    h, y = moe_stages.expert_ffn(x, d, layer.gate, layer.up, layer.down, k=layer.K, impl=impl)
    staged = moe_stages.combine(y, d["inv"], r["w"], k=layer.K, impl=impl).reshape(T, layer.D)
    packed = PACK_CACHE.get(layer.gate, layer.up, layer.down)
    out, idx, w = _moe_forward(
        x.reshape(1, T, layer.D), layer.router, layer.gate, layer.up, layer.down, num_experts=layer.E,
        num_experts_per_tok=layer.K, packed=packed, return_routing=True, **forward_args(impl),
    )  # fmt: skip
    out = out.reshape(T, layer.D)
    assert torch.equal(idx, r["idx"])
    if impl == "gather_einsum":
        assert torch.equal(out, staged)
        return
    a, b = bf16_np(out), bf16_np(staged)
    rel, mabs = mean_rel(a, b), float(np.abs(a - b).max())
    print(f"planes vs hi/lo: max-abs {mabs:.2e} mean-rel {rel:.2e}")
    assert not torch.equal(out, staged)
    assert 1e-5 < rel <= 5e-4 and mabs <= 2e-2


def test_large_chunk_nonfinite_row_stays_in_its_token(dev, l30):
    """In the int8-plane down product every h row has its own scale: a token
    whose h overflows f32 (x of 3e38) gets a non-finite output row, and every
    other token's output stays finite and equal, to rounding, to the same call
    with that token replaced by an ordinary row."""
    from kappa_amd.qwen3.ffn_moe import _moe_forward

    T, bad = 2048, 7
    x = make_x(T, l30.D, seed=1800)
    clean = x.clone()
    x[bad] = 3e38
    outs = []
    for xi in (x, clean):
        o = _moe_forward(
            xi.reshape(1, T, l30.D), l30.router, l30.gate, l30.up, l30.down, num_experts=l30.E,
            num_experts_per_tok=l30.K, packed=None, **forward_args("ragged"),
        )  # fmt: skip
        outs.append(bf16_np(o.reshape(T, l30.D)))
    keep = np.arange(T) != bad
    assert not np.isfinite(outs[0][bad]).all()
    assert np.isfinite(outs[0][keep]).all()
    assert mean_rel(outs[0][keep], outs[1][keep]) <= 1e-5


@pytest.mark.parametrize("T", [8, 64, 512, 2048])
def test_nan_gate_scale_reaches_exactly_its_experts_tokens(dev, l30, T):
    """A NaN scale on one gate column of expert e: in the reference every h row
    of e is NaN in that column (silu(g) * u, kappa/qwen3/ffn_moe.py:209), so
    y = h @ W_down is NaN across the row and so is the output of every token
    routed to e, with no inf anywhere; every other token's output is unchanged
    (bit-identical to the clean layer). T = 8 and 64 run the decode kernels,
    512 the hi + lo down GEMM, 2048 the int8-plane down product, whose plane
    pass must flag a row holding a NaN and no inf."""
    from kappa_amd.qwen3 import Q8Weight
    from kappa_amd.qwen3.ffn_moe import _moe_forward

    x = make_x(T, l30.D, seed=1900 + T)
    r, _ = _route_and_dispatch(x, l30.router, l30.E, l30.K)
    idx = r["idx"].cpu().numpy()
    e = int(idx[0, 0])
    sc = l30.gate.scale.clone()
    sc[e, 0, 5] = float("nan")
    gates = (Q8Weight(l30.gate.values, sc), l30.gate)
    outs = []
    for g in gates:
        o = _moe_forward(
            x.reshape(1, T, l30.D), l30.router, g, l30.up, l30.down, num_experts=l30.E,
            num_experts_per_tok=l30.K, packed=None, **forward_args("ragged"),
        )  # fmt: skip
        outs.append(bf16_np(o.reshape(T, l30.D)))
    hit = (idx == e).any(axis=1)
    print(f"T={T}: expert {e} holds {int(hit.sum())} tokens")
    assert np.isnan(outs[0][hit]).all()
    assert np.array_equal(outs[0][~hit], outs[1][~hit])


@pytest.mark.parametrize("T", [4, 64, 512])
def test_packed_experts_alone(dev, l30, T):
    """A model that prepacked at load time passes packed= and no source weights; the
    call runs the same kernels as with them (bit-identical)."""
    from kappa_amd.qwen3 import moe_swiglu_ffn, prepack_moe_experts

    packed = prepack_moe_experts(l30.gate, l30.up, l30.down)
    x = make_x(T, l30.D, seed=900 + T).reshape(1, T, l30.D)
    cfg = layer_cfg(l30, "ragged")
    with_src = moe_swiglu_ffn(x, l30.router, l30.gate, l30.up, l30.down, cfg=cfg, packed=packed)
    alone = moe_swiglu_ffn(x, l30.router, None, None, None, cfg=cfg, packed=packed)
    assert torch.equal(with_src, alone)


@pytest.mark.parametrize("T,K", [(1, 8), (2, 4), (2, 8), (3, 8), (8, 8)])
def test_whole_block_with_drops_matches_staged_path(dev, l30, T, K):
    """Capacity 1 under a skewed router drops assignments whenever two tokens
    pick one expert; at T * K <= 32 the whole-block call runs the down
    projection and the combine as one kernel, which must skip the dropped rows
    exactly as the staged combine does and give the staged output bit for
    bit."""
    from kappa_amd.qwen3 import moe_stages
    from kappa_amd.qwen3.ffn_moe import PACK_CACHE, _moe_forward

    router = skew_router(l30.router, lam=1.5)
    x = make_x(T, l30.D, seed=760 + T)
    x[:, 0] = 1.0
    r = moe_stages.route(x, router, num_experts=l30.E, k=K)
    d = moe_stages.dispatch(r["idx"], r["hist"], num_experts=l30.E, capacity=1)
    if T > 1:
        assert bool((d["inv"] < 0).any())
    h, y = moe_stages.expert_ffn(x, d, l30.gate, l30.up, l30.down, k=K, impl="fixed_capacity", capacity=1)
    staged = moe_stages.combine(y, d["inv"], r["w"], k=K, impl="fixed_capacity")
    out = _moe_forward(
        x.reshape(1, T, l30.D), router, l30.gate, l30.up, l30.down, num_experts=l30.E, num_experts_per_tok=K,
        impl="fixed_capacity", decode_threshold=64, packed=PACK_CACHE.get(l30.gate, l30.up, l30.down), capacity=1,
    )  # fmt: skip
    assert torch.equal(out.reshape(T, l30.D), staged.reshape(T, l30.D))


@pytest.mark.parametrize("impl", ["ragged", "gather_einsum"])
@pytest.mark.parametrize("T,K", [(1, 1), (1, 8), (3, 2), (4, 2), (8, 1), (2, 3), (2, 8), (3, 8), (4, 8), (13, 2), (5, 6)])
def test_fused_down_combine_shapes(dev, l30, l30t, T, K, impl):
    """The whole-block call at T * K <= 32 (down projection and combine in one
    kernel; blocks of 8 / K tokens, two waves per assignment, 16 combine
    threads per token; a last block with fewer tokens) against the staged
    calls, bit for bit, on both rounding chains."""
    from kappa_amd.qwen3 import moe_stages
    from kappa_amd.qwen3.ffn_moe import PACK_CACHE, _moe_forward

    layer = l30 if impl == "ragged" else l30t
    x = make_x(T, layer.D, seed=830 + 10 * T + K)
    r = moe_stages.route(x, layer.router, num_experts=layer.E, k=K)
    d = moe_stages.dispatch(r["idx"], r["hist"], num_experts=layer.E)
    h, y = moe_stages.expert_ffn(x, d, layer.gate, layer.up, layer.down, k=K, impl=impl)
    staged = moe_stages.combine(y, d["inv"], r["w"], k=K, impl=impl)
    out = _moe_forward(
        x.reshape(1, T, layer.D), layer.router, layer.gate, layer.up, layer.down, num_experts=layer.E,
        num_experts_per_tok=K, packed=PACK_CACHE.get(layer.gate, layer.up, layer.down), **forward_args(impl),
    )  # fmt: skip
    assert torch.equal(out.reshape(T, layer.D), staged.reshape(T, layer.D))


@pytest.mark.parametrize("T", [1, 4, 8, 15, 16, 63, 100, 127])
def test_decode_batch_invariance(dev, l30, T):
    """A token's output does not depend on the other tokens of the call, on
    either side of 64 tokens: the first T rows of a (T + 1)-token call equal
    the T-token call bit for bit. The pairs up to 64 cross every kernel-shape
    switch of the decode kernels: the fused down + combine (T * K <= 32), the
    dense token tile of the gate/up kernel (T <= 4), the one-block router
    finish and dispatch (T <= 16), and eight against four gate/up waves
    (T = 16/17; both sum the same eight reduction parts in the same order).
    From 65 tokens the grouped GEMMs sum each row's products in another
    order, the same for every row and tile shape (T = 100/101, 127/128)."""
    from kappa_amd.qwen3 import moe_swiglu_ffn

    cfg = layer_cfg(l30, "ragged")
    x = make_x(T + 1, l30.D, seed=880 + T)
    a = moe_swiglu_ffn(x[:T].reshape(1, T, l30.D), l30.router, l30.gate, l30.up, l30.down, cfg=cfg)
    b = moe_swiglu_ffn(x.reshape(1, T + 1, l30.D), l30.router, l30.gate, l30.up, l30.down, cfg=cfg)
    assert torch.equal(a.reshape(T, l30.D), b.reshape(T + 1, l30.D)[:T])


@pytest.mark.parametrize("impl", ["ragged", "gather_einsum"])
def test_layout_native_experts_match_packed(dev, l30, l30t, impl):
    from kappa_amd.qwen3 import moe_stages

    layer = l30 if impl == "ragged" else l30t
    for T in (8, 200):
        x = make_x(T, layer.D, seed=400 + T)
        r, d = _route_and_dispatch(x, layer.router, layer.E, layer.K)
        h1, y1 = moe_stages.expert_ffn(x, d, layer.gate, layer.up, layer.down, k=layer.K, impl=impl)
        h2, y2 = moe_stages.expert_ffn(x, d, layer.gate, layer.up, layer.down, k=layer.K, impl=impl,
                                       layout_native=True)  # fmt: skip
        if impl == "ragged":
            from kappa_amd.qwen3.moe_stages import h_float

            check_h32(h1, h_float(h2, layer.I).cpu().numpy(), layer.I)
        else:
            check_inter(bf16_np(h1), bf16_np(h2), "h")
        check_inter(bf16_np(y1), bf16_np(y2), "y")


def test_repeat_runs_are_bitwise_identical(dev, l30):
    from kappa_amd.qwen3 import moe_swiglu_ffn

    cfg = layer_cfg(l30, "ragged")
    for T in (7, 333):
        x = make_x(T, l30.D, seed=500 + T).reshape(1, T, l30.D)
        a = moe_swiglu_ffn(x, l30.router, l30.gate, l30.up, l30.down, cfg=cfg)
        b = moe_swiglu_ffn(x, l30.router, l30.gate, l30.up, l30.down, cfg=cfg)
        assert torch.equal(a, b)


@pytest.mark.parametrize("T", [0, 3, 65, 1000])
def test_ragged_token_counts(dev, T):
    from kappa_amd.qwen3 import moe_layer_config, moe_swiglu_ffn

    spec = Spec("ragged", T=max(T, 1), D=128, E=16, K=4, I=64, base_seed=80 + T)
    inp = make_inputs(spec)
    x, r, (g, u, d) = spec_to_dev(spec, inp, dev)
    x = x[:T].reshape(1, T, spec.D)
    # threshold -1: the ragged program also at T = 0 (T <= 0 would select the gather
    # program, which has no per-channel form)
    cfg = moe_layer_config(hidden=128, experts=16, top_k=4, intermediate=64, moe_impl="ragged_jax",
                           moe_ragged_decode_token_threshold=-1)  # fmt: skip
    out = moe_swiglu_ffn(x, r, g, u, d, cfg=cfg)
    assert out.shape == (1, T, 128) and out.dtype == torch.bfloat16
    if T:
        ref = oracle.forward(inp["x"][:T], inp["router"], inp["gate"], inp["up"], inp["down"], k=4, act_bf16=True,
                             impl="ragged")  # fmt: skip
        check_out(bf16_np(out.reshape(T, 128)), ref["out"], True)


@pytest.mark.parametrize(
    "spec",
    [
        Spec("odd_e_bf16", T=5, D=100, E=9, K=3, I=32, base_seed=150, impl="ragged"),  # per-element router loads
        Spec("tiny_e_f32", T=3, D=64, E=3, K=1, I=32, act="f32", weights="f32", router="f32", base_seed=151),
        Spec("e33_qrouter", T=17, D=192, E=33, K=4, I=64, router="w8t", scale_dtype="bf16", base_seed=152,
             impl="ragged"),  # fmt: skip
        Spec("wide_d_bf16", T=9, D=4096, E=64, K=6, I=64, base_seed=153, impl="ragged"),  # 64 slices: Q = 16 groups
        Spec("e200_bf16", T=40, D=256, E=200, K=8, I=32, weights="w8t", scale_dtype="bf16", base_seed=154),
    ],
    ids=lambda s: s.name,
)
def test_split_router_shapes_match_oracle(dev, spec):
    """The whole-block call at T <= 64 routes with the split router: top-k
    indices bit-exact against the oracle (its canonical order) and the output
    within tolerance, on shapes that take its less common paths."""
    from kappa_amd import _lib

    inp = make_inputs(spec)
    bf16 = spec.act == "bf16"
    out, idx, w = _spec_forward(spec, inp, dev, _lib.KERNELS_AUTO)
    ref = oracle.forward(inp["x"], inp["router"], inp["gate"], inp["up"], inp["down"], k=spec.K, act_bf16=bf16,
                         impl=spec.impl)  # fmt: skip
    np.testing.assert_array_equal(idx.cpu().numpy(), ref["idx"])
    np.testing.assert_array_equal(w.float().cpu().numpy(), ref["w"])
    check_out(out.reshape(spec.T, spec.D).float().cpu().numpy(), ref["out"], bf16)


def test_legacy_entry_point_runs_the_gather_program(dev, l30t):
    """moe_swiglu_ffn_legacy (kappa/qwen3/ffn_moe.py:302-316) ignores config flags and
    always runs the gather program: one decode and one prefill token count."""
    from kappa_amd.qwen3 import moe_swiglu_ffn_legacy

    host = l30t.host()
    for T, n_tok in ((8, 8), (512, 16)):
        x = make_x(T, l30t.D, seed=1200 + T)
        out = moe_swiglu_ffn_legacy(x.reshape(1, T, l30t.D), l30t.router, l30t.gate, l30t.up, l30t.down,
                                    num_experts=l30t.E, num_experts_per_tok=l30t.K)  # fmt: skip
        xn = bf16_np(x)
        idx, w = oracle.topk_softmax(oracle.router_logits(xn, l30t.router.float().cpu().numpy()), l30t.K, True)
        toks = np.unique(np.concatenate([np.random.default_rng(T).choice(T, n_tok, replace=False), [0, T - 1]]))
        rows_t = np.repeat(toks, l30t.K)
        _, yo = oracle_rows(oracle, xn, rows_t, idx[toks].reshape(-1), host, impl="gather_einsum")
        ref = oracle.combine(yo, np.arange(len(rows_t), dtype=np.int32), w[toks], True, impl="gather_einsum")
        check_out(bf16_np(out.reshape(T, l30t.D))[toks], ref, True, f"legacy T={T}")


def test_gather_program_rejects_per_channel_layer(dev, l30):
    from kappa_amd.qwen3 import moe_swiglu_ffn

    x = make_x(4, l30.D, seed=1).reshape(1, 4, l30.D)
    with pytest.raises(ValueError, match="one scale per tensor"):
        moe_swiglu_ffn(x, l30.router, l30.gate, l30.up, l30.down, cfg=layer_cfg(l30, "gather_einsum"))


# --- weights ------------------------------------------------------------------


def test_quantiser_matches_oracle(dev):
    from kappa_amd.qwen3 import quantize_weight_per_channel

    rng = np.random.default_rng(12)
    w = (rng.standard_normal((3, 512, 96)) * 0.02).astype(np.float32)
    q, s = quantize_weight_per_channel(torch.from_numpy(w).to(dev))
    qo, so = oracle.quantize_per_channel(w)
    np.testing.assert_array_equal(q.cpu().numpy(), qo)
    np.testing.assert_array_equal(s.cpu().numpy(), so)
    wb = torch.from_numpy(w).to(dev).to(torch.bfloat16)
    q2, s2 = quantize_weight_per_channel(wb)
    qo2, so2 = oracle.quantize_per_channel(wb.float().cpu().numpy())
    np.testing.assert_array_equal(q2.cpu().numpy(), qo2)
    np.testing.assert_array_equal(s2.cpu().numpy(), so2)


def test_per_tensor_quantiser_matches_oracle(dev):
    from kappa_amd.qwen3 import quantize_weight

    rng = np.random.default_rng(15)
    w = (rng.standard_normal((4, 256, 48)) * 0.02).astype(np.float32)
    q, s = quantize_weight(torch.from_numpy(w).to(dev), scale_dtype=torch.float32)
    qo, so = oracle.quantize_per_tensor(w)
    np.testing.assert_array_equal(q.cpu().numpy(), qo)
    assert float(s) == float(so)


def test_to_compute_dtype_matches_reference_rule(dev):
    from kappa_amd.qwen3 import Q8Weight, to_compute_dtype

    rng = np.random.default_rng(13)
    q = rng.integers(-128, 128, (4, 64, 48)).astype(np.int8)
    s = (rng.random((4, 1, 48)) * 0.01).astype(np.float32)
    w = Q8Weight(torch.from_numpy(q).to(dev), torch.from_numpy(s).to(dev))
    bf = to_compute_dtype(w, torch.bfloat16).float().cpu().numpy()
    ref = oracle.bf16_round(q.astype(np.float32) * oracle.bf16_round(s))
    np.testing.assert_array_equal(bf, ref)
    f32 = to_compute_dtype(w, torch.float32).cpu().numpy()
    np.testing.assert_array_equal(f32, q.astype(np.float32) * s)
    wt = Q8Weight(torch.from_numpy(q).to(dev), torch.tensor(0.0123, dtype=torch.bfloat16, device=dev))
    st = np.float32(torch.tensor(0.0123, dtype=torch.bfloat16).float().item())
    np.testing.assert_array_equal(
        to_compute_dtype(wt, torch.bfloat16).float().cpu().numpy(), oracle.bf16_round(q.astype(np.float32) * st)
    )


def test_prepack_layout(dev):
    from kappa_amd import _lib
    from kappa_amd.qwen3 import Q8Weight, prepack_moe_experts

    rng = np.random.default_rng(14)
    E, D, I = 3, 128, 64
    qs = [rng.integers(-128, 128, shp).astype(np.int8) for shp in ((E, D, I), (E, D, I), (E, I, D))]
    ss = [(rng.random((E, 1, n)) * 0.01).astype(np.float32) for n in (I, I, D)]
    ws = [Q8Weight(torch.from_numpy(q).to(dev), torch.from_numpy(s).to(dev)) for q, s in zip(qs, ss)]
    p = prepack_moe_experts(*ws)
    assert (p.num_experts, p.hidden, p.intermediate, p.source_scale_kind) == (E, D, I, _lib.SCALE_CHANNEL)
    w13 = p.w13.cpu().numpy().reshape(E, I // 16, 2, D // 16, 16, 16)
    # cell [e, ig, which, kg, col, kk] = src[e, kg*16+kk, ig*16+col]
    for which in (0, 1):
        src = qs[which].reshape(E, D // 16, 16, I // 16, 16)  # e, kg, kk, ig, col
        np.testing.assert_array_equal(w13[:, :, which], src.transpose(0, 3, 1, 4, 2))
    w2 = p.w2.cpu().numpy().reshape(E, D // 16, I // 16, 16, 16)
    src = qs[2].reshape(E, I // 16, 16, D // 16, 16)  # e, kg, kk, dg, col
    np.testing.assert_array_equal(w2, src.transpose(0, 3, 1, 4, 2))
    # the scales as given (f32): the kernels round them to bf16 only for the
    # gather and fixed_capacity programs
    s13 = p.s13.cpu().numpy().reshape(E, I // 16, 2, 16)
    for which in (0, 1):
        np.testing.assert_array_equal(s13[:, :, which], ss[which].reshape(E, I // 16, 16))
    np.testing.assert_array_equal(p.s2.cpu().numpy().reshape(E, D), ss[2].reshape(E, D))
    pt = prepack_moe_experts(*[Q8Weight(w.values, torch.tensor(0.01, device=dev)) for w in ws])
    assert pt.source_scale_kind == _lib.SCALE_TENSOR


# --- fixed_capacity (token dropping, kappa/qwen3/ffn_moe.py:107-158) ----------


@pytest.mark.parametrize("kernels", ["auto", "grouped"])
@pytest.mark.parametrize("case", CAPACITY_SPECS, ids=[c[0].name for c in CAPACITY_SPECS])
def test_fixed_capacity_golden(dev, case, kernels):
    """moe_swiglu_ffn with moe_impl='fixed_capacity' against the oracle and the
    golden restatement: the same slot limit, the same dropped assignments, the
    bf16 expert chain and the bf16 scatter-add combine."""
    import dataclasses

    from kappa_amd import _lib
    from kappa_amd.qwen3 import moe_layer_config, moe_stages
    from kappa_amd.qwen3.ffn_moe import _fixed_capacity, _moe_forward

    spec, cf, slots = case
    inp = make_inputs(spec)
    bf16 = spec.act == "bf16"
    x, r, (g, u, d) = spec_to_dev(spec, inp, dev)
    cfg = moe_layer_config(hidden=spec.D, experts=spec.E, top_k=spec.K, intermediate=spec.I,
                           moe_impl="fixed_capacity", moe_capacity_factor=cf)  # fmt: skip
    if slots is not None:
        cfg = dataclasses.replace(cfg, moe_fixed_capacity_slots=slots)
    cap = _fixed_capacity(cfg, spec.T)
    gold = np.load(f"tests/golden/{spec.name}.npz")
    assert cap == int(gold["capacity"]) == oracle.capacity_slots(spec.T, spec.K, spec.E, cf, slots)
    ref = oracle.forward(inp["x"], inp["router"], inp["gate"], inp["up"], inp["down"], k=spec.K,
                         act_bf16=bf16, impl="fixed_capacity", capacity=cap)  # fmt: skip
    # dispatch stage: inv carries -1 exactly for the dropped assignments
    rt = moe_stages.route(x, r, num_experts=spec.E, k=spec.K)
    dp = moe_stages.dispatch(rt["idx"], rt["hist"], num_experts=spec.E, capacity=cap)
    np.testing.assert_array_equal(dp["inv"].cpu().numpy(), ref["inv"])
    np.testing.assert_array_equal(dp["inv"].cpu().numpy(), gold["inv_cap"])
    fam = _lib.KERNELS_AUTO if kernels == "auto" else _lib.KERNELS_GROUPED
    out = _moe_forward(
        x.reshape(1, spec.T, spec.D), r, g, u, d, num_experts=spec.E, num_experts_per_tok=spec.K,
        impl="fixed_capacity", decode_threshold=64, packed=None, capacity=cap, kernels=fam,
    ).reshape(spec.T, spec.D)  # fmt: skip
    check_out(out.float().cpu().numpy(), ref["out"], bf16)
    check_out(out.float().cpu().numpy(), gold["out"], bf16, "vs golden")


@pytest.mark.parametrize("T,cf", [(64, 1.0), (4096, 1.0), (4096, 0.5)])
def test_30b_fixed_capacity(dev, l30, T, cf):
    """30B-A3B W8 layer with token dropping at decode and prefill sizes (sampled
    tokens against the oracle); every token's kept experts match the slot rule."""
    from kappa_amd.qwen3 import moe_stages, moe_swiglu_ffn
    from kappa_amd.qwen3.ffn_moe import _fixed_capacity

    cfg = layer_cfg(l30, "fixed_capacity", moe_capacity_factor=cf)
    cap = _fixed_capacity(cfg, T)
    x = make_x(T, l30.D, seed=700 + T)
    r, d = _route_and_dispatch(x, l30.router, l30.E, l30.K)
    xn, idx, w, od = _check_routing(x, l30.router, l30.E, l30.K, r, d)
    inv_cap = oracle.drop_over_capacity(idx, od, cap)
    dc = moe_stages.dispatch(r["idx"], r["hist"], num_experts=l30.E, capacity=cap)
    np.testing.assert_array_equal(dc["inv"].cpu().numpy(), inv_cap)
    assert np.any(inv_cap < 0)
    out = moe_swiglu_ffn(x.reshape(1, T, l30.D), l30.router, l30.gate, l30.up, l30.down, cfg=cfg)
    rng = np.random.default_rng(T)
    toks = np.unique(np.concatenate([rng.choice(T, size=min(32, T), replace=False), [0, T - 1]]))
    rows_t = np.repeat(toks, l30.K)
    rows_e = idx[toks].reshape(-1)
    _, yo = oracle_rows(oracle, xn, rows_t, rows_e, l30.host(), impl="fixed_capacity")
    kept = inv_cap.reshape(T, l30.K)[toks].reshape(-1)
    ref = oracle.combine(yo, np.where(kept >= 0, np.arange(len(rows_t)), -1).astype(np.int32), w[toks], True,
                         impl="fixed_capacity")  # fmt: skip
    check_out(bf16_np(out.reshape(T, l30.D))[toks], ref, True, "out rows")


# --- the two-phase router (MFMA logits, canonical recompute of the candidates) --


def _route_two_phase_check(x, router, E, K):
    """The two-phase router (kmoe_route with its scratch and no logits) against the
    oracle: indices bit-exact; weights and per-64-token histograms bit-identical to
    the all-VALU form (same canonical logits, same expf)."""
    from kappa_amd.qwen3 import moe_stages

    r2 = moe_stages.route(x, router, num_experts=E, k=K, logits=False)
    r1 = moe_stages.route(x, router, num_experts=E, k=K)
    assert "logits" not in r2
    lg = oracle.router_logits(bf16_np(x), router.float().cpu().numpy())
    np.testing.assert_array_equal(r1["logits"].cpu().numpy(), lg)
    idx, _ = oracle.topk_softmax(lg, K, act_bf16=True)
    np.testing.assert_array_equal(r2["idx"].cpu().numpy(), idx)
    np.testing.assert_array_equal(r2["idx"].cpu().numpy(), r1["idx"].cpu().numpy())
    np.testing.assert_array_equal(r2["w"].cpu().numpy(), r1["w"].cpu().numpy())
    np.testing.assert_array_equal(r2["hist"].cpu().numpy(), r1["hist"].cpu().numpy())
    return lg, idx


@pytest.mark.parametrize("T", [241, 512, 1000, 4096])
def test_two_phase_router_30b(dev, l30, T):
    """The prefill sizes of the 30B-A3B layer, uniform and Zipf-skewed routing."""
    x = make_x(T, l30.D, seed=1200 + T)
    _route_two_phase_check(x, l30.router, l30.E, l30.K)
    x[:, 0] = 1.0
    _route_two_phase_check(x, skew_router(l30.router, lam=1.5), l30.E, l30.K)


@pytest.mark.parametrize(
    "D,E,K,T",
    [(4096, 128, 8, 300), (4096, 128, 8, 2048), (1024, 64, 4, 333), (512, 256, 8, 700), (2048, 48, 6, 500),
     (1024, 16, 2, 400), (512, 240, 8, 333)],
)  # fmt: skip
def test_two_phase_router_shapes(dev, D, E, K, T):
    """The 235B-A22B router (64 slices per candidate) and other slice counts and
    expert counts (the kernel's template forms), including expert counts whose
    16-expert tiles do not divide the block's waves (48: five reduction splits
    of three tiles, one wave idle in phase 1; 240: fifteen tiles, one wave
    idle) and a single tile (16 experts, sixteen reduction splits)."""
    g = torch.Generator(device="cuda").manual_seed(D + E + T)
    router = (torch.randn(D, E, generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    x = make_x(T, D, seed=1300 + T)
    _route_two_phase_check(x, router, E, K)


def test_two_phase_router_ties_near_ties_and_fallback(dev):
    """Exact ties straddling the K-th place on every token (experts in groups of three
    identical router columns: the top K = 8 ends inside a group), near ties (copies
    that differ in one entry by one bf16 ulp), an all-zero row (all logits 0: the
    first K experts, weights 1/K) and rows whose norm overflows f32 (the token takes
    every expert as a candidate); the oracle's tie rule is the lower index first."""
    D, E, K, T = 2048, 128, 8, 600
    g = torch.Generator(device="cuda").manual_seed(77)
    base = (torch.randn(D, 43, generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    router = base[:, torch.arange(E, device="cuda") % 43].contiguous()
    x = make_x(T, D, seed=1400)
    _route_two_phase_check(x, router, E, K)
    near = router.clone()
    for e in range(43, E):  # each copy one ulp away from its source in one entry
        dd = (e * 37) % D
        bits = near[dd, e].view(torch.int16)
        near[dd, e] = (bits + 1).view(torch.bfloat16)
    x[0] = 0.0
    x[1] = x[1] * 2.0**100  # ||x||^2 overflows f32; the logits stay finite
    x[2, ::3] = 0.0
    lg, idx = _route_two_phase_check(x, near, E, K)
    np.testing.assert_array_equal(idx[0], np.arange(K))
    assert np.isfinite(lg[1]).all()


@pytest.mark.parametrize("T", [512, 2048, 2049, 3001, 4096])
def test_forward_routing_two_phase(dev, l30, T):
    """kmoe_forward from 2048 tokens routes with the two-phase form (below, the
    all-VALU router): its indices and weights equal the stage router's, also
    where its last block holds fewer than 16 tokens (T = 2049, 3001)."""
    from kappa_amd.qwen3 import moe_stages
    from kappa_amd.qwen3.ffn_moe import _moe_forward

    x = make_x(T, l30.D, seed=1500 + T)
    _, idx, w = _moe_forward(
        x.reshape(1, T, l30.D), l30.router, l30.gate, l30.up, l30.down, num_experts=l30.E,
        num_experts_per_tok=l30.K, packed=None, return_routing=True, **forward_args("ragged"),
    )  # fmt: skip
    r = moe_stages.route(x, l30.router, num_experts=l30.E, k=l30.K)
    lg = oracle.router_logits(bf16_np(x), l30.router.float().cpu().numpy())
    oidx, _ = oracle.topk_softmax(lg, l30.K, act_bf16=True)
    np.testing.assert_array_equal(idx.cpu().numpy(), oidx)
    assert torch.equal(w.float(), r["w"])
