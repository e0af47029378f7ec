"""Pin the oracle with closed forms, special cases and invariants (CPU).

Each check is chosen so that a plausible mistake in the oracle (a dropped
term, a transposed operand, a wrong tie rule or rounding point) fails it.
"""

import numpy as np
import pytest
import torch

import oracle
from inputs import Spec, bf16_rne, make_inputs, quantize_per_channel_np


def torch_bf16(a):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(torch.bfloat16).float().numpy()


# --- bf16 rounding -----------------------------------------------------------


def test_bf16_round_matches_torch_including_ties():
    rng = np.random.default_rng(0)
    a = rng.standard_normal(100_000).astype(np.float32) * np.float32(10.0) ** rng.integers(-8, 8, 100_000)
    # exact ties: low 16 bits = 0x8000 with both parities of bit 16
    ties = (rng.integers(0, 2**15, 2000, dtype=np.uint32) << 17 | 0x8000).view(np.float32)
    ties2 = ((rng.integers(0, 2**15, 2000, dtype=np.uint32) << 17) | 0x18000).view(np.float32)
    special = np.array([0.0, -0.0, 1.0, -1.0, 3.3895314e38, 1e-40, -1e-40], np.float32)
    for arr in (a, ties, ties2, special):
        arr = arr[np.isfinite(arr)]  # NaN payloads are not part of the contract
        np.testing.assert_array_equal(oracle.bf16_round(arr).view(np.uint32), torch_bf16(arr).view(np.uint32))
        np.testing.assert_array_equal(bf16_rne(arr).view(np.uint32), torch_bf16(arr).view(np.uint32))


# --- router logits (N0) --------------------------------------------------------


def test_logits_exact_on_exactly_representable_sums():
    # small integers times powers of two: every partial sum is exact in fp32, so any
    # summation order must return the exact dot product
    rng = np.random.default_rng(1)
    T, D, E = 5, 300, 12
    x = rng.integers(-8, 9, (T, D)).astype(np.float32) * np.float32(0.5)
    r = rng.integers(-8, 9, (D, E)).astype(np.float32) * np.float32(0.25)
    exact = x.astype(np.float64) @ r.astype(np.float64)
    np.testing.assert_array_equal(oracle.router_logits(x, r), exact.astype(np.float32))


def test_logits_error_bound_and_not_transposed():
    rng = np.random.default_rng(2)
    T, D, E = 7, 2048, 16
    x = bf16_rne(rng.standard_normal((T, D)).astype(np.float32))
    r = bf16_rne((rng.standard_normal((D, E)) * 0.02).astype(np.float32))
    lg = oracle.router_logits(x, r)
    ref = x.astype(np.float64) @ r.astype(np.float64)
    bound = 2 * D * np.finfo(np.float32).eps * (np.abs(x).astype(np.float64) @ np.abs(r).astype(np.float64))
    assert np.all(np.abs(lg - ref) <= bound)
    # the canonical order is not the plain sequential one: the slice tree must change
    # some low bits relative to a single fmaf chain (otherwise the slicing is not applied)
    seq = np.zeros((T, E), np.float32)
    for d in range(D):
        seq = (seq.astype(np.float64) + x[:, d : d + 1].astype(np.float64) * r[d].astype(np.float64)).astype(np.float32)
    assert np.any(seq != lg)


def test_logits_slice_tree_order_small():
    # D = 130 -> slices [0,64), [64,128), [128,130); tree ((p0 + p1) + (p2 + 0))
    rng = np.random.default_rng(3)
    x = rng.standard_normal((1, 130)).astype(np.float32)
    r = rng.standard_normal((130, 1)).astype(np.float32)
    p = []
    for s0 in (0, 64, 128):
        acc = np.float32(0.0)
        for d in range(s0, min(130, s0 + 64)):
            acc = np.float32(np.float64(x[0, d]) * np.float64(r[d, 0]) + np.float64(acc))
        p.append(acc)
    expect = np.float32(np.float32(p[0] + p[1]) + np.float32(p[2] + np.float32(0.0)))
    # products of random fp32 are not exact; a float64 fma emulation is exact for one
    # product plus one addend when the result is rounded once to fp32 - it is here
    assert oracle.router_logits(x, r)[0, 0] == expect


def test_quantized_router_logits_use_f32_dequant():
    rng = np.random.default_rng(4)
    x = bf16_rne(rng.standard_normal((3, 128)).astype(np.float32))
    rq = rng.integers(-128, 128, (128, 8)).astype(np.int8)
    s = np.float32(0.0123)
    a = oracle.router_logits(x, (rq, s))
    b = oracle.router_logits(x, (rq.astype(np.float32) * s).astype(np.float32))
    np.testing.assert_array_equal(a, b)


# --- top-k and softmax (N1, N2) ------------------------------------------------


def test_topk_matches_stable_descending_sort():
    rng = np.random.default_rng(5)
    T, E, K = 200, 64, 8
    lg = rng.integers(-20, 20, (T, E)).astype(np.float32) * np.float32(0.125)  # many exact ties
    idx, w = oracle.topk_softmax(lg, K, act_bf16=False)
    order = np.lexsort((np.broadcast_to(np.arange(E), (T, E)), -lg), axis=-1)[:, :K]
    np.testing.assert_array_equal(idx, order)
    top = np.take_along_axis(lg, order, axis=-1).astype(np.float64)
    ex = np.exp(top - top[:, :1])
    ref = ex / ex.sum(-1, keepdims=True)
    assert np.all(np.abs(w - ref) <= 4 * np.finfo(np.float32).eps * ref)
    assert np.all(np.abs(w.sum(-1) - 1) <= K * np.finfo(np.float32).eps)
    assert np.all(np.diff(w, axis=-1) <= 0)  # non-increasing in j


def test_topk_weights_are_renormalised_full_softmax():
    # softmax over the top-k equals the full softmax restricted to the top-k and renormalised
    rng = np.random.default_rng(6)
    lg = rng.standard_normal((50, 32)).astype(np.float32)
    idx, w = oracle.topk_softmax(lg, 4, act_bf16=False)
    full = np.exp(lg.astype(np.float64) - lg.max(-1, keepdims=True))
    full /= full.sum(-1, keepdims=True)
    sel = np.take_along_axis(full, idx.astype(np.int64), axis=-1)
    np.testing.assert_allclose(w, sel / sel.sum(-1, keepdims=True), rtol=1e-6)


def test_topk_bf16_weights_are_rounded():
    rng = np.random.default_rng(7)
    lg = rng.standard_normal((40, 16)).astype(np.float32)
    _, w32 = oracle.topk_softmax(lg, 3, act_bf16=False)
    _, w16 = oracle.topk_softmax(lg, 3, act_bf16=True)
    np.testing.assert_array_equal(w16, torch_bf16(w32))


def test_topk_k_equals_e_is_a_permutation():
    rng = np.random.default_rng(8)
    lg = rng.standard_normal((10, 8)).astype(np.float32)
    idx, w = oracle.topk_softmax(lg, 8, act_bf16=False)
    np.testing.assert_array_equal(np.sort(idx, -1), np.tile(np.arange(8), (10, 1)))


# --- dispatch (N3) -------------------------------------------------------------


@pytest.mark.parametrize("T,E,K", [(1, 8, 2), (37, 16, 4), (300, 128, 8), (64, 4, 4)])
def test_dispatch_is_stable_argsort(T, E, K):
    rng = np.random.default_rng(T * E + K)
    idx = np.stack([rng.permutation(E)[:K] for _ in range(T)]).astype(np.int32)
    d = oracle.dispatch(idx, E)
    flat = idx.reshape(-1)
    order = np.argsort(flat, kind="stable")
    np.testing.assert_array_equal(d["order"], order)
    np.testing.assert_array_equal(d["group_sizes"], np.bincount(flat, minlength=E))
    np.testing.assert_array_equal(d["offsets"], np.concatenate([[0], np.cumsum(np.bincount(flat, minlength=E))]))
    np.testing.assert_array_equal(d["order"][d["inv"]], np.arange(T * K))
    np.testing.assert_array_equal(d["sorted_token"], order // K)
    for e in range(E):  # ascending tokens within every expert
        seg = d["sorted_token"][d["offsets"][e] : d["offsets"][e + 1]]
        assert np.all(np.diff(seg) > 0)


# --- expert FFN special cases (N4, N5) -----------------------------------------


def _dense_swiglu64(x, wg, wu, wd, bf16):
    """kappa/qwen3/ffn.py:12-22 in float64 with rounding to the activation dtype."""
    rnd = torch_bf16 if bf16 else (lambda a: np.asarray(a, np.float32))
    g = rnd(x.astype(np.float64) @ wg.astype(np.float64))
    u = rnd(x.astype(np.float64) @ wu.astype(np.float64))
    h = rnd(g / (1 + np.exp(-g.astype(np.float64))) * u)
    return rnd(h.astype(np.float64) @ wd.astype(np.float64))


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("impl", ["gather_einsum", "ragged"])
def test_single_expert_reduces_to_dense_swiglu(bf16, impl):
    # E = 1, K = 1: the weight is exactly 1 and the layer is the dense swiglu_ffn
    # (kappa/qwen3/ffn.py:12-22) with the impl's weight dtype: the gather path casts
    # the weights to x.dtype, the ragged path computes in f32 and rounds only y
    spec = Spec("e1", T=9, D=64, E=1, K=1, I=48, act="bf16" if bf16 else "f32", weights="f32", router="f32")
    inp = make_inputs(spec)
    r = oracle.forward(inp["x"], inp["router"], inp["gate"], inp["up"], inp["down"], k=1, act_bf16=bf16, impl=impl)
    np.testing.assert_array_equal(r["w"], np.ones((9, 1), np.float32))
    act_w = bf16 and impl == "gather_einsum"
    rnd = torch_bf16 if act_w else (lambda a: a)
    ref = _dense_swiglu64(inp["x"], rnd(inp["gate"][0]), rnd(inp["up"][0]), rnd(inp["down"][0]), act_w)
    if bf16:
        ref = torch_bf16(ref)
    tol = 2.0**-7 if bf16 else 1e-5
    assert np.all(np.abs(r["out"] - ref) <= tol * np.abs(ref).max())


def test_identical_experts_give_ffn_times_weight_sum():
    spec = Spec("same", T=12, D=64, E=6, K=3, I=32, act="f32", weights="f32", router="f32")
    inp = make_inputs(spec)
    for n in ("gate", "up", "down"):
        inp[n] = np.repeat(inp[n][:1], 6, axis=0)
    r = oracle.forward(inp["x"], inp["router"], inp["gate"], inp["up"], inp["down"], k=3, act_bf16=False,
                       impl="gather_einsum")  # fmt: skip
    ffn = _dense_swiglu64(inp["x"], inp["gate"][0], inp["up"][0], inp["down"][0], False)
    ref = ffn * r["w"].sum(-1, keepdims=True)
    np.testing.assert_allclose(r["out"], ref, rtol=1e-5, atol=1e-6 * np.abs(ref).max())


def test_k_equals_e_is_a_dense_softmax_mixture():
    spec = Spec("dense", T=5, D=32, E=4, K=4, I=16, act="f32", weights="f32", router="f32", x_std=1.0, r_std=0.5)
    inp = make_inputs(spec)
    r = oracle.forward(inp["x"], inp["router"], inp["gate"], inp["up"], inp["down"], k=4, act_bf16=False, impl="ragged")
    lg = inp["x"].astype(np.float64) @ inp["router"].astype(np.float64)
    p = np.exp(lg - lg.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    ref = sum(
        p[:, e : e + 1] * _dense_swiglu64(inp["x"], inp["gate"][e], inp["up"][e], inp["down"][e], False) for e in range(4)
    )
    np.testing.assert_allclose(r["out"], ref, rtol=1e-5, atol=1e-5 * np.abs(ref).max())


def _sigmoid32(g):
    g = np.asarray(g, np.float32)
    return (np.float32(1.0) / (np.float32(1.0) + np.exp(-g))).astype(np.float32)


def test_dequant_rounds_scale_first_in_bf16():
    # one expert, one row: the gather path uses bf16(q * bf16(s)) (kappa/qwen3/quant.py:74),
    # and h = bf16(bf16(g * bf16(sigmoid(g))) * u) (jax.nn.silu(g) * u in bf16)
    rng = np.random.default_rng(9)
    D, I = 64, 16
    x = bf16_rne(rng.standard_normal((1, D)).astype(np.float32))
    q = rng.integers(-128, 128, (1, D, I)).astype(np.int8)
    s = np.full((1, 1, I), 0.0123456, np.float32)
    off = np.array([0, 1], np.int32)
    st = np.array([0], np.int32)
    down = (q.transpose(0, 2, 1).copy(), s[:, :, :1].repeat(D, 2))
    h, y = oracle.expert_ffn(x, off, st, (q, s), (q, s), down, True, impl="gather_einsum")
    w_deq = torch_bf16(q[0].astype(np.float32) * torch_bf16(s[0]))
    g = torch_bf16(x.astype(np.float64) @ w_deq.astype(np.float64))
    np.testing.assert_array_equal(h, torch_bf16(torch_bf16(g * torch_bf16(_sigmoid32(g))) * g))
    w_plain = q[0].astype(np.float32) * s[0]
    g2 = torch_bf16(x.astype(np.float64) @ w_plain.astype(np.float64))
    assert np.any(g2 != g), "scale rounding must matter for this input"
    # the ragged path dequantises in f32 with the unrounded scale and keeps g, u and h
    # in f32 (kappa/qwen3/ffn_moe.py:202-209); only y is rounded to bf16 (:213)
    hr, yr = oracle.expert_ffn(x, off, st, (q, s), (q, s), down, True, impl="ragged")
    gr = (x.astype(np.float64) @ w_plain.astype(np.float64)).astype(np.float32)
    assert np.all(np.abs(hr - gr * _sigmoid32(gr) * gr) <= 1e-5 * np.abs(hr).max())
    assert np.any(torch_bf16(hr) != hr), "ragged h must not be rounded to bf16"
    yr64 = hr.astype(np.float64) @ (q[0].T.astype(np.float64) * np.float64(s[0, 0, 0]))
    assert np.all(np.abs(yr - torch_bf16(yr64)) <= 2.0**-8 * np.abs(yr64) + 1e-30)


@pytest.mark.parametrize("impl", ["gather_einsum", "ragged", "fixed_capacity"])
def test_combine_rounding_points(impl):
    # y * w rounded to bf16 for every impl; gather sums the products in f32 and rounds
    # once (jnp.sum, kappa/qwen3/ffn_moe.py:103); ragged and fixed_capacity add them into
    # a bf16 buffer, rounding after every add (.at[].add, :157, :215)
    y = np.array([[1.0], [2.0**-8], [2.0**-8]], np.float32)  # three y rows of one column
    inv = np.array([0, 1, 2], np.int32)
    w = np.array([[1.0, 1.0, 1.0]], np.float32)
    out = oracle.combine(y, inv, w, True, impl=impl)
    # 1 + 2^-8 rounds to 1 in bf16 (a tie to even), twice; in f32 the sum is 1 + 2^-7 exactly
    assert out[0, 0] == (np.float32(1.0 + 2.0**-7) if impl == "gather_einsum" else np.float32(1.0))
    # the product is rounded before it is added: (1 + 2^-7)^2 = 1 + 2^-6 + 2^-14 -> 1 + 2^-6;
    # plus 2^-8 that is a tie, which rounds to 1 + 2^-6. With the exact product the sum lies
    # above the tie and rounds up to 1 + 2^-6 + 2^-7.
    y2 = np.array([[1.0 + 2.0**-7], [2.0**-8]], np.float32)
    w2 = np.array([[1.0 + 2.0**-7, 1.0]], np.float32)
    got = oracle.combine(y2, np.array([0, 1], np.int32), w2, True, impl=impl)[0, 0]
    assert got == np.float32(1.0 + 2.0**-6)


def test_per_tensor_equals_per_channel_with_equal_scales():
    spec = Spec("pt", T=16, D=128, E=8, K=2, I=64, weights="w8t", scale_dtype="f32", base_seed=70)
    inp = make_inputs(spec)
    a = oracle.forward(inp["x"], inp["router"], inp["gate"], inp["up"], inp["down"], k=2, act_bf16=True, impl="ragged")
    ag = oracle.forward(inp["x"], inp["router"], inp["gate"], inp["up"], inp["down"], k=2, act_bf16=True,
                        impl="gather_einsum")  # fmt: skip
    chan = {}
    for n, N in (("gate", 64), ("up", 64), ("down", 128)):
        q, s = inp[n]
        chan[n] = (q, np.full((8, 1, N), s, np.float32))
    b = oracle.forward(inp["x"], inp["router"], chan["gate"], chan["up"], chan["down"], k=2, act_bf16=True,
                       impl="ragged")  # fmt: skip
    np.testing.assert_array_equal(a["out"], b["out"])
    bg = oracle.forward(inp["x"], inp["router"], chan["gate"], chan["up"], chan["down"], k=2, act_bf16=True,
                        impl="gather_einsum")  # fmt: skip
    np.testing.assert_array_equal(ag["out"], bg["out"])


# --- quantiser (A7) ------------------------------------------------------------


def test_quantiser_matches_numpy_and_round_trip_bound():
    rng = np.random.default_rng(10)
    w = (rng.standard_normal((4, 96, 40)) * 0.02).astype(np.float32)
    q, s = oracle.quantize_per_channel(w)
    qn, sn = quantize_per_channel_np(w)
    np.testing.assert_array_equal(q, qn)
    np.testing.assert_array_equal(s, sn)
    assert np.all(np.abs(w - q.astype(np.float32) * s) <= s / 2 * (1 + 1e-6))
    assert q.min() >= -127 and q.max() <= 127  # symmetric: amax maps to +-127
    qt, st = oracle.quantize_per_tensor(w)
    assert st == np.float32(np.abs(w).max() / np.float32(127))
    # per-channel on a tensor whose channels share one max-abs equals per-tensor
    w2 = w.copy()
    w2[:, 0, :] = np.abs(w).max()
    qc, sc = oracle.quantize_per_channel(w2)
    qt2, st2 = oracle.quantize_per_tensor(w2)
    assert np.all(sc == st2)
    np.testing.assert_array_equal(qc, qt2)


def test_w8_relative_error_matches_reference_check():
    # scripts/verify_qwen3_quant.py:13-25 asserts relative L2 <= 0.02 for random W8
    rng = np.random.default_rng(11)
    x = rng.standard_normal((10, 64)).astype(np.float32)
    w = rng.standard_normal((4, 64, 16)).astype(np.float32)
    for q, s in (oracle.quantize_per_tensor(w), oracle.quantize_per_channel(w)):
        y0 = np.einsum("td,hdk->thk", x, w)
        y1 = np.einsum("td,hdk->thk", x, q.astype(np.float32) * s)
        assert np.linalg.norm(y0 - y1) / np.linalg.norm(y0) <= 0.02


# --- fixed_capacity (kappa/qwen3/ffn_moe.py:107-158) ---------------------------


def test_capacity_slots_closed_forms():
    """c_dyn = max(1, round_half_even(f32(cf) * f32(T*K) / f32(E))) and
    c_buf = ceil(cf * 8192 * K / E) or the explicit slot count (:23-31, 136-141)."""
    assert oracle.capacity_slots(4096, 8, 128, 1.25) == 320
    assert oracle.capacity_slots(64, 8, 128, 1.25) == 5
    assert oracle.capacity_slots(1, 8, 128, 1.25) == 1  # 0.078125 rounds to 0: floor of one
    assert oracle.capacity_slots(8, 2, 8, 1.25) == 2  # 2.5 -> 2 (half to even)
    assert oracle.capacity_slots(8, 2, 8, 1.75) == 4  # 3.5 -> 4
    assert oracle.capacity_slots(32768, 8, 128, 1.25) == 640  # c_dyn 2560 capped by c_buf 640
    assert oracle.capacity_slots(4096, 8, 128, 1.25, fixed_slots=7) == 7


def _slots_brute(idx):
    """_slot_within_expert by its definition: for each (t, j), the number of
    earlier tokens that also chose that expert (the stable (expert, token) order)."""
    T, K = idx.shape
    slot = np.zeros((T, K), np.int32)
    for t in range(T):
        for j in range(K):
            slot[t, j] = int(np.sum(idx[:t] == idx[t, j]))
    return slot


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_drop_over_capacity_matches_slot_definition(seed):
    rng = np.random.default_rng(300 + seed)
    T, K, E = 37, 3, 7
    idx = np.stack([rng.choice(E, size=K, replace=False) for _ in range(T)]).astype(np.int32)
    disp = oracle.dispatch(idx, E)
    slot = _slots_brute(idx)
    for cap in (1, 2, 5, 100):
        inv = oracle.drop_over_capacity(idx, disp, cap).reshape(T, K)
        np.testing.assert_array_equal(inv < 0, slot >= cap)
        np.testing.assert_array_equal(inv[inv >= 0], disp["inv"].reshape(T, K)[inv >= 0])


def _tiny_block(seed, act_bf16):
    from inputs import Spec, make_inputs

    spec = Spec("cap_tiny", T=20, D=64, E=6, K=2, I=32, base_seed=400 + seed,
                act="bf16" if act_bf16 else "f32", weights="w8c" if act_bf16 else "f32",
                router="bf16" if act_bf16 else "f32")  # fmt: skip
    return spec, make_inputs(spec)


@pytest.mark.parametrize("act_bf16", [True, False])
def test_capacity_at_or_above_largest_group_is_dropless(act_bf16):
    # nothing dropped: _moe_fixed_capacity is then the x.dtype expert chain of the gather
    # path (to_compute_dtype(., x.dtype), :146-152) with the scatter-add combine (:157)
    spec, inp = _tiny_block(0, act_bf16)
    args = (inp["x"], inp["router"], inp["gate"], inp["up"], inp["down"])
    a = oracle.forward(*args, k=spec.K, act_bf16=act_bf16, impl="gather_einsum")
    cap = int(a["group_sizes"].max())
    b = oracle.forward(*args, k=spec.K, act_bf16=act_bf16, impl="fixed_capacity", capacity=cap)
    np.testing.assert_array_equal(b["y_sorted"], a["y_sorted"])
    np.testing.assert_array_equal(b["out"], oracle.combine(a["y_sorted"], a["inv"], a["w"], act_bf16, impl="ragged"))
    assert np.all(b["inv"] >= 0)


def test_dropped_assignments_remove_exactly_their_term():
    """out(capacity) = out(dropless) with each dropped assignment's weighted term
    removed: recomputed here with the dropless rows and a zero weight."""
    spec, inp = _tiny_block(1, False)
    args = (inp["x"], inp["router"], inp["gate"], inp["up"], inp["down"])
    a = oracle.forward(*args, k=spec.K, act_bf16=False, impl="gather_einsum")
    b = oracle.forward(*args, k=spec.K, act_bf16=False, impl="fixed_capacity", capacity=2)
    dropped = (b["inv"] < 0).reshape(spec.T, spec.K)
    assert dropped.any()
    w0 = np.where(dropped, np.float32(0.0), a["w"]).astype(np.float32)
    ref = oracle.combine(a["y_sorted"], a["inv"], w0, False, impl="fixed_capacity")
    np.testing.assert_allclose(b["out"], ref, rtol=0, atol=1e-7)
    # tokens with nothing dropped are bit-identical to the dropless output
    keep_all = ~dropped.any(axis=1)
    np.testing.assert_array_equal(b["out"][keep_all], a["out"][keep_all])


# --- rms_norm and the residual (kappa/qwen3/norms.py:10-16, block.py:196-207) ----


@pytest.mark.parametrize("c", [1.0, -4.0, 0.5])
def test_rms_norm_of_a_constant_row_is_its_sign(c):
    # var = c^2 exactly, r = 1/|c| exactly (powers of two): out = sign(c) * scale
    h = np.full((3, 128), c, np.float32)
    out = oracle.rms_norm(h, np.ones(128, np.float32), 0.0, False)
    np.testing.assert_array_equal(out, np.full_like(h, np.sign(c)))


def test_rms_norm_epsilon_is_added_to_the_mean_square():
    # var = 1 and eps = 1: r = 1 / sqrt(2) (not 1/sqrt(1) + 1, not 1/(1 + 1))
    h = np.ones((1, 64), np.float32)
    out = oracle.rms_norm(h, np.ones(64, np.float32), 1.0, False)
    want = np.float32(1.0) / np.sqrt(np.float32(2.0))
    np.testing.assert_array_equal(out, np.full_like(h, want))


def test_rms_norm_is_invariant_to_power_of_two_scaling_and_scales_per_channel():
    rng = np.random.default_rng(3)
    h = rng.standard_normal((5, 192)).astype(np.float32)
    scale = rng.standard_normal(192).astype(np.float32)
    a = oracle.rms_norm(h, scale, 0.0, False)
    np.testing.assert_array_equal(oracle.rms_norm(h * np.float32(4.0), scale, 0.0, False), a)
    onehot = np.zeros(192, np.float32)
    onehot[17] = 2.0
    b = oracle.rms_norm(h, onehot, 0.0, False)
    np.testing.assert_array_equal(b[:, 17], oracle.rms_norm(h, np.ones(192, np.float32), 0.0, False)[:, 17] * 2)
    assert not np.any(np.delete(b, 17, axis=1))


@pytest.mark.parametrize("D", [16, 100, 2048])
def test_rms_norm_within_float32_rounding_of_float64(D):
    rng = np.random.default_rng(D)
    h = (rng.standard_normal((7, D)) * rng.uniform(0.01, 10.0, (7, 1))).astype(np.float32)
    scale = (1.0 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    out = oracle.rms_norm(h, scale, 1e-6, False)
    hf = h.astype(np.float64)
    ref = hf / np.sqrt(np.mean(hf * hf, axis=1, keepdims=True) + 1e-6) * scale
    assert np.all(np.abs(out - ref) <= 8 * np.finfo(np.float32).eps * np.abs(ref) + 1e-30)


def test_rms_norm_bf16_output_is_rounded():
    rng = np.random.default_rng(4)
    h = oracle.bf16_round(rng.standard_normal((4, 64)).astype(np.float32))
    scale = oracle.bf16_round((1 + 0.1 * rng.standard_normal(64)).astype(np.float32))
    a = oracle.rms_norm(h, scale, 1e-6, True)
    np.testing.assert_array_equal(a, oracle.bf16_round(oracle.rms_norm(h, scale, 1e-6, False)))


@pytest.mark.parametrize("act_bf16", [False, True])
def test_block_with_zero_norm_scale_returns_the_residual(act_bf16):
    # rms_norm(h) * 0 = 0 -> all-equal logits, g = u = 0, h = silu(0) * 0 = 0, y = 0:
    # the block adds exactly zero, so out == h (a residual dropped or added twice fails)
    rng = np.random.default_rng(5)
    T, D, E, K, I = 6, 64, 8, 2, 32
    h = rng.standard_normal((T, D)).astype(np.float32)
    if act_bf16:
        h = oracle.bf16_round(h)
    router = (0.02 * rng.standard_normal((D, E))).astype(np.float32)
    gate, up = (0.02 * rng.standard_normal((2, E, D, I))).astype(np.float32)
    down = (0.02 * rng.standard_normal((E, I, D))).astype(np.float32)
    r = oracle.forward_block(h, np.zeros(D, np.float32), router, gate, up, down, k=K, act_bf16=act_bf16,
                             impl="gather_einsum")  # fmt: skip
    np.testing.assert_array_equal(r["idx"], np.tile(np.arange(K, dtype=np.int32), (T, 1)))
    np.testing.assert_array_equal(r["out"], h)
    # and with nonzero norm but zero down weights the block output is zero too
    r2 = oracle.forward_block(h, np.ones(D, np.float32), router, gate, up, np.zeros_like(down), k=K, act_bf16=act_bf16,
                              impl="ragged")  # fmt: skip
    assert not np.any(r2["moe_out"])
    np.testing.assert_array_equal(r2["out"], h)
