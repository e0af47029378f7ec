"""The Python boundary mirrors the reference's errors (CPU; no compute)."""

import dataclasses

import pytest
import torch

from kappa_amd.qwen3 import Q8Weight, moe_layer_config, moe_swiglu_ffn, qwen3_config_for_preset
from kappa_amd.qwen3.ffn_moe import _effective_moe_impl


def cfg(**kw):
    return moe_layer_config(hidden=16, experts=8, top_k=2, intermediate=32, **kw)


def args(d=16, e=8, i=32):
    x = torch.zeros(2, 3, d)
    return x, torch.zeros(d, e), torch.zeros(e, d, i), torch.zeros(e, d, i), torch.zeros(e, i, d)


def test_requires_use_moe():
    with pytest.raises(ValueError, match="moe_swiglu_ffn requires cfg.use_moe"):
        moe_swiglu_ffn(*args(), cfg=cfg(use_moe=False))


def test_router_shape_message_matches_reference():
    x, r, g, u, d = args()
    with pytest.raises(ValueError, match=r"router_w shape \(16, 4\) != \(16, 8\)"):
        moe_swiglu_ffn(x, torch.zeros(16, 4), g, u, d, cfg=cfg())
    q = Q8Weight(torch.zeros(8, 16, dtype=torch.int8), torch.tensor(1.0))
    with pytest.raises(ValueError, match=r"router_w shape \(8, 16\) != \(16, 8\)"):
        moe_swiglu_ffn(x, q, g, u, d, cfg=cfg())


def test_unknown_impl_and_capacity_errors():
    with pytest.raises(ValueError, match="unknown moe_impl: 'bogus'"):
        moe_swiglu_ffn(*args(), cfg=cfg(moe_impl="bogus"))
    with pytest.raises(ValueError, match="fixed_capacity requires cfg.moe_capacity_factor > 0"):
        moe_swiglu_ffn(*args(), cfg=cfg(moe_impl="fixed_capacity", moe_capacity_factor=0.0))


def test_cpu_tensors_are_rejected_not_computed():
    with pytest.raises(ValueError, match="HIP device"):
        moe_swiglu_ffn(*args(), cfg=cfg())


def test_effective_impl_mirrors_reference_threshold():
    c = cfg(moe_impl="ragged_jax")
    assert _effective_moe_impl(c, total_tokens=64) == "gather_einsum"
    assert _effective_moe_impl(c, total_tokens=65) == "ragged_jax"
    assert _effective_moe_impl(cfg(), total_tokens=4096) == "gather_einsum"
    c0 = dataclasses.replace(c, moe_ragged_decode_token_threshold=0)
    assert _effective_moe_impl(c0, total_tokens=1) == "ragged_jax"


def test_presets_match_reference_values():
    c = qwen3_config_for_preset("qwen3-30b-a3b")
    assert (c.model_dim, c.num_experts, c.num_experts_per_tok, c.intermediate_size) == (2048, 128, 8, 768)
    assert c.moe_impl == "gather_einsum" and c.moe_ragged_decode_token_threshold == 64
    with pytest.raises(ValueError, match="unknown preset"):
        qwen3_config_for_preset("nope")


def test_fixed_capacity_slots_follow_reference_formula():
    """c_buf (kappa/qwen3/ffn_moe.py:23-31) and c_dyn (:136-139), including the
    float32 round-half-even of c_dyn and the floor of one slot."""
    from kappa_amd.qwen3.ffn_moe import _fixed_capacity, _fixed_capacity_buffer_slots

    c30 = moe_layer_config(hidden=2048, experts=128, top_k=8, intermediate=768, moe_impl="fixed_capacity")
    assert _fixed_capacity_buffer_slots(c30) == 640  # ceil(1.25 * 8192 * 8 / 128)
    assert _fixed_capacity(c30, 4096) == 320  # 1.25 * 32768 / 128
    assert _fixed_capacity(c30, 64) == 5
    assert _fixed_capacity(c30, 1) == 1  # round(0.078125) = 0 -> floor of one slot
    # c_dyn capped by the static buffer
    assert _fixed_capacity(c30, 8192 * 4) == 640
    # explicit slots override the derived buffer depth
    c_fix = dataclasses.replace(c30, moe_fixed_capacity_slots=3)
    assert _fixed_capacity_buffer_slots(c_fix) == 3 and _fixed_capacity(c_fix, 4096) == 3
    # half-even: cf * T*K / E = 2.5 -> 2, 3.5 -> 4
    c_he = moe_layer_config(hidden=16, experts=8, top_k=2, intermediate=32, moe_capacity_factor=1.25)
    assert _fixed_capacity(c_he, 8) == 2  # 1.25 * 16 / 8 = 2.5
    assert _fixed_capacity(c_he, 11) == 3  # 1.25 * 22 / 8 = 3.4375
    c_he2 = dataclasses.replace(c_he, moe_capacity_factor=1.75)
    assert _fixed_capacity(c_he2, 8) == 4  # 1.75 * 16 / 8 = 3.5


def test_block_api_mirrors_the_moe_errors_and_rejects_cpu_tensors():
    from kappa_amd.qwen3 import moe_block_ffn, rms_norm

    x, r, g, u, d = args()
    scale = torch.ones(16)
    with pytest.raises(ValueError, match="moe_swiglu_ffn requires cfg.use_moe"):
        moe_block_ffn(x, scale, r, g, u, d, cfg=cfg(use_moe=False))
    with pytest.raises(ValueError, match="unknown moe_impl"):
        moe_block_ffn(x, scale, r, g, u, d, cfg=cfg(moe_impl="bogus", moe_ragged_decode_token_threshold=0))
    with pytest.raises(ValueError, match=r"router_w shape \(16, 4\) != \(16, 8\)"):
        moe_block_ffn(x, scale, torch.zeros(16, 4), g, u, d, cfg=cfg())
    with pytest.raises(ValueError, match="HIP device"):
        moe_block_ffn(x, scale, r, g, u, d, cfg=cfg())
    with pytest.raises(ValueError, match="HIP device"):
        rms_norm(x, scale)
    with pytest.raises(ValueError, match="out_dtype"):
        rms_norm(x, scale, out_dtype=torch.float16)


def test_gather_program_rejects_per_channel_scales():
    """moe_take_dequant (kappa/qwen3/quant.py:71-74) multiplies the gathered values by
    the scale as stored; [E, 1, N] scales do not broadcast there, so per-channel W8 runs
    on the ragged path (threshold 0 for decode batches) or fixed_capacity."""
    x, r, g, u, d = args()
    qc = [Q8Weight(torch.zeros(8, 16, 32, dtype=torch.int8), torch.ones(8, 1, 32)) for _ in range(2)]
    qd = Q8Weight(torch.zeros(8, 32, 16, dtype=torch.int8), torch.ones(8, 1, 16))
    with pytest.raises(ValueError, match="gather_einsum takes one scale per tensor"):
        moe_swiglu_ffn(x, r, *qc, qd, cfg=cfg())
    # ragged_jax at T <= threshold runs the gather program too (kappa/qwen3/ffn_moe.py:219-223)
    with pytest.raises(ValueError, match="gather_einsum takes one scale per tensor"):
        moe_swiglu_ffn(x, r, *qc, qd, cfg=cfg(moe_impl="ragged_jax"))
    # the ragged program (above the threshold) and fixed_capacity accept them: the call
    # gets as far as the device check
    for c in (cfg(moe_impl="ragged_jax", moe_ragged_decode_token_threshold=0), cfg(moe_impl="fixed_capacity")):
        with pytest.raises(ValueError, match="HIP device"):
            moe_swiglu_ffn(x, r, *qc, qd, cfg=c)
    # one scale per tensor is the gather path's own format
    qt = [Q8Weight(w.values, torch.tensor(0.5)) for w in (*qc, qd)]
    with pytest.raises(ValueError, match="HIP device"):
        moe_swiglu_ffn(x, r, *qt, cfg=cfg())


def test_packed_argument_must_match_the_layer():
    from kappa_amd import _lib
    from kappa_amd.qwen3 import PackedExperts

    x, r, g, u, d = args()
    t = torch.zeros(1)
    c = cfg(moe_impl="ragged_jax", moe_ragged_decode_token_threshold=0)
    for E, D, I in ((16, 16, 32), (8, 32, 32), (8, 16, 64)):
        p = PackedExperts(t, t, t, t, D, I, E, _lib.SCALE_CHANNEL)
        with pytest.raises(ValueError, match="packed experts hold"):
            moe_swiglu_ffn(x, r, g, u, d, cfg=c, packed=p)
    with pytest.raises(ValueError, match="PackedExperts"):
        moe_swiglu_ffn(x, r, g, u, d, cfg=c, packed=(t, t, t, t))


def test_packed_experts_without_their_sources():
    """After a load-time prepack the int8 sources may be freed: the expert weights are
    then None, all three, with packed= (which then carries E, D, I and the scale kind)."""
    from kappa_amd import _lib
    from kappa_amd.qwen3 import PackedExperts

    x, r, g, u, d = args()
    t = torch.zeros(1)
    c = cfg(moe_impl="ragged_jax", moe_ragged_decode_token_threshold=0)
    p = PackedExperts(t, t, t, t, 16, 32, 8, _lib.SCALE_CHANNEL)
    with pytest.raises(ValueError, match="None only all together"):
        moe_swiglu_ffn(x, r, None, None, None, cfg=c)
    with pytest.raises(ValueError, match="None only all together"):
        moe_swiglu_ffn(x, r, None, u, d, cfg=c, packed=p)
    with pytest.raises(ValueError, match="PackedExperts"):
        moe_swiglu_ffn(x, r, None, None, None, cfg=c, packed=(t, t, t, t))
    # the gather program still refuses per-channel scales, now by the packed copy's record
    with pytest.raises(ValueError, match="gather_einsum takes one scale per tensor"):
        moe_swiglu_ffn(x, r, None, None, None, cfg=cfg(), packed=p)
    with pytest.raises(ValueError, match="packed experts hold"):
        moe_swiglu_ffn(x, r, None, None, None, cfg=c, packed=PackedExperts(t, t, t, t, 32, 32, 8, _lib.SCALE_CHANNEL))


class _FakePack:
    """Stands in for PackedExperts: a device (the CPU here) and a size."""

    nbytes = 1000

    def __init__(self):
        self.w13 = torch.empty(0)


@pytest.fixture
def pack_cache(monkeypatch):
    """A fresh pack cache whose prepack step is a stand-in (no device needed)."""
    from kappa_amd.qwen3 import ffn_moe

    monkeypatch.setattr(ffn_moe, "prepack_moe_experts", lambda g, u, d: _FakePack())
    return ffn_moe._PackCache(max_bytes=1 << 40)


def _layer(seed):
    gen = torch.Generator().manual_seed(seed)

    def q(*shape):
        return Q8Weight(torch.randint(-128, 127, shape, generator=gen, dtype=torch.int8), torch.rand(shape[0], 1,
                                                                                                      shape[2]))

    return q(4, 16, 8), q(4, 16, 8), q(4, 8, 16)


def test_pack_cache_holds_a_whole_model_and_does_not_repack(pack_cache):
    layers = [_layer(s) for s in range(48)]
    first = [pack_cache.get(*lw) for lw in layers]
    assert pack_cache.packs == 48 and len(pack_cache) == 48
    second = [pack_cache.get(*lw) for lw in layers]
    assert pack_cache.packs == 48
    assert all(a is b for a, b in zip(first, second))


def test_pack_cache_entry_dies_with_its_weights(pack_cache):
    import gc

    lw = _layer(0)
    p0 = pack_cache.get(*lw)
    assert len(pack_cache) == 1
    del lw
    gc.collect()
    assert len(pack_cache) == 0, "a freed source must drop its entry"
    # a new layer, even one that reuses the freed memory, misses and is packed anew
    lw2 = _layer(1)
    p1 = pack_cache.get(*lw2)
    assert p1 is not p0 and pack_cache.packs == 2


def test_pack_cache_misses_after_an_in_place_write(pack_cache):
    lw = _layer(2)
    p0 = pack_cache.get(*lw)
    lw[1].values.add_(1)  # bumps the tensor's version
    p1 = pack_cache.get(*lw)
    assert p1 is not p0 and pack_cache.packs == 2
    assert pack_cache.get(*lw) is p1


def test_pack_cache_keys_on_identity_not_address(pack_cache):
    # two layers whose tensors share storage (views of one buffer) are still two entries
    base = _layer(3)
    alias = tuple(Q8Weight(w.values.view(w.values.shape), w.scale.view(w.scale.shape)) for w in base)
    assert all(a.values.data_ptr() == b.values.data_ptr() for a, b in zip(alias, base))
    pa = pack_cache.get(*base)
    pb = pack_cache.get(*alias)
    assert pa is not pb and pack_cache.packs == 2


def test_pack_cache_is_bounded_by_bytes_and_warns_once(pack_cache):
    """The implicit cache doubles a layer's expert memory; past its byte budget it
    evicts the least recently used layers (they are packed again on their next call)
    and warns once that large models should prepack at load time."""
    import warnings

    pack_cache.max_bytes = 10 * _FakePack.nbytes
    layers = [_layer(s) for s in range(16)]
    with warnings.catch_warnings(record=True) as caught:
        warnings.simplefilter("always")
        for lw in layers:
            pack_cache.get(*lw)
    assert len(pack_cache) == 10 and pack_cache.evicted_for_room == 6
    assert sum(issubclass(c.category, ResourceWarning) for c in caught) == 1
    assert "prepack_moe_experts" in str(caught[0].message)
    # the newest ten stay; the oldest is packed again
    before = pack_cache.packs
    pack_cache.get(*layers[-1])
    assert pack_cache.packs == before
    pack_cache.get(*layers[0])
    assert pack_cache.packs == before + 1 and len(pack_cache) == 10
