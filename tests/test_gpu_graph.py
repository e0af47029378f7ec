"""The MoE block captured in a HIP graph (GPU).

Serving loops capture a decode step once and replay it; the layer must then
give, on every replay, what the same call gives eagerly. Each case captures
the call after an eager warm-up (which also prepacks the experts), replays it
three times on fresh inputs copied into the captured input, runs the eager
call between the replays and compares bit for bit. The library issues no
memset inside a call, so nothing else enters the graph.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

from moe_cases import layer_cfg, make_layer, make_x

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    return torch.device("cuda:0")


@pytest.fixture(scope="module")
def l30(dev):
    return make_layer("30b", seed=0)


def _capture(fn):
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()  # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = fn()
    return g, out


@pytest.mark.parametrize("impl", ["ragged", "fixed_capacity"])
@pytest.mark.parametrize("T", [1, 8, 64, 300])
def test_graph_replay_matches_eager(dev, l30, T, impl):
    from kappa_amd.qwen3 import moe_swiglu_ffn

    cfg = layer_cfg(l30, impl, **({"moe_capacity_factor": 0.5} if impl == "fixed_capacity" else {}))
    w = (l30.router, l30.gate, l30.up, l30.down)
    static_x = make_x(T, l30.D, seed=40 + T).reshape(1, T, l30.D)
    moe_swiglu_ffn(static_x, *w, cfg=cfg)
    g, static_out = _capture(lambda: moe_swiglu_ffn(static_x, *w, cfg=cfg))
    for i in range(3):
        xi = make_x(T, l30.D, seed=100 * i + T).reshape(1, T, l30.D)
        static_x.copy_(xi)
        g.replay()
        torch.cuda.synchronize()
        want = moe_swiglu_ffn(xi, *w, cfg=cfg)
        torch.cuda.synchronize()
        assert torch.equal(static_out, want), f"replay {i}"


def test_graph_replay_of_the_block(dev, l30):
    from kappa_amd.qwen3 import moe_block_ffn

    cfg = layer_cfg(l30, "ragged")
    w = (l30.router, l30.gate, l30.up, l30.down)
    T = 16
    scale = torch.ones(l30.D, dtype=torch.bfloat16, device=dev) * 1.25
    static_h = make_x(T, l30.D, seed=7).reshape(1, T, l30.D)
    moe_block_ffn(static_h, scale, *w, cfg=cfg)
    g, static_out = _capture(lambda: moe_block_ffn(static_h, scale, *w, cfg=cfg))
    for i in range(3):
        hi = make_x(T, l30.D, seed=300 + i).reshape(1, T, l30.D)
        static_h.copy_(hi)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(static_out, moe_block_ffn(hi, scale, *w, cfg=cfg)), f"replay {i}"


def test_graph_replay_of_the_allocation_free_entry_point(dev, l30):
    """kmoe_forward_noalloc captured with no allocation at all inside the graph."""
    from kappa_amd import _lib
    from kappa_amd.qwen3.ffn_moe import PACK_CACHE, _desc
    from kappa_amd.qwen3.quant import weight_struct

    L = _lib.lib()
    T = 8
    desc = _desc(T, l30.D, l30.E, l30.K, l30.I, torch.bfloat16, impl="ragged_jax", threshold=0)
    r, _kr = weight_struct(l30.router, dev, n_out=l30.E, n_groups=None, name="router")
    gs, _kg = weight_struct(l30.gate, dev, n_out=l30.I, n_groups=l30.E, name="gate")
    us, _ku = weight_struct(l30.up, dev, n_out=l30.I, n_groups=l30.E, name="up")
    ds, _kd = weight_struct(l30.down, dev, n_out=l30.D, n_groups=l30.E, name="down")
    packed = PACK_CACHE.get(l30.gate, l30.up, l30.down)
    p = packed.struct()
    static_x = make_x(T, l30.D, seed=11)
    out = torch.empty_like(static_x)

    def call():
        st = L.kmoe_forward_noalloc(desc, static_x.data_ptr(), r, gs, us, ds, p, out.data_ptr(), None, None,
                                    ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))  # fmt: skip
        _lib.check(st)
        return out

    g, _ = _capture(call)
    ws = torch.empty(_workspace_bytes(L, desc), dtype=torch.uint8, device=dev)
    want = torch.empty_like(out)
    for i in range(3):
        xi = make_x(T, l30.D, seed=500 + i)
        static_x.copy_(xi)
        g.replay()
        torch.cuda.synchronize()
        got = out.clone()
        _lib.check(L.kmoe_forward(desc, xi.data_ptr(), r, gs, us, ds, p, want.data_ptr(), None, None, ws.data_ptr(),
                                  ws.numel(), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)))  # fmt: skip
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"replay {i}"


def _workspace_bytes(L, desc):
    from kappa_amd import _lib

    n = ctypes.c_size_t()
    _lib.check(L.kmoe_workspace_bytes(desc, ctypes.byref(n)))
    return n.value
