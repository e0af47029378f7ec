"""kmoe_forward_noalloc (GPU): the allocation-free variant of kmoe_forward.

It runs the same kernels on a workspace inside the library (a device array per
GPU) instead of a caller's buffer, so its outputs and routing must equal
kmoe_forward's bit for bit. Two calls in a row, the second with fewer tokens,
check that the shared array's leftover contents from the first call do not
leak into the second; kmoe_forward's workspace starts as all-ones bytes (NaN),
so a read of a byte no kernel wrote would differ; the second call is also
checked against the oracle.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

import oracle
from moe_cases import bf16_np, make_layer, make_x, mean_rel

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    return torch.device("cuda:0")


def _structs(layer, T, impl, threshold, capacity=0):
    from kappa_amd import _lib
    from kappa_amd.qwen3.ffn_moe import PACK_CACHE, _desc
    from kappa_amd.qwen3.quant import weight_struct

    dev = layer.router.device
    desc = _desc(T, layer.D, layer.E, layer.K, layer.I, torch.bfloat16, impl=impl, threshold=threshold,
                 capacity=capacity)  # fmt: skip
    keep = []
    ws = []
    for w, n, grp in ((layer.router, layer.E, None), (layer.gate, layer.I, layer.E), (layer.up, layer.I, layer.E),
                      (layer.down, layer.D, layer.E)):  # fmt: skip
        st, k = weight_struct(w, dev, n_out=n, n_groups=grp, name="w")
        ws.append(st)
        keep.append(k)
    packed = PACK_CACHE.get(layer.gate, layer.up, layer.down)
    return desc, ws, packed, keep


def _both(layer, x, impl, threshold, capacity=0):
    """(out, idx, w) of kmoe_forward with a workspace and of kmoe_forward_noalloc."""
    from kappa_amd import _lib

    L = _lib.lib()
    T = x.shape[0]
    desc, (r, g, u, d), packed, keep = _structs(layer, T, impl, threshold, capacity)
    n = ctypes.c_size_t()
    _lib.check(L.kmoe_workspace_bytes(desc, ctypes.byref(n)))
    assert n.value <= _lib.NOALLOC_SCRATCH_BYTES
    # all-ones bytes (NaN as bf16 and f32, -1 as int32): a kernel that read a
    # workspace byte it did not write first would show in the comparison below
    wsb = torch.full((n.value,), 0xFF, dtype=torch.uint8, device=x.device)
    stream = torch.cuda.current_stream().cuda_stream
    res = []
    for noalloc in (False, True):
        out = torch.empty_like(x)
        idx = torch.empty((T, layer.K), dtype=torch.int32, device=x.device)
        w = torch.empty((T, layer.K), dtype=x.dtype, device=x.device)
        pk = packed.struct()
        if noalloc:
            st = L.kmoe_forward_noalloc(desc, x.data_ptr(), r, g, u, d, pk, out.data_ptr(), idx.data_ptr(),
                                        w.data_ptr(), stream)  # fmt: skip
        else:
            st = L.kmoe_forward(desc, x.data_ptr(), r, g, u, d, pk, out.data_ptr(), idx.data_ptr(), w.data_ptr(),
                                wsb.data_ptr(), wsb.numel(), stream)  # fmt: skip
        _lib.check(st)
        res.append((out, idx, w))
    torch.cuda.synchronize()
    return res


@pytest.mark.parametrize(
    "impl,threshold,capacity",
    [("ragged_jax", 0, 0), ("fixed_capacity", 64, 2)],
    ids=["ragged", "fixed_capacity"],
)
def test_noalloc_equals_forward_on_two_calls(dev, impl, threshold, capacity):
    layer = make_layer("30b", seed=0)
    # the second call is smaller: it must not pick up the first call's leftovers
    for T, seed in ((200, 11), (5, 12)):
        x = make_x(T, layer.D, seed=seed)
        (o1, i1, w1), (o2, i2, w2) = _both(layer, x, impl, threshold, capacity)
        assert torch.equal(i1, i2) and torch.equal(w1, w2)
        assert torch.equal(o1, o2), f"T={T}"
        assert torch.isfinite(o2.float()).all()
    # and the smaller call against the oracle of its program
    h = layer.host()
    ref = oracle.forward(bf16_np(x), h["router"], h["gate"], h["up"], h["down"], k=layer.K, act_bf16=True,
                         impl="ragged" if impl == "ragged_jax" else impl, capacity=capacity or None)  # fmt: skip
    np.testing.assert_array_equal(i2.cpu().numpy(), ref["idx"])
    d = np.abs(bf16_np(o2) - ref["out"])
    assert d.max() <= 2e-2 and mean_rel(bf16_np(o2), ref["out"]) <= 1e-3


def test_noalloc_rejects_calls_beyond_its_scratch(dev):
    from kappa_amd import _lib

    L = _lib.lib()
    layer = make_layer("30b", seed=0)
    desc, (r, g, u, d), packed, keep = _structs(layer, 4096, "ragged_jax", 0)
    x = torch.empty(1, dtype=torch.bfloat16, device=dev)
    st = L.kmoe_forward_noalloc(desc, x.data_ptr(), r, g, u, d, packed.struct(), x.data_ptr(), None, None,
                                torch.cuda.current_stream().cuda_stream)  # fmt: skip
    assert st == _lib.ERR_WORKSPACE_TOO_SMALL
    assert "scratch" in L.kmoe_last_error().decode()
