"""The C ABI on the host (CPU): exports, argument validation and error statuses.

No compute call runs here: every call either fails validation before touching
HIP, or reaches the device check and reports that no device is visible (this
suite also runs where there is no GPU)."""

import ctypes
import os
import re

import pytest

from conftest import ROOT, gpu_available
from kappa_amd import _lib

HEADER = os.path.join(ROOT, "include", "kmoe.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(kmoe_[a-z_0-9]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    L = _lib.lib()
    names = declared_functions()
    assert len(names) >= 15
    assert sorted(_lib.EXPORTS) == names
    for n in names:
        assert hasattr(L, n), n


def test_version_and_status_strings():
    L = _lib.lib()
    assert L.kmoe_abi_version() == 4 == _lib.ABI_VERSION
    assert b"gfx950" in L.kmoe_version()
    for s in range(6):
        assert L.kmoe_status_string(s)
    assert L.kmoe_status_string(99) == b"unknown status"


def desc(T=4, D=128, E=8, K=2, I=64, act=_lib.DTYPE_BF16, thr=0, cap=0, impl=_lib.IMPL_RAGGED,
         kernels=_lib.KERNELS_AUTO):  # fmt: skip
    return _lib.KmoeDesc(T, D, E, K, I, act, impl, thr, cap, kernels)


def packed(E=8, D=128, I=64, kind=_lib.SCALE_CHANNEL, s2=1):
    return _lib.KmoePacked(1, 1, 1, s2, E, D, I, kind)


def status_and_msg(st):
    return st, _lib.lib().kmoe_last_error().decode()


@pytest.mark.parametrize(
    "kw,frag",
    [
        (dict(T=-1), "tokens"),
        (dict(D=0), "hidden"),
        (dict(K=0), "top_k"),
        (dict(K=9), "top_k"),
        (dict(act=_lib.DTYPE_I8), "act_dtype"),
        (dict(cap=-1), "expert_capacity"),
        (dict(impl=7), "unknown impl"),
        (dict(impl=_lib.IMPL_FIXED_CAPACITY), "expert_capacity >= 1"),
        (dict(impl=_lib.IMPL_GATHER_EINSUM, cap=4), "unless impl is fixed_capacity"),
        (dict(kernels=5), "unknown kernels"),
    ],
)
def test_workspace_bytes_rejects_bad_desc(kw, frag):
    n = ctypes.c_size_t()
    st, msg = status_and_msg(_lib.lib().kmoe_workspace_bytes(desc(**kw), ctypes.byref(n)))
    assert st == _lib.ERR_INVALID_ARG and frag in msg


def test_unsupported_sizes():
    n = ctypes.c_size_t()
    L = _lib.lib()
    assert L.kmoe_workspace_bytes(desc(E=2048, K=2), ctypes.byref(n)) == _lib.ERR_UNSUPPORTED
    assert L.kmoe_workspace_bytes(desc(D=8192), ctypes.byref(n)) == _lib.ERR_UNSUPPORTED
    sizes = _lib.KmoePackedSizes()
    assert L.kmoe_prepack_bytes(desc(D=96), sizes) == _lib.ERR_UNSUPPORTED
    st = L.kmoe_workspace_bytes(desc(T=129, kernels=_lib.KERNELS_DECODE), ctypes.byref(n))
    assert st == _lib.ERR_UNSUPPORTED and "at most 128 tokens" in L.kmoe_last_error().decode()


def test_workspace_and_packed_sizes():
    L = _lib.lib()
    n = ctypes.c_size_t()
    assert L.kmoe_workspace_bytes(desc(T=4096, D=2048, E=128, K=8, I=768), ctypes.byref(n)) == _lib.OK
    M = 4096 * 8
    # the ragged program above the threshold keeps h as two bf16 planes
    assert n.value >= 2 * M * (2 * 768 + 2048) + 4 * 3 * M
    ragged = n.value
    assert L.kmoe_workspace_bytes(desc(T=4096, D=2048, E=128, K=8, I=768, thr=4096), ctypes.byref(n)) == _lib.OK
    assert ragged - n.value >= 2 * M * 768 - 256  # at the threshold: the gather program, one plane
    assert L.kmoe_workspace_bytes(desc(T=4096, D=2048, E=128, K=8, I=768, impl=_lib.IMPL_GATHER_EINSUM),
                                  ctypes.byref(n)) == _lib.OK  # fmt: skip
    assert n.value >= 2 * M * (768 + 2048) + 4 * 3 * M
    sizes = _lib.KmoePackedSizes()
    assert L.kmoe_prepack_bytes(desc(D=2048, E=128, I=768), sizes) == _lib.OK
    assert sizes.w13_bytes == 2 * 128 * 2048 * 768 and sizes.w2_bytes == 128 * 2048 * 768
    assert sizes.s13_bytes == 4 * 2 * 128 * 768 and sizes.s2_bytes == 4 * 128 * 2048


def weight(values=1, dtype=_lib.DTYPE_I8, scale=1, sdtype=_lib.DTYPE_F32, kind=_lib.SCALE_CHANNEL):
    return _lib.KmoeWeight(values, dtype, scale, sdtype, kind)


def test_forward_validation_before_any_hip_call():
    L = _lib.lib()
    d = desc()
    w = weight()
    f = weight(dtype=_lib.DTYPE_BF16, scale=None, kind=_lib.SCALE_NONE)
    cases = [
        (dict(router=weight(values=None)), _lib.ERR_INVALID_ARG, "router values"),
        (dict(router=weight(kind=_lib.SCALE_NONE)), _lib.ERR_INVALID_ARG, "TENSOR or CHANNEL"),
        (dict(router=weight(scale=None)), _lib.ERR_INVALID_ARG, "scale pointer"),
        (dict(router=weight(dtype=_lib.DTYPE_BF16)), _lib.ERR_INVALID_ARG, "takes no scale"),
        (dict(x=None), _lib.ERR_INVALID_ARG, "x and out"),
        (dict(ws=None), _lib.ERR_WORKSPACE_TOO_SMALL, "workspace"),
        (dict(ws_bytes=16), _lib.ERR_WORKSPACE_TOO_SMALL, "workspace"),
    ]
    for over, want, frag in cases:
        a = dict(router=f, x=1, ws=1, ws_bytes=1 << 40)
        a.update(over)
        st = L.kmoe_forward(d, a["x"], a["router"], w, w, w, None, 1, None, None, a["ws"], a["ws_bytes"], None)
        msg = L.kmoe_last_error().decode()
        assert st == want and frag in msg, (over, st, msg)


def test_gather_program_rejects_per_channel_scales():
    """moe_take_dequant (kappa/qwen3/quant.py:71-74) cannot apply [E, 1, N] scales; the
    ragged and fixed_capacity programs can. Checked before any HIP call."""
    L = _lib.lib()
    ch = weight(kind=_lib.SCALE_CHANNEL)
    pt = weight(kind=_lib.SCALE_TENSOR)
    f = weight(dtype=_lib.DTYPE_BF16, scale=None, kind=_lib.SCALE_NONE)

    def fwd(d, g, p=None):
        return status_and_msg(L.kmoe_forward(d, 1, f, g, g, g, p, 1, None, None, 1, 1 << 40, None))

    st, msg = fwd(desc(impl=_lib.IMPL_GATHER_EINSUM), ch)
    assert st == _lib.ERR_INVALID_ARG and "one scale per tensor" in msg
    # ragged at or below the decode threshold runs the gather program (:219-223)
    st, msg = fwd(desc(impl=_lib.IMPL_RAGGED, thr=64), ch)
    assert st == _lib.ERR_INVALID_ARG and "one scale per tensor" in msg
    st, msg = fwd(desc(impl=_lib.IMPL_GATHER_EINSUM, E=1, K=1), ch)  # [1, 1, N] broadcasts
    assert st != _lib.ERR_INVALID_ARG, msg
    for d in (desc(impl=_lib.IMPL_GATHER_EINSUM), desc(impl=_lib.IMPL_RAGGED, thr=0),
              desc(impl=_lib.IMPL_FIXED_CAPACITY, cap=3)):  # fmt: skip
        st, msg = fwd(d, pt)
        assert st != _lib.ERR_INVALID_ARG, msg
    st, msg = fwd(desc(impl=_lib.IMPL_RAGGED, thr=0), ch)
    assert st != _lib.ERR_INVALID_ARG, msg
    # packed experts carry the kind of their source scales
    st, msg = fwd(desc(impl=_lib.IMPL_GATHER_EINSUM), ch, packed(kind=_lib.SCALE_CHANNEL))
    assert st == _lib.ERR_INVALID_ARG and "one scale per tensor" in msg
    st, msg = fwd(desc(impl=_lib.IMPL_GATHER_EINSUM), ch, packed(kind=_lib.SCALE_TENSOR))
    assert st != _lib.ERR_INVALID_ARG, msg


@pytest.mark.skipif(gpu_available(), reason="checks the no-device status")
def test_valid_call_without_device_reports_no_device():
    L = _lib.lib()
    w = weight()
    f = weight(dtype=_lib.DTYPE_BF16, scale=None, kind=_lib.SCALE_NONE)
    st = L.kmoe_forward(desc(), 1, f, w, w, w, None, 1, None, None, 1, 1 << 40, None)
    assert st == _lib.ERR_NO_DEVICE
    assert "no HIP device" in L.kmoe_last_error().decode()
    assert L.kmoe_device_check() == _lib.ERR_NO_DEVICE


def test_packed_argument_rules():
    L = _lib.lib()
    w = weight()
    f = weight(dtype=_lib.DTYPE_BF16, scale=None, kind=_lib.SCALE_NONE)
    st = L.kmoe_forward(desc(), 1, f, w, w, w, packed(s2=None), 1, None, None, 1, 1 << 40, None)
    assert st == _lib.ERR_INVALID_ARG
    st = L.kmoe_forward(desc(act=_lib.DTYPE_F32), 1, f, w, w, w, packed(), 1, None, None, 1, 1 << 40, None)
    assert st == _lib.ERR_UNSUPPORTED
    st = L.kmoe_forward(desc(D=96), 1, f, w, w, w, packed(D=96), 1, None, None, 1, 1 << 40, None)
    assert st == _lib.ERR_UNSUPPORTED
    # the packed copy must hold the call's E, D and I (a mismatch would index past it)
    for p in (packed(E=16), packed(D=256), packed(I=128)):
        st = L.kmoe_forward(desc(), 1, f, w, w, w, p, 1, None, None, 1, 1 << 40, None)
        assert st == _lib.ERR_INVALID_ARG and "packed experts hold" in L.kmoe_last_error().decode()
    st = L.kmoe_forward(desc(), 1, f, w, w, w, packed(kind=_lib.SCALE_NONE), 1, None, None, 1, 1 << 40, None)
    assert st == _lib.ERR_INVALID_ARG and "source_scale_kind" in L.kmoe_last_error().decode()


def test_stage_entry_points_validate():
    L = _lib.lib()
    f = weight(dtype=_lib.DTYPE_BF16, scale=None, kind=_lib.SCALE_NONE)
    assert L.kmoe_route(desc(), 1, f, None, None, 0, None, 1, 1, None) == _lib.ERR_INVALID_ARG
    # a scratch smaller than kmoe_route_scratch_bytes is refused
    n = ctypes.c_size_t()
    assert L.kmoe_route_scratch_bytes(desc(), ctypes.byref(n)) == _lib.OK and n.value >= 2 * 8 * 128
    st, msg = status_and_msg(L.kmoe_route(desc(), 1, f, None, 1, n.value - 1, 1, 1, 1, None))
    assert st == _lib.ERR_WORKSPACE_TOO_SMALL and "scratch" in msg
    assert L.kmoe_dispatch(desc(), 1, 1, 1, 1, 1, 1, 1, None, None) == _lib.ERR_INVALID_ARG
    assert L.kmoe_combine(desc(), 1, None, 1, 1, None) == _lib.ERR_INVALID_ARG
    assert L.kmoe_expert_ffn(desc(), 1, 1, 1, 1, 1, None, None, None, None, 1, 1, None) == _lib.ERR_INVALID_ARG
    i8 = weight()
    assert L.kmoe_prepack(desc(), f, i8, i8, packed(), None) == _lib.ERR_UNSUPPORTED
    assert L.kmoe_prepack(desc(), i8, i8, i8, packed(E=4), None) == _lib.ERR_INVALID_ARG
    # the recorded kind of the source scales must be theirs: the forward calls trust
    # it when they refuse per-channel scales under the gather program
    pt = weight(kind=_lib.SCALE_TENSOR)
    st, msg = status_and_msg(L.kmoe_prepack(desc(), i8, i8, i8, packed(kind=_lib.SCALE_TENSOR), None))
    assert st == _lib.ERR_INVALID_ARG and "source_scale_kind must be CHANNEL" in msg
    st, msg = status_and_msg(L.kmoe_prepack(desc(), pt, pt, i8, packed(kind=_lib.SCALE_TENSOR), None))
    assert st == _lib.ERR_INVALID_ARG and "source_scale_kind must be CHANNEL" in msg
    st, msg = status_and_msg(L.kmoe_prepack(desc(), pt, pt, pt, packed(kind=_lib.SCALE_CHANNEL), None))
    assert st == _lib.ERR_INVALID_ARG and "source_scale_kind must be TENSOR" in msg
    assert L.kmoe_to_compute_dtype(i8, 4, 0, 1, _lib.DTYPE_BF16, 1, None) == _lib.ERR_INVALID_ARG
    assert L.kmoe_quantize_per_channel(1, 4, 4, 1, _lib.DTYPE_I8, 1, 1, None) == _lib.ERR_INVALID_ARG


def test_zero_tokens_is_a_no_op_after_validation():
    if gpu_available():
        pytest.skip("the device check passes on a GPU host")
    L = _lib.lib()
    w = weight()
    f = weight(dtype=_lib.DTYPE_BF16, scale=None, kind=_lib.SCALE_NONE)
    # T = 0 still validates, then reports the missing device (no launch is attempted)
    st = L.kmoe_forward(desc(T=0, thr=-1), 1, f, w, w, w, None, 1, None, None, None, 0, None)
    assert st == _lib.ERR_NO_DEVICE


def test_block_and_norm_entry_points_validate_before_any_hip_call():
    L = _lib.lib()
    d = desc()
    w = weight()
    f = weight(dtype=_lib.DTYPE_BF16, scale=None, kind=_lib.SCALE_NONE)
    BF = _lib.DTYPE_BF16
    cases = [
        (dict(scale=None), _lib.ERR_INVALID_ARG, "norm scale pointer"),
        (dict(sdt=_lib.DTYPE_I8), _lib.ERR_INVALID_ARG, "norm scale dtype"),
        (dict(eps=-1.0), _lib.ERR_INVALID_ARG, "epsilon"),
        (dict(eps=float("nan")), _lib.ERR_INVALID_ARG, "epsilon"),
        (dict(h=None), _lib.ERR_INVALID_ARG, "h and out"),
        (dict(out=7), _lib.ERR_INVALID_ARG, "alias"),
        (dict(ws=None), _lib.ERR_WORKSPACE_TOO_SMALL, "workspace"),
        (dict(router=weight(values=None)), _lib.ERR_INVALID_ARG, "router values"),
    ]
    for over, want, frag in cases:
        a = dict(h=7, scale=1, sdt=BF, eps=1e-6, router=f, out=9, ws=1)
        a.update(over)
        st = L.kmoe_forward_block(d, a["h"], a["scale"], a["sdt"], a["eps"], a["router"], w, w, w, None, a["out"],
                                  None, None, a["ws"], 1 << 40, None)  # fmt: skip
        msg = L.kmoe_last_error().decode()
        assert st == want and frag in msg, (over, st, msg)
    assert L.kmoe_rms_norm(d, 1, None, BF, 1e-6, 2, None) == _lib.ERR_INVALID_ARG
    assert L.kmoe_rms_norm(d, 1, 1, _lib.DTYPE_I8, 1e-6, 2, None) == _lib.ERR_INVALID_ARG
    assert L.kmoe_rms_norm(d, None, 1, BF, 1e-6, 2, None) == _lib.ERR_INVALID_ARG
    if not gpu_available():
        assert L.kmoe_rms_norm(d, 1, 1, BF, 1e-6, 2, None) == _lib.ERR_NO_DEVICE
        st = L.kmoe_forward_block(d, 7, 1, BF, 1e-6, f, w, w, w, None, 9, None, None, 1, 1 << 40, None)
        assert st == _lib.ERR_NO_DEVICE


def test_noalloc_entry_point_limits_before_any_hip_call():
    """kmoe_forward_noalloc runs on a fixed scratch array: a call whose workspace does
    not fit is refused before any HIP call; one that fits reaches the device check."""
    L = _lib.lib()
    w = weight()
    f = weight(dtype=_lib.DTYPE_BF16, scale=None, kind=_lib.SCALE_NONE)
    big = desc(T=4096, D=2048, E=128, K=8, I=768)
    n = ctypes.c_size_t()
    assert L.kmoe_workspace_bytes(big, ctypes.byref(n)) == _lib.OK and n.value > _lib.NOALLOC_SCRATCH_BYTES
    st, msg = status_and_msg(L.kmoe_forward_noalloc(big, 1, f, w, w, w, None, 1, None, None, None))
    assert st == _lib.ERR_WORKSPACE_TOO_SMALL and "scratch" in msg
    fits = desc(T=200, D=2048, E=128, K=8, I=768)
    assert L.kmoe_workspace_bytes(fits, ctypes.byref(n)) == _lib.OK and n.value <= _lib.NOALLOC_SCRATCH_BYTES
    st, msg = status_and_msg(L.kmoe_forward_noalloc(fits, None, f, w, w, w, None, 1, None, None, None))
    assert st == _lib.ERR_INVALID_ARG and "x and out" in msg
    if not gpu_available():
        st, msg = status_and_msg(L.kmoe_forward_noalloc(fits, 1, f, w, w, w, None, 1, None, None, None))
        assert st == _lib.ERR_NO_DEVICE
    # the documented limits (include/kmoe.h): 30B-A3B up to 291 tokens, 235B-A22B up to 136
    for D, I, limit in ((2048, 768, 291), (4096, 1536, 136)):
        over = desc(T=limit + 1, D=D, E=128, K=8, I=I)
        st, msg = status_and_msg(L.kmoe_forward_noalloc(over, 1, f, w, w, w, None, 1, None, None, None))
        assert st == _lib.ERR_WORKSPACE_TOO_SMALL and "scratch" in msg, (D, st, msg)
        if not gpu_available():  # a fitting call with placeholder pointers only reaches the device check here
            at = desc(T=limit, D=D, E=128, K=8, I=I)
            st, msg = status_and_msg(L.kmoe_forward_noalloc(at, 1, f, w, w, w, None, 1, None, None, None))
            assert st == _lib.ERR_NO_DEVICE, (D, st, msg)
