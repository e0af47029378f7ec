"""ctypes binding of libkmoe.so (include/kmoe.h).

The library is built in-tree by ``python -m kappa_amd.build``. Loading fails
loudly when it is missing: there is no CPU or framework fallback for the block.
"""

from __future__ import annotations

import ctypes
import os
import threading

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libkmoe.so")

# kmoe_status
OK = 0
ERR_INVALID_ARG = 1
ERR_UNSUPPORTED = 2
ERR_WORKSPACE_TOO_SMALL = 3
ERR_NO_DEVICE = 4
ERR_HIP = 5

# kmoe_dtype
DTYPE_F32 = 0
DTYPE_BF16 = 1
DTYPE_I8 = 2

# kmoe_scale_kind
SCALE_NONE = 0
SCALE_TENSOR = 1
SCALE_CHANNEL = 2

# kmoe_impl
IMPL_GATHER_EINSUM = 0
IMPL_RAGGED = 1
IMPL_FIXED_CAPACITY = 2

# kmoe_kernels
KERNELS_AUTO = 0
KERNELS_DECODE = 1
KERNELS_GROUPED = 2

ABI_VERSION = 4

# kmoe_forward_noalloc's workspace (KMOE_NOALLOC_SCRATCH_BYTES)
NOALLOC_SCRATCH_BYTES = 16 << 20

# Every symbol include/kmoe.h declares.
EXPORTS = (
    "kmoe_version",
    "kmoe_abi_version",
    "kmoe_status_string",
    "kmoe_last_error",
    "kmoe_device_check",
    "kmoe_workspace_bytes",
    "kmoe_prepack_bytes",
    "kmoe_forward",
    "kmoe_forward_noalloc",
    "kmoe_forward_block",
    "kmoe_rms_norm",
    "kmoe_route",
    "kmoe_route_scratch_bytes",
    "kmoe_dispatch",
    "kmoe_expert_ffn",
    "kmoe_expert_gate_up",
    "kmoe_expert_down",
    "kmoe_combine",
    "kmoe_prepack",
    "kmoe_to_compute_dtype",
    "kmoe_quantize_per_channel",
)


class KmoeWeight(ctypes.Structure):
    _fields_ = [
        ("values", ctypes.c_void_p),
        ("dtype", ctypes.c_int),
        ("scale", ctypes.c_void_p),
        ("scale_dtype", ctypes.c_int),
        ("scale_kind", ctypes.c_int),
    ]


class KmoeDesc(ctypes.Structure):
    _fields_ = [
        ("tokens", ctypes.c_int64),
        ("hidden", ctypes.c_int64),
        ("num_experts", ctypes.c_int64),
        ("top_k", ctypes.c_int64),
        ("intermediate", ctypes.c_int64),
        ("act_dtype", ctypes.c_int),
        ("impl", ctypes.c_int),
        ("decode_token_threshold", ctypes.c_int64),
        ("expert_capacity", ctypes.c_int64),
        ("kernels", ctypes.c_int),
    ]


class KmoePacked(ctypes.Structure):
    _fields_ = [
        ("w13", ctypes.c_void_p),
        ("s13", ctypes.c_void_p),
        ("w2", ctypes.c_void_p),
        ("s2", ctypes.c_void_p),
        ("num_experts", ctypes.c_int64),
        ("hidden", ctypes.c_int64),
        ("intermediate", ctypes.c_int64),
        ("source_scale_kind", ctypes.c_int),
    ]


class KmoePackedSizes(ctypes.Structure):
    _fields_ = [
        ("w13_bytes", ctypes.c_size_t),
        ("s13_bytes", ctypes.c_size_t),
        ("w2_bytes", ctypes.c_size_t),
        ("s2_bytes", ctypes.c_size_t),
    ]


class KmoeError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(message)
        self.status = status


_lock = threading.Lock()
_lib: ctypes.CDLL | None = None

_P = ctypes.c_void_p
_WP = ctypes.POINTER(KmoeWeight)
_DP = ctypes.POINTER(KmoeDesc)
_PP = ctypes.POINTER(KmoePacked)


def _declare(L: ctypes.CDLL) -> None:
    L.kmoe_version.restype = ctypes.c_char_p
    L.kmoe_abi_version.restype = ctypes.c_int
    L.kmoe_status_string.restype = ctypes.c_char_p
    L.kmoe_status_string.argtypes = [ctypes.c_int]
    L.kmoe_last_error.restype = ctypes.c_char_p
    L.kmoe_device_check.restype = ctypes.c_int
    L.kmoe_workspace_bytes.restype = ctypes.c_int
    L.kmoe_workspace_bytes.argtypes = [_DP, ctypes.POINTER(ctypes.c_size_t)]
    L.kmoe_prepack_bytes.restype = ctypes.c_int
    L.kmoe_prepack_bytes.argtypes = [_DP, ctypes.POINTER(KmoePackedSizes)]
    L.kmoe_forward.restype = ctypes.c_int
    L.kmoe_forward.argtypes = [_DP, _P, _WP, _WP, _WP, _WP, _PP, _P, _P, _P, _P, ctypes.c_size_t, _P]
    L.kmoe_forward_noalloc.restype = ctypes.c_int
    L.kmoe_forward_noalloc.argtypes = [_DP, _P, _WP, _WP, _WP, _WP, _PP, _P, _P, _P, _P]
    L.kmoe_route.restype = ctypes.c_int
    L.kmoe_forward_block.restype = ctypes.c_int
    L.kmoe_forward_block.argtypes = [
        _DP, _P, _P, ctypes.c_int, ctypes.c_float, _WP, _WP, _WP, _WP, _PP, _P, _P, _P, _P, ctypes.c_size_t, _P,
    ]  # fmt: skip
    L.kmoe_rms_norm.restype = ctypes.c_int
    L.kmoe_rms_norm.argtypes = [_DP, _P, _P, ctypes.c_int, ctypes.c_float, _P, _P]
    L.kmoe_route.argtypes = [_DP, _P, _WP, _P, _P, ctypes.c_size_t, _P, _P, _P, _P]
    L.kmoe_route_scratch_bytes.restype = ctypes.c_int
    L.kmoe_route_scratch_bytes.argtypes = [_DP, ctypes.POINTER(ctypes.c_size_t)]
    L.kmoe_dispatch.restype = ctypes.c_int
    L.kmoe_dispatch.argtypes = [_DP, _P, _P, _P, _P, _P, _P, _P, _P, _P]
    L.kmoe_expert_ffn.restype = ctypes.c_int
    L.kmoe_expert_ffn.argtypes = [_DP, _P, _P, _P, _P, _P, _WP, _WP, _WP, _PP, _P, _P, _P]
    L.kmoe_expert_gate_up.restype = ctypes.c_int
    L.kmoe_expert_gate_up.argtypes = [_DP, _P, _P, _P, _P, _P, _WP, _WP, _PP, _P, _P]
    L.kmoe_expert_down.restype = ctypes.c_int
    L.kmoe_expert_down.argtypes = [_DP, _P, _P, _P, _P, _WP, _PP, _P, _P]
    L.kmoe_combine.restype = ctypes.c_int
    L.kmoe_combine.argtypes = [_DP, _P, _P, _P, _P, _P]
    L.kmoe_prepack.restype = ctypes.c_int
    L.kmoe_prepack.argtypes = [_DP, _WP, _WP, _WP, _PP, _P]
    L.kmoe_to_compute_dtype.restype = ctypes.c_int
    L.kmoe_to_compute_dtype.argtypes = [_WP, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int, _P, _P]
    L.kmoe_quantize_per_channel.restype = ctypes.c_int
    L.kmoe_quantize_per_channel.argtypes = [
        ctypes.c_int64,
        ctypes.c_int64,
        ctypes.c_int64,
        _P,
        ctypes.c_int,
        _P,
        _P,
        _P,
    ]


def lib() -> ctypes.CDLL:
    """Load libkmoe.so (once). Raises if it has not been built."""
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not os.path.exists(LIB_PATH):
                    raise ImportError(
                        f"{LIB_PATH} is missing: build the HIP library with `python -m kappa_amd.build`"
                    )
                L = ctypes.CDLL(LIB_PATH)
                _declare(L)
                if L.kmoe_abi_version() != ABI_VERSION:
                    raise ImportError(
                        f"{LIB_PATH} has ABI {L.kmoe_abi_version()}, this binding expects {ABI_VERSION}: rebuild it"
                    )
                _lib = L
    return _lib


def check(status: int) -> None:
    """Raise on a non-OK status: ValueError for argument errors, KmoeError otherwise."""
    if status == OK:
        return
    L = lib()
    msg = L.kmoe_last_error().decode() or L.kmoe_status_string(status).decode()
    if status in (ERR_INVALID_ARG, ERR_UNSUPPORTED, ERR_WORKSPACE_TOO_SMALL):
        raise ValueError(msg)
    raise KmoeError(status, msg)
