"""ctypes binding of ``librepresentax_amd.so`` (the C ABI in include/).

``import torch`` happens first on purpose: torch's ROCm wheel ships its own
HIP runtime under the same soname, so the library binds to that one runtime
and torch's streams and device pointers are valid inside it.
"""

from __future__ import annotations

import ctypes
import importlib.machinery
import importlib.util
import os
import sysconfig
from pathlib import Path

import torch  # noqa: F401  (load torch's HIP runtime before the library)

LIB_PATH = Path(__file__).resolve().parent / "_lib" / "librepresentax_amd.so"
FAST_PATH = LIB_PATH.parent / ("_rpxfast" + (sysconfig.get_config_var("EXT_SUFFIX") or ".so"))

RPX_OK = 0
RPX_ERR_INVALID = 1
RPX_ERR_HIP = 2
RPX_ERR_DEVICE = 3
DTYPE_F32 = 0
DTYPE_BF16 = 1
FP8_E4M3FN = 0
FP8_E5M2 = 1
ACT_GELU = 1
ACT_SILU_MUL = 2
ACT_ADD = 3
# kernel-variant knobs (rpx_set_tuning)
TUNE_INT4_TILE = 0
TUNE_BF16_TILE = 1
TUNE_FP8_TILE = 2
TUNE_SKINNY_TILE = 3
TUNE_SKINNY2 = 4
TUNE_SKINNY2_ONE = 5
TUNE_SPIN_LIMIT = 6
TUNE_GEMM_BAND = 7
TUNE_DX_PACKED = 8
TUNE_RANK_BLOCKS = 9
TUNE_RANK_NT_U = 10
TUNE_FP8_SPLITS = 11
TUNE_FP8_PAIR = 12

_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_int = ctypes.c_int
_f32 = ctypes.c_float
_size = ctypes.c_size_t

# name -> (restype, argtypes); mirrors include/representax_amd.h
SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "rpx_last_error": (ctypes.c_char_p, []),
    "rpx_abi_version": (_int, []),
    "rpx_set_tuning": (_int, [_int, _int]),
    "rpx_get_tuning": (_int, [_int]),
    "rpx_check_device_errors": (_int, [_p, _p]),
    "rpx_int4_pack": (_int, [_p, _int, _i64, _i64, _i64, _p, _p, _p]),
    "rpx_int4_dequant": (_int, [_p, _p, _i64, _i64, _i64, _p, _p]),
    "rpx_int4_merge": (_int, [_p, _p, _p, _p, _i64, _i64, _i64, _i64, _f32, _p, _p]),
    "rpx_int4lora_forward_workspace": (_size, [_i64, _i64, _i64, _i64, _i64, _int]),
    "rpx_int4lora_forward": (
        _int,
        [_p, _int, _i64, _i64, _p, _p, _i64, _i64, _p, _p, _p, _i64, _f32, _p, _p, _p, _size, _p],
    ),
    "rpx_int4lora_forward_static": (
        _int, [_p, _int, _i64, _i64, _p, _p, _i64, _i64, _p, _p, _p, _i64, _f32, _p, _p, _p],
    ),
    "rpx_int4lora_backward_workspace": (_size, [_i64, _i64, _i64, _i64, _i64, _int]),
    "rpx_int4lora_backward": (
        _int,
        [_p, _p, _int, _i64, _i64, _p, _p, _i64, _i64, _p, _p, _i64, _f32, _p, _p, _p, _p, _p,
         _size, _p],
    ),
    "rpx_int4lora_forward_act": (
        _int,
        [_p, _int, _i64, _i64, _p, _p, _i64, _i64, _p, _p, _p, _i64, _f32, _int, _p, _p, _p, _p,
         _p, _size, _p],
    ),
    "rpx_int4lora_backward_act": (
        _int,
        [_p, _p, _int, _i64, _i64, _p, _p, _i64, _i64, _p, _p, _i64, _f32, _p, _int, _p, _p, _p,
         _p, _p, _p, _p, _size, _p],
    ),
    "rpx_int4lora_forward_promoted_workspace": (_size, [_i64, _i64, _i64, _i64, _i64]),
    "rpx_int4lora_forward_promoted": (
        _int,
        [_p, _i64, _i64, _p, _p, _i64, _i64, _p, _p, _p, _i64, _f32, _p, _p, _p, _size, _p],
    ),
    "rpx_int4lora_backward_promoted_workspace": (_size, [_i64, _i64, _i64, _i64, _i64]),
    "rpx_int4lora_backward_promoted": (
        _int,
        [_p, _p, _i64, _i64, _p, _p, _i64, _i64, _p, _p, _i64, _f32, _p, _p, _p, _p, _p, _size,
         _p],
    ),
    "rpx_fp8_scale_workspace": (_size, [_i64]),
    "rpx_fp8_scale": (_int, [_p, _int, _i64, _int, _p, _p, _size, _p]),
    "rpx_fp8_cast": (_int, [_p, _int, _i64, _i64, _i64, _i64, _p, _int, _p, _p, _p]),
    "rpx_fp8_gemm_workspace": (_size, [_i64, _i64, _i64]),
    "rpx_fp8_gemm": (
        _int, [_p, _int, _p, _p, _int, _p, _i64, _i64, _i64, _p, _int, _p, _size, _p]
    ),
    "rpx_fp8_linear_forward_workspace": (_size, [_i64, _i64, _i64]),
    "rpx_fp8_linear_forward": (
        _int, [_p, _int, _i64, _i64, _p, _int, _i64, _i64, _i64, _p, _int, _p, _p, _p, _p, _size, _p]
    ),
    "rpx_fp8_linear_backward_workspace": (_size, [_i64, _i64, _i64]),
    "rpx_fp8_linear_backward": (
        _int,
        [_p, _int, _p, _int, _i64, _i64, _i64, _i64, _i64, _p, _int, _p, _p, _p, _int, _int, _p,
         _size, _p],
    ),
    "rpx_fp8_linear_backward_codes": (
        _int, [_p, _p, _p, _i64, _i64, _i64, _p, _int, _p, _p, _int, _int, _p, _size, _p]
    ),
    "rpx_fp8_linear_backward_gemms_workspace": (_size, [_i64, _i64, _i64]),
    "rpx_fp8_linear_backward_gemms": (
        _int, [_p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _p, _p, _int, _int, _p, _size, _p]
    ),
    "rpx_fp8_delayed_pending_words": (_size, []),
    "rpx_fp8_cast_delayed": (
        _int, [_p, _int, _i64, _i64, _i64, _i64, _int, _p, _p, _i64, _i64, _p, _p, _p]
    ),
    "rpx_fp8_cast_delayed2": (
        _int,
        [_p, _i64, _i64, _i64, _i64, _i64, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _p, _p, _int,
         _int, _p, _p, _i64, _p],
    ),
    "rpx_fp8_scale_update": (_int, [_p, _p, _p, _p, _p, _i64, _i64, _p]),
    "rpx_fp8_encode_selfcheck": (
        _int, [_int, ctypes.c_uint64, ctypes.c_uint64, _p, _p, _i64, _p]
    ),
    "rpx_host_fp8_quantize": (_int, [_p, _i64, _f32, _int, _p]),
    "rpx_int4lora_forward_multi_workspace": (_size, [_i64, _i64, _int, _p, _int]),
    "rpx_int4lora_forward_multi": (_int, [_p, _int, _i64, _i64, _int, _p, _p, _size, _p]),
    "rpx_mnr_saved_bytes": (ctypes.c_size_t, [_i64, _i64, _i64]),
    "rpx_mnr_forward": (_int, [_p, _p, _int, _i64, _i64, _i64, _f32, _p, _p, ctypes.c_size_t, _p]),
    "rpx_mnr_backward": (_int, [_p, _p, ctypes.c_size_t, _i64, _i64, _i64, _f32, _p, _p, _int, _p]),
}


class Int4LoraProjection(ctypes.Structure):
    """``rpx_int4lora_projection`` of include/representax_amd.h."""

    _fields_ = [
        ("packed", ctypes.c_void_p),
        ("scale_bits", ctypes.c_void_p),
        ("n", ctypes.c_int64),
        ("group_size", ctypes.c_int64),
        ("bias_bits", ctypes.c_void_p),
        ("lora_a", ctypes.c_void_p),
        ("lora_b", ctypes.c_void_p),
        ("rank", ctypes.c_int64),
        ("scaling", ctypes.c_float),
        ("y", ctypes.c_void_p),
        ("h", ctypes.c_void_p),
    ]


class NativeError(RuntimeError):
    """A HIP-side failure reported by the library."""


class DeviceError(NativeError):
    """A kernel reported a problem through the device error word."""


_LIB: ctypes.CDLL | None = None


def load() -> ctypes.CDLL:
    """Load the library, or raise: there is no fallback implementation."""

    global _LIB
    if _LIB is not None:
        return _LIB
    path = Path(os.environ.get("RPX_LIBRARY", LIB_PATH))
    if not path.exists():
        raise ImportError(
            f"{path} is missing; build it with `python -m representax_amd.build` "
            "(the quantized-linear path has no non-HIP implementation)"
        )
    lib = ctypes.CDLL(str(path))
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    _LIB = lib
    return lib


_FAST = None


def fast():
    """The CPython fast-call binding of the small-M forward entry points
    (``csrc/pyfast.c``), or None where it is not built or the library was
    loaded from another path (``RPX_LIBRARY``): it links the library in its
    own directory, and a second copy of the library would not share its
    state. Callers fall back to the ctypes functions, which reach the same
    kernels."""

    global _FAST
    if _FAST is not None:
        return _FAST or None
    load()
    mod = False
    if FAST_PATH.exists() and Path(os.environ.get("RPX_LIBRARY", LIB_PATH)).resolve() == LIB_PATH:
        loader = importlib.machinery.ExtensionFileLoader("_rpxfast", str(FAST_PATH))
        spec = importlib.util.spec_from_file_location("_rpxfast", str(FAST_PATH), loader=loader)
        mod = importlib.util.module_from_spec(spec)
        loader.exec_module(mod)
    _FAST = mod
    return mod or None


def check(status: int) -> None:
    if status == RPX_OK:
        return
    msg = (load().rpx_last_error() or b"").decode(errors="replace")
    if status == RPX_ERR_INVALID:
        raise ValueError(msg)
    if status == RPX_ERR_DEVICE:
        raise DeviceError(msg)
    raise NativeError(msg)


def call(name: str, *args) -> None:
    check(getattr(load(), name)(*args))


def query(name: str, *args) -> int:
    return int(getattr(load(), name)(*args))
