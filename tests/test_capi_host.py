"""The C-ABI library on the host: exports, validation, and the device
quantizer run through its host hook (CPU only, no kernel launches)."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

from oracle import fp8 as ofp8
from oracle.codecs import bf16_bits_to_f32
from representax_amd import _native as nat

HEADER = Path(__file__).resolve().parents[1] / "include" / "representax_amd.h"


def _declared() -> list[str]:
    text = HEADER.read_text()
    return sorted(set(re.findall(r"\b(rpx_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = nat.load()
    names = _declared()
    assert len(names) >= 15
    for name in names:
        assert hasattr(lib, name), name
    assert set(names) <= set(nat.SIGNATURES), set(names) - set(nat.SIGNATURES)


def test_abi_version_matches_header():
    m = re.search(r"#define RPX_ABI_VERSION (\d+)", HEADER.read_text())
    assert nat.load().rpx_abi_version() == int(m.group(1))


def test_workspace_queries():
    lib = nat.load()
    assert lib.rpx_int4lora_forward_workspace(4096, 3072, 768, 0, 16, nat.DTYPE_BF16) == 0
    assert lib.rpx_int4lora_backward_workspace(4096, 3072, 768, 0, 16, nat.DTYPE_BF16) > 768 * 3072 * 2
    assert lib.rpx_int4lora_forward_workspace(4, 6, 8, 0, 2, nat.DTYPE_BF16) > 0  # generic path
    assert lib.rpx_fp8_linear_forward_workspace(8192, 3072, 768) >= 8192 * 768 + 3072 * 768
    # gradient codes [M, N] plus both operands' codes
    assert lib.rpx_fp8_linear_backward_workspace(8192, 3072, 768) >= 8192 * 3072 + 768 * 3072 + 8192 * 768


def test_invalid_arguments_are_rejected_before_any_launch():
    p = ctypes.c_void_p(16)  # never dereferenced: validation fails first
    with pytest.raises(ValueError, match="group_size"):
        nat.call("rpx_int4_dequant", p, p, 4, 8, 3, p, None)
    with pytest.raises(ValueError, match="rank"):
        nat.call("rpx_int4lora_forward", p, nat.DTYPE_BF16, 2, 8, p, p, 6, 0, None, p, p, 7,
                 ctypes.c_float(1.0), p, p, None, 0, None)
    with pytest.raises(ValueError, match="dtype"):
        nat.call("rpx_int4_pack", p, 7, 4, 8, 0, p, p, None)
    with pytest.raises(ValueError, match="format"):
        nat.call("rpx_fp8_cast", p, nat.DTYPE_BF16, 4, 4, 4, 1, p, 9, p, None, None)
    with pytest.raises(ValueError, match="slot"):
        nat.call("rpx_fp8_cast_delayed", p, nat.DTYPE_BF16, 4, 4, 4, 1, nat.FP8_E4M3FN, p, p, 3, 3,
                 p, None, None)
    with pytest.raises(ValueError, match="null scale state"):
        nat.call("rpx_fp8_cast_delayed", p, nat.DTYPE_BF16, 4, 4, 4, 1, nat.FP8_E4M3FN, None, p,
                 3, 0, p, None, None)
    with pytest.raises(ValueError, match="slot"):
        nat.call("rpx_fp8_cast_delayed2", p, 4, 4, 4, 1, 0, p, None, p, 4, 4, 4, 1, 5, p, None,
                 nat.DTYPE_BF16, nat.FP8_E4M3FN, p, p, 3, None)
    with pytest.raises(ValueError, match="history row"):
        nat.call("rpx_fp8_scale_update", p, p, p, p, p, 3, 0, None)
    assert nat.query("rpx_fp8_delayed_pending_words") >= 64
    with pytest.raises(ValueError, match="unknown activation"):
        nat.call("rpx_int4lora_forward_act", p, nat.DTYPE_BF16, 2, 8, p, p, 6, 0, None, p, p, 2,
                 ctypes.c_float(1.0), 9, None, p, p, p, None, 0, None)
    with pytest.raises(ValueError, match="bf16"):
        nat.call("rpx_int4lora_forward_act", p, nat.DTYPE_F32, 2, 8, p, p, 6, 0, None, p, p, 2,
                 ctypes.c_float(1.0), nat.ACT_GELU, None, p, p, p, None, 0, None)
    with pytest.raises(ValueError, match="null pointer"):
        nat.call("rpx_int4lora_forward_act", p, nat.DTYPE_BF16, 2, 8, p, p, 6, 0, None, p, p, 2,
                 ctypes.c_float(1.0), nat.ACT_SILU_MUL, None, p, p, p, None, 0, None)
    with pytest.raises(ValueError, match="null pointer"):
        nat.call("rpx_int4lora_backward_act", p, p, nat.DTYPE_BF16, 2, 8, p, p, 6, 0, p, p, 2,
                 ctypes.c_float(1.0), p, nat.ACT_SILU_MUL, p, p, p, None, p, p, None, 0, None)
    with pytest.raises(ValueError, match="rank"):
        nat.call("rpx_int4lora_backward_act", p, p, nat.DTYPE_BF16, 2, 8, p, p, 6, 0, p, p, 7,
                 ctypes.c_float(1.0), p, nat.ACT_GELU, p, None, p, None, p, p, None, 0, None)
    with pytest.raises(ValueError, match="alias"):
        nat.call("rpx_int4lora_backward_act", p, p, nat.DTYPE_BF16, 2, 8, p, p, 6, 0, p, p, 2,
                 ctypes.c_float(1.0), p, nat.ACT_ADD, p, None, p, None, p, p, None, 0, None)
    with pytest.raises(ValueError, match="null pointer"):
        nat.call("rpx_fp8_linear_backward_gemms", p, None, p, p, p, p, 256, 256, 256, p, p, 1,
                 nat.DTYPE_BF16, p, 1 << 30, None)
    with pytest.raises(ValueError, match="null pointer"):
        nat.call("rpx_fp8_linear_backward_gemms", p, p, None, p, p, p, 256, 256, 256, p, p, 1,
                 nat.DTYPE_BF16, p, 1 << 30, None)
    with pytest.raises(ValueError, match="workspace too small"):
        need = nat.load().rpx_fp8_linear_backward_gemms_workspace(8192, 768, 768)
        assert need > 0  # the 768 x 768 weight gradient over 8192 tokens is split-K
        nat.call("rpx_fp8_linear_backward_gemms", p, p, p, p, p, p, 8192, 768, 768, p, p, 1,
                 nat.DTYPE_BF16, p, need - 1, None)


def _host_quantize(x: np.ndarray, scale: float, fmt: int) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(x.size, np.uint8)
    nat.call("rpx_host_fp8_quantize", ctypes.c_void_p(x.ctypes.data), x.size,
             ctypes.c_float(scale), fmt, ctypes.c_void_p(out.ctypes.data))
    return out.reshape(x.shape)


@pytest.mark.parametrize("fmt,name", [(nat.FP8_E4M3FN, "e4m3fn"), (nat.FP8_E5M2, "e5m2")])
def test_device_quantizer_on_host_matches_oracle(fmt, name):
    """The kernels' divide (one Newton correction) and integer fp8 encoder,
    compiled for the host: bit-exact against an IEEE divide plus the oracle's
    encoder, for every bf16 value and many scales."""

    x = bf16_bits_to_f32(np.arange(65536, dtype=np.uint32).astype(np.uint16))
    rng = np.random.Generator(np.random.PCG64(1))
    scales = [1.0, 1.17549435e-38, 1e-30, 1e30, 3e38, 0.1, 3.0]
    scales += list((10.0 ** rng.uniform(-38, 38, 60)).astype(np.float32))
    for s in scales:
        s = np.float32(s)
        assert np.array_equal(_host_quantize(x, s, fmt), ofp8.cast_with_scale(x, s, name)), s


def test_device_quantizer_on_host_random_f32():
    rng = np.random.Generator(np.random.PCG64(2))
    x = rng.integers(0, 2**32, size=400_000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    for s in (np.float32(1e-3), np.float32(2.5), np.float32(7e4)):
        for fmt, name in ((nat.FP8_E4M3FN, "e4m3fn"), (nat.FP8_E5M2, "e5m2")):
            assert np.array_equal(_host_quantize(x, s, fmt), ofp8.cast_with_scale(x, s, name))


def test_fp8_linear_forward_rejects_empty_operands():
    """The reference's dynamic scale takes jnp.max over the operand, which
    raises on an empty array (precision.py:133-137); the C-ABI refuses an
    empty operand before any launch."""

    p = ctypes.c_void_p(16)
    for m, k, n in ((0, 8, 8), (8, 0, 8), (8, 8, 0)):
        with pytest.raises(ValueError, match="empty operand"):
            nat.call("rpx_fp8_linear_forward", p, nat.DTYPE_BF16, m, k, p, nat.DTYPE_BF16, n, n, 1,
                     p, nat.DTYPE_BF16, p, None, None, p, 1 << 20, None)


def test_fast_binding_shares_the_library_and_validates():
    """The CPython fast-call binding (small-M forward) is built next to the
    library, sees the same loaded instance (a knob set through ctypes reads
    back through it), sizes workspaces as the C ABI does, and passes invalid
    arguments through to the library's own validation."""

    fast = nat.fast()
    assert fast is not None
    lib = nat.load()
    old = lib.rpx_get_tuning(nat.TUNE_GEMM_BAND)
    try:
        assert lib.rpx_set_tuning(nat.TUNE_GEMM_BAND, 5) == 0
        assert fast.get_tuning(nat.TUNE_GEMM_BAND) == 5
    finally:
        lib.rpx_set_tuning(nat.TUNE_GEMM_BAND, old)
    for shape in [(1, 6144, 2048, 64, 32), (4, 2048, 6144, 0, 32), (4096, 3072, 768, 0, 16),
                  (4, 6, 8, 0, 2)]:
        assert fast.int4lora_forward_workspace(*shape, nat.DTYPE_BF16) == \
            lib.rpx_int4lora_forward_workspace(*shape, nat.DTYPE_BF16)
    p = 16  # never dereferenced: validation fails first
    with pytest.raises(ValueError, match="rank"):
        nat.check(fast.int4lora_forward(p, nat.DTYPE_BF16, 2, 8, p, p, 6, 0, None, p, p, 7, 1.0,
                                        p, p, None, 0, None))
    with pytest.raises(TypeError):
        fast.int4lora_forward(p, nat.DTYPE_BF16)
    with pytest.raises(ValueError):
        fast.int4lora_forward_multi(p, nat.DTYPE_BF16, 1, 8, (p,) * 10, None, 0, None)
    proj = (p, p, 6, 0, None, p, p, 7, 1.0, p, p)
    with pytest.raises(ValueError, match="rank"):
        nat.check(fast.int4lora_forward_multi(p, nat.DTYPE_BF16, 1, 8, proj * 2, None, 0, None))
    assert fast.int4lora_forward_multi_workspace(1, 2048, (p, p, 2048, 64, None, p, p, 32, 2.0, p,
                                                            p) * 3, nat.DTYPE_BF16) == \
        lib.rpx_int4lora_forward_multi_workspace(
            1, 2048, 3, (nat.Int4LoraProjection * 3)(*[nat.Int4LoraProjection(
                p, p, 2048, 64, None, p, p, 32, 2.0, p, p)] * 3), nat.DTYPE_BF16)
