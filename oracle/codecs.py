"""Bit-level bf16 and OCP fp8 codecs (numpy only).

Restates the dtype conversions the reference performs through JAX/ml_dtypes:
``astype(jnp.bfloat16)`` and ``bitcast_convert_type`` in
``src/representax/models/adapters.py:30-35``, and ``astype(float8_e4m3fn)`` /
``astype(float8_e5m2)`` in ``src/representax/precision.py:140``.

Every encoder rounds to nearest, ties to even, directly from float32. fp8
encoders are non-saturating like ml_dtypes: e4m3fn overflow and infinities
become NaN (0x7F|sign), e5m2 overflow becomes infinity.
"""

from __future__ import annotations

import numpy as np

# OCP fp8 formats: (exponent bits, mantissa bits, bias, has_inf, max_finite)
E4M3FN = "e4m3fn"
E5M2 = "e5m2"
_FORMATS = {
    E4M3FN: (4, 3, 7, False, 448.0),
    E5M2: (5, 2, 15, True, 57344.0),
}
FP8_MAX = {E4M3FN: 448.0, E5M2: 57344.0}
FLT_MIN = np.float32(np.finfo(np.float32).tiny)


def f32_bits(x) -> np.ndarray:
    """float32 bit patterns (same shape, including 0-d)."""

    return np.array(x, dtype=np.float32, copy=True).view(np.uint32)


def bits_f32(u) -> np.ndarray:
    return np.array(u, dtype=np.uint32, copy=True).view(np.float32)


def f32_to_bf16_bits(x) -> np.ndarray:
    """float32 -> bf16 bit pattern, round to nearest even.

    NaN maps to a quiet NaN that keeps the sign and top payload bits.
    """

    u = f32_bits(x).astype(np.uint64)
    is_nan = (u & 0x7FFFFFFF) > 0x7F800000
    rounded = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    out = np.where(is_nan, (u >> 16) | 0x0040, rounded)
    return (out & 0xFFFF).astype(np.uint16)


def bf16_bits_to_f32(b) -> np.ndarray:
    b = np.asarray(b, dtype=np.uint16).astype(np.uint32)
    return bits_f32(b << 16)


def bf16_round(x) -> np.ndarray:
    """Round float32 (or float64, first rounded to float32) to bf16 values."""

    return bf16_bits_to_f32(f32_to_bf16_bits(np.asarray(x, dtype=np.float32)))


def _fp8_decode_table(fmt: str) -> np.ndarray:
    ebits, mbits, bias, has_inf, _ = _FORMATS[fmt]
    table = np.zeros(256, dtype=np.float32)
    for code in range(256):
        sign = -1.0 if code & 0x80 else 1.0
        exp = (code >> mbits) & ((1 << ebits) - 1)
        mant = code & ((1 << mbits) - 1)
        all_ones = (1 << ebits) - 1
        if has_inf and exp == all_ones:
            value = np.inf if mant == 0 else np.nan
        elif not has_inf and exp == all_ones and mant == (1 << mbits) - 1:
            value = np.nan
        elif exp == 0:
            value = mant * 2.0 ** (1 - bias - mbits)
        else:
            value = (1.0 + mant / (1 << mbits)) * 2.0 ** (exp - bias)
        table[code] = sign * value
    return table


_DECODE = {fmt: _fp8_decode_table(fmt) for fmt in _FORMATS}


def fp8_decode(codes, fmt: str) -> np.ndarray:
    """fp8 code (uint8) -> float32 value (exact)."""

    return _DECODE[fmt][np.asarray(codes, dtype=np.uint8)]


def fp8_encode(x, fmt: str) -> np.ndarray:
    """float32 -> fp8 code, round to nearest even, non-saturating."""

    ebits, mbits, bias, has_inf, fmax = _FORMATS[fmt]
    x32 = np.asarray(x, dtype=np.float32)
    u = f32_bits(x32)
    sign = ((u >> 31) & 1).astype(np.uint8) << 7
    is_nan = np.isnan(x32)
    is_inf = np.isinf(x32)
    a = np.abs(np.where(is_nan, 0, x32).astype(np.float64))
    emin = 1 - bias
    safe = np.where(is_inf | (a == 0), 1.0, a)
    _, e2 = np.frexp(safe)  # safe = f * 2**e2 with f in [0.5, 1)
    e = e2.astype(np.int64) - 1  # unbiased exponent of the leading bit
    q_exp = np.maximum(e, emin) - mbits  # exponent of one unit in the last place
    units = np.rint(np.ldexp(safe, -q_exp))  # exact scaling; rint is half-even
    value = np.ldexp(units, q_exp)
    _, ev2 = np.frexp(value)
    ev = ev2.astype(np.int64) - 1
    subnormal = ev < emin
    exp_field = np.where(subnormal, 0, ev + bias)
    mant_field = np.where(
        subnormal,
        np.ldexp(value, -(emin - mbits)),
        np.ldexp(value, -(ev - mbits)) - (1 << mbits),
    )
    code = (exp_field.astype(np.int64) << mbits) | mant_field.astype(np.int64)
    overflow = value > fmax
    if has_inf:
        special_inf = (((1 << ebits) - 1) << mbits)
        special_nan = special_inf | ((1 << mbits) - 1)
        code = np.where(overflow | is_inf, special_inf, code)
        code = np.where(is_nan, special_nan, code)
    else:
        nan_code = 0x7F
        code = np.where(overflow | is_inf | is_nan, nan_code, code)
    underflow = ((a == 0) | (value == 0)) & ~is_nan & ~is_inf
    code = np.where(underflow, 0, code)
    return (code.astype(np.uint8) | sign).astype(np.uint8)


__all__ = [
    "E4M3FN",
    "E5M2",
    "FLT_MIN",
    "FP8_MAX",
    "bf16_bits_to_f32",
    "bf16_round",
    "bits_f32",
    "f32_bits",
    "f32_to_bf16_bits",
    "fp8_decode",
    "fp8_encode",
]
