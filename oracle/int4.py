"""Signed symmetric INT4 packer and unpacker (numpy restatement).

Follows ``src/representax/models/adapters.py:38-65`` (``_pack_int4_rows``) and
``adapters.py:68-79`` (``_unpack_int4_rows``). The reference uses one bf16
scale per output row (``group_size=None`` here). ``group_size=G`` applies the
same formula independently to each run of G input columns, giving scales of
shape ``[*, N, K/G]``; that layout is an extension with no reference
counterpart.
"""

from __future__ import annotations

import numpy as np

from .codecs import bf16_bits_to_f32, f32_to_bf16_bits, bf16_round


def _groups(k: int, group_size: int | None) -> int:
    if group_size is None:
        return 1
    if group_size <= 0 or k % group_size:
        raise ValueError("group_size must divide the input size")
    return k // group_size


def pack_int4(weight, group_size: int | None = None):
    """Quantize ``weight[*, N, K]`` (float32 or bf16-valued) to packed INT4.

    Returns ``(packed uint8[*, N, ceil(K/2)], scale_bits uint16[*, N])`` for
    the per-row scheme or ``scale_bits uint16[*, N, K/G]`` for groups.
    Steps (adapters.py:47-65): ``w_b = bf16(w)``; ``m = max|w_b|`` over the
    row (or group); ``s = bf16(m / 7)`` in float32, or 1.0 when ``m`` is not
    positive; ``q = clip(rint(bf16(w_b / s)), -7, 7)``; nibble ``q & 0xF``;
    low nibble holds the even column; odd K pads a zero high nibble.
    """

    w = np.asarray(weight, dtype=np.float32)
    *stack, n, k = w.shape
    ng = _groups(k, group_size)
    gs = k // ng
    w_b = bf16_round(w)
    grouped = w_b.reshape(*stack, n, ng, gs)
    maximum = np.max(np.abs(grouped), axis=-1).astype(np.float32)
    with np.errstate(invalid="ignore", divide="ignore"):
        quotient = (maximum / np.float32(7.0)).astype(np.float32)
    scale = bf16_round(np.where(maximum > 0, quotient, np.float32(1.0)))
    with np.errstate(invalid="ignore", divide="ignore"):
        t = bf16_round(grouped / scale[..., None])
    q = np.clip(np.rint(t), -7, 7)
    q = np.nan_to_num(q, nan=0.0).astype(np.int8).reshape(*stack, n, k)
    u = (q.astype(np.int16) & 0x0F).astype(np.uint8)
    if k % 2:
        u = np.concatenate([u, np.zeros((*stack, n, 1), np.uint8)], axis=-1)
    pairs = u.reshape(*stack, n, -1, 2)
    packed = (pairs[..., 0] | (pairs[..., 1] << 4)).astype(np.uint8)
    scale_bits = f32_to_bf16_bits(scale)
    if group_size is None:
        scale_bits = scale_bits[..., 0]
    return packed, scale_bits


def unpack_nibbles(packed, input_size: int) -> np.ndarray:
    """Packed bytes -> signed int8 values ``[*, N, K]`` (adapters.py:73-77).

    Low nibble first; nibbles >= 8 decode as ``u - 16`` (so 0x8 gives -8,
    although the packer never emits it).
    """

    p = np.asarray(packed, dtype=np.uint8)
    low = p & 0x0F
    high = p >> 4
    u = np.stack((low, high), axis=-1).reshape(*p.shape[:-1], -1)[..., :input_size]
    u = u.astype(np.int8)
    return np.where(u < 8, u, u - 16).astype(np.int8)


def dequant_int4_bits(packed, scale_bits, input_size: int, group_size: int | None = None):
    """Dequantized weight as bf16 bit patterns ``uint16[*, N, K]``.

    ``bf16(f32(q) * f32(s))``: the float32 product is exact, so this is one
    round-to-nearest-even (adapters.py:78-79).
    """

    q = unpack_nibbles(packed, input_size).astype(np.float32)
    s = bf16_bits_to_f32(scale_bits)
    if group_size is None:
        s_full = s[..., None]
        prod = q * s_full
    else:
        ng = _groups(input_size, group_size)
        *stack, n, k = q.shape
        prod = (q.reshape(*stack, n, ng, group_size) * s[..., None]).reshape(*stack, n, k)
    return f32_to_bf16_bits(prod.astype(np.float32))


def dequant_int4(packed, scale_bits, input_size: int, group_size: int | None = None):
    """Dequantized weight as float32 values equal to the bf16 result."""

    return bf16_bits_to_f32(dequant_int4_bits(packed, scale_bits, input_size, group_size))


__all__ = ["dequant_int4", "dequant_int4_bits", "pack_int4", "unpack_nibbles"]
