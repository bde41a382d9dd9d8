"""INT4-base + LoRA linear: forward and backward restatement (numpy).

Forward follows ``src/representax/models/adapters.py:158-182``
(``QuantizedLoRALinear.__call__``) with the casts of
``src/representax/precision.py:102-124``: under a bf16 policy the fp32 LoRA
masters are viewed as bf16, every dot accumulates in float32 (here: float64
or float32, chosen by ``acc``) and rounds its output to bf16, and the Python
float ``alpha / rank`` is a weakly typed scalar, so it is first rounded to the
operand dtype.

The backward is JAX's transpose of that forward (the reference has no
hand-written VJP for this path): with ``c = dtype(alpha / rank)``

* ``g_a = rnd(g * c)``, ``dh = rnd(g_a @ B)``
* ``dB = f32(rnd(g_a^T @ h))``
* ``dx = rnd(rnd(g @ W) + rnd(dh @ A))``
* ``dA = f32(rnd(dh^T @ x))``

where ``rnd`` rounds to the compute dtype. The packed base and the bias are
integer leaves and receive no gradient.
"""

from __future__ import annotations

import numpy as np

from .codecs import bf16_bits_to_f32, bf16_round
from .int4 import dequant_int4


def _rounder(compute: str):
    """Rounding applied after every op in the given compute dtype; "f64" keeps
    float64 throughout (used to check the transpose rules against finite
    differences)."""

    if compute == "bf16":
        return bf16_round
    if compute == "f32":
        return lambda v: np.asarray(v, dtype=np.float32)
    if compute == "f64":
        return lambda v: np.asarray(v, dtype=np.float64)
    raise ValueError(compute)


def _master(v, compute: str):
    return np.asarray(v, dtype=np.float64 if compute == "f64" else np.float32)


def _dot(a, b, acc):
    return np.asarray(a, dtype=acc) @ np.asarray(b, dtype=acc)


def lora_scaling(alpha: float, rank: int, compute: str = "bf16") -> np.float32:
    """``alpha / rank`` as the weakly typed scalar the reference multiplies by."""

    if compute == "f64":
        return np.float64(alpha / rank)
    return _rounder(compute)(np.float32(alpha / rank))


def lora_forward(
    x,
    packed,
    scale_bits,
    lora_a,
    lora_b,
    *,
    alpha: float,
    rank: int,
    bias_bits=None,
    group_size: int | None = None,
    compute: str = "bf16",
    acc=np.float64,
    weight=None,
):
    """Return ``(y, h)`` as float32 arrays holding compute-dtype values.

    ``x``: ``[M, K]`` values already in the compute dtype. ``lora_a``:
    ``[r, K]`` fp32 master; ``lora_b``: ``[N, r]`` fp32 master. ``weight``
    may pass a precomputed dequantized base ``[N, K]``.
    """

    rnd = _rounder(compute)
    x = rnd(x)
    k = x.shape[-1]
    w = dequant_int4(packed, scale_bits, k, group_size) if weight is None else weight
    a_c = rnd(lora_a)
    b_c = rnd(lora_b)
    base = rnd(_dot(x, w.T, acc))
    h = rnd(_dot(x, a_c.T, acc))
    a_out = rnd(_dot(h, b_c.T, acc))
    c = lora_scaling(alpha, rank, compute)
    y = rnd(base + rnd(a_out * c))
    if bias_bits is not None:
        y = rnd(y + rnd(bf16_bits_to_f32(bias_bits)))
    return y, h


def lora_backward(
    g,
    x,
    packed,
    scale_bits,
    lora_a,
    lora_b,
    h,
    *,
    alpha: float,
    rank: int,
    group_size: int | None = None,
    compute: str = "bf16",
    acc=np.float64,
    weight=None,
):
    """Return ``(dx, dA, dB)``: dx in the compute dtype, dA/dB as float32."""

    rnd = _rounder(compute)
    g = rnd(g)
    x = rnd(x)
    k = x.shape[-1]
    w = dequant_int4(packed, scale_bits, k, group_size) if weight is None else weight
    a_c = rnd(lora_a)
    b_c = rnd(lora_b)
    c = lora_scaling(alpha, rank, compute)
    g_a = rnd(g * c)
    dh = rnd(_dot(g_a, b_c, acc))
    d_b = _master(rnd(_dot(g_a.T, h, acc)), compute)
    dx = rnd(rnd(_dot(g, w, acc)) + rnd(_dot(dh, a_c, acc)))
    d_a = _master(rnd(_dot(dh.T, x, acc)), compute)
    return dx, d_a, d_b


def merged_weight(packed, scale_bits, lora_a, lora_b, *, alpha, rank, input_size, group_size=None):
    """``f32(W_b) + (B @ A) * (alpha / rank)`` in float32 (adapters.py:150-156)."""

    w = dequant_int4(packed, scale_bits, input_size, group_size)
    adapter = (np.asarray(lora_b, np.float32) @ np.asarray(lora_a, np.float32)).astype(np.float32)
    return (w + adapter * np.float32(alpha / rank)).astype(np.float32)


__all__ = ["lora_backward", "lora_forward", "lora_scaling", "merged_weight"]
