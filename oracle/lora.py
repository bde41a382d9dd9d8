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

``compute="promoted"`` is the reference without a precision policy on bf16
activations (``compute_parameter`` then returns the fp32 masters unchanged,
precision.py:111-117): the base product is bf16 x bf16 -> bf16, but
``jnp.matmul`` promotes bf16 x f32 to f32, so the adapter runs in float32 on
the unrounded masters and the sum (and the module output) is float32:

* ``base = bf16(x @ W^T)``, ``h = f32(x @ A^T)``, ``a = f32(h @ B^T)``
* ``y = f32(f32(base) + f32(a * c))`` with ``c = f32(alpha / rank)``,
  then ``y = f32(y + bias)``

and JAX's transpose of it, with ``g`` the float32 output cotangent:

* ``dx = bf16(bf16(bf16(g) @ W) + bf16(f32(dh @ A)))``, ``dh = f32(g_a @ B)``,
  ``g_a = f32(g * c)``
* ``dB = f32(g_a^T @ h)``, ``dA = f32(dh^T @ x)``

(the bf16 matmul's cotangent is bf16; the adapter's arrives through the
transpose of the bf16 -> f32 convert of x; the two are summed in bf16).
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
    if compute == "promoted":
        return lambda v: np.asarray(v, dtype=np.float32)
    raise ValueError(compute)


def _f32(v):
    return np.asarray(v, dtype=np.float32)


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

    if compute == "promoted":
        return _promoted_forward(x, packed, scale_bits, lora_a, lora_b, alpha, rank, bias_bits,
                                 group_size, acc, weight)
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
    dx_rows=None,
):
    """Return ``(dx, dA, dB)``: dx in the compute dtype, dA/dB as float32.

    ``dx_rows`` (an index array) restricts dx to those rows of the batch (dx
    is row-separable); dA and dB always reduce over the whole batch.
    """

    if compute == "promoted":
        return _promoted_backward(g, x, packed, scale_bits, lora_a, lora_b, h, alpha, rank,
                                  group_size, acc, weight, dx_rows)
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
    if dx_rows is not None:
        dx = rnd(rnd(_dot(g[dx_rows], w, acc)) + rnd(_dot(dh[dx_rows], a_c, acc)))
    else:
        dx = rnd(rnd(_dot(g, w, acc)) + rnd(_dot(dh, a_c, acc)))
    d_a = _master(rnd(_dot(dh.T, x, acc)), compute)
    return dx, d_a, d_b


def _promoted_forward(x, packed, scale_bits, lora_a, lora_b, alpha, rank, bias_bits, group_size,
                      acc, weight):
    x = bf16_round(x)
    k = x.shape[-1]
    w = dequant_int4(packed, scale_bits, k, group_size) if weight is None else weight
    a = _f32(lora_a)
    b = _f32(lora_b)
    c = np.float32(alpha / rank)
    base = bf16_round(_dot(x, w.T, acc))
    h = _f32(_dot(x, a.T, acc))
    a_out = _f32(_dot(h, b.T, acc))
    y = _f32(base + _f32(a_out * c))
    if bias_bits is not None:
        y = _f32(y + bf16_bits_to_f32(bias_bits))
    return y, h


def _promoted_backward(g, x, packed, scale_bits, lora_a, lora_b, h, alpha, rank, group_size, acc,
                       weight, dx_rows):
    g = _f32(g)
    x = bf16_round(x)
    k = x.shape[-1]
    w = dequant_int4(packed, scale_bits, k, group_size) if weight is None else weight
    a = _f32(lora_a)
    b = _f32(lora_b)
    c = np.float32(alpha / rank)
    g_a = _f32(g * c)
    dh = _f32(_dot(g_a, b, acc))
    d_b = _f32(_dot(g_a.T, h, acc))
    rows = slice(None) if dx_rows is None else dx_rows
    dx_base = bf16_round(_dot(bf16_round(g[rows]), w, acc))
    dx_adapter = bf16_round(_f32(_dot(dh[rows], a, acc)))
    dx = bf16_round(dx_base + dx_adapter)
    d_a = _f32(_dot(dh.T, x, acc))
    return dx, d_a, d_b


def merged_weight(packed, scale_bits, lora_a, lora_b, *, alpha, rank, input_size, group_size=None):
    """``f32(W_b) + (B @ A) * (alpha / rank)`` in float32 (adapters.py:150-156)."""

    w = dequant_int4(packed, scale_bits, input_size, group_size)
    adapter = (np.asarray(lora_b, np.float32) @ np.asarray(lora_a, np.float32)).astype(np.float32)
    return (w + adapter * np.float32(alpha / rank)).astype(np.float32)


__all__ = ["lora_backward", "lora_forward", "lora_scaling", "merged_weight"]
