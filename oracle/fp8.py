"""Dynamically scaled fp8 linear (numpy restatement).

Follows ``src/representax/precision.py``:

* ``_scaled_quantize`` (``:127-140``): ``s = max(max|f32(t)| / fmax, FLT_MIN)``
  with ``fmax`` 448 (e4m3fn) or 57344 (e5m2); ``q = f8(f32(t) / s)`` with an
  IEEE float32 divide and a round-to-nearest-even cast.
* ``_scaled_fp8_dot`` (``:143-170``): ``((sum_k q_l * q_r) * s_l) * s_r`` in
  float32. fp8 x fp8 products are exact in float32; the sum is taken in
  ``acc`` precision here.
* ``_fp8_linear_dot`` and its VJP (``:173-221``): e4m3 x e4m3 forward;
  backward ``dL = dot(g[e5m2], R^T[e4m3])``, ``dR = dot(L^T[e4m3], g[e5m2])``,
  each cast to the operand dtype.
* ``linear_matmul`` (``:224-239``): flatten leading dims, fp8 dot, cast to
  the activation dtype (bf16 under ``float8_mixed``).
"""

from __future__ import annotations

import numpy as np

from .codecs import E4M3FN, E5M2, FLT_MIN, FP8_MAX, bf16_round, fp8_decode, fp8_encode


def amax(t) -> np.float32:
    """``max|f32(t)|``; NaN anywhere gives NaN (XLA max propagates NaN)."""

    a = np.abs(np.asarray(t, dtype=np.float32))
    if a.size == 0:
        return np.float32(0.0)
    if np.isnan(a).any():
        return np.float32(np.nan)
    return np.float32(a.max())


def scale_from_amax(maximum, fmt: str) -> np.float32:
    """``max(amax / fmax, FLT_MIN)`` in float32 with NaN propagation."""

    with np.errstate(invalid="ignore", over="ignore"):
        ratio = np.float32(np.float32(maximum) / np.float32(FP8_MAX[fmt]))
    if np.isnan(ratio):
        return np.float32(np.nan)
    return np.float32(max(ratio, FLT_MIN))


def scaled_quantize(t, fmt: str):
    """Return ``(codes uint8, scale float32)``."""

    t32 = np.asarray(t, dtype=np.float32)
    s = scale_from_amax(amax(t32), fmt)
    return cast_with_scale(t32, s, fmt), s


def cast_with_scale(t, s, fmt: str) -> np.ndarray:
    """``f8(f32(t) / s)`` with one IEEE float32 divide per element."""

    with np.errstate(invalid="ignore", divide="ignore", over="ignore"):
        q = (np.asarray(t, dtype=np.float32) / np.float32(s)).astype(np.float32)
    return fp8_encode(q, fmt)


def scaled_dot_codes(qa, sa, fa, qb, sb, fb, acc=np.float64) -> np.ndarray:
    """``((qa @ qb) * sa) * sb`` from fp8 codes; ``qa [M,K]``, ``qb [K,N]``."""

    va = fp8_decode(qa, fa).astype(acc)
    vb = fp8_decode(qb, fb).astype(acc)
    with np.errstate(invalid="ignore", over="ignore"):
        out = (va @ vb).astype(np.float32)
        out = (out * np.float32(sa)).astype(np.float32)
        out = (out * np.float32(sb)).astype(np.float32)
    return out


def scaled_fp8_dot(left, right, fmt_left: str, fmt_right: str, acc=np.float64):
    """float32 ``[M, N]`` result of ``_scaled_fp8_dot(left [M,K], right [K,N])``."""

    qa, sa = scaled_quantize(left, fmt_left)
    qb, sb = scaled_quantize(right, fmt_right)
    return scaled_dot_codes(qa, sa, fmt_left, qb, sb, fmt_right, acc)


def fp8_linear_forward(left, right, acc=np.float64):
    """``_fp8_linear_dot(left [M,K], right [K,N])`` -> float32 ``[M,N]``."""

    return scaled_fp8_dot(left, right, E4M3FN, E4M3FN, acc)


def fp8_linear_backward(left, right, g, acc=np.float64, operand_round=bf16_round):
    """Return ``(d_left [M,K], d_right [K,N])`` cast to the operand dtype."""

    g32 = np.asarray(g, dtype=np.float32)
    left = np.asarray(left, dtype=np.float32)
    right = np.asarray(right, dtype=np.float32)
    d_left = scaled_fp8_dot(g32, right.T, E5M2, E4M3FN, acc)
    d_right = scaled_fp8_dot(left.T, g32, E4M3FN, E5M2, acc)
    return operand_round(d_left), operand_round(d_right)


def linear_matmul_fp8(left, right, acc=np.float64):
    """fp8-policy ``linear_matmul``: flatten, fp8 dot, round to bf16."""

    left = np.asarray(left, dtype=np.float32)
    lead = left.shape[:-1]
    out = fp8_linear_forward(left.reshape(-1, left.shape[-1]), right, acc)
    return bf16_round(out).reshape(*lead, np.asarray(right).shape[-1])


# ---------------------------------------------------------------------------
# Delayed scaling (an extension: the reference's roadmap item, todo.org:
# 1149-1154 and docs/precision.md:67-71, which the reference has not built).
# A cast takes the scale its slot holds instead of computing one from the
# tensor, saturates at the format's largest finite value, and records the
# tensor's amax; once per step every slot's scale becomes
# scale_from_amax(max of its recorded amaxes), unless nothing nonzero was
# recorded. Pins: with a history holding exactly the tensor's own amax the
# saturating cast equals the reference's dynamic cast (no quotient then
# exceeds fmax: |t / s| <= amax / (amax / fmax) = fmax up to one rounding,
# which the encoder rounds back to fmax); saturation and the update rule
# follow from their closed forms.
# ---------------------------------------------------------------------------
def cast_saturating(t, s, fmt: str) -> np.ndarray:
    """``f8(clamp(f32(t) / s, -fmax, fmax))`` (NaN stays NaN)."""

    fmax = np.float32(FP8_MAX[fmt])
    with np.errstate(invalid="ignore", divide="ignore", over="ignore"):
        q = (np.asarray(t, dtype=np.float32) / np.float32(s)).astype(np.float32)
        q = np.where(np.abs(q) > fmax, np.copysign(fmax, q), q).astype(np.float32)
    return fp8_encode(q, fmt)


def delayed_update(history, scales, formats) -> np.ndarray:
    """New scales from recorded amaxes ``history [H, S]`` (float32; 0 =
    nothing recorded): ``scale_from_amax(max_h history[:, s])`` where that
    maximum is nonzero (NaN if any NaN), else the old scale."""

    h = np.asarray(history, dtype=np.float32)
    out = np.asarray(scales, dtype=np.float32).copy()
    for sl, fmt in enumerate(formats):
        col = h[:, sl]
        m = np.float32(np.nan) if np.isnan(col).any() else np.float32(col.max())
        if np.isnan(m) or m != 0:
            out[sl] = scale_from_amax(m, fmt)
    return out


__all__ = [
    "amax",
    "cast_saturating",
    "delayed_update",
    "cast_with_scale",
    "fp8_linear_backward",
    "fp8_linear_forward",
    "linear_matmul_fp8",
    "scale_from_amax",
    "scaled_dot_codes",
    "scaled_fp8_dot",
    "scaled_quantize",
]
