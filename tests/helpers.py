"""Shared helpers for the parity tests: seeded inputs and comparisons."""

from __future__ import annotations

import numpy as np
import torch

from oracle.codecs import bf16_bits_to_f32, f32_to_bf16_bits

DEVICE = "cuda:0"


def rng(seed: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(seed))


def bf16_values(a) -> np.ndarray:
    """float32 array holding the bf16-rounded values of ``a``."""

    return bf16_bits_to_f32(f32_to_bf16_bits(np.asarray(a, np.float32)))


def to_dev_bf16(a) -> torch.Tensor:
    bits = f32_to_bf16_bits(np.asarray(a, np.float32))
    return torch.from_numpy(bits.view(np.int16).copy()).to(DEVICE).view(torch.bfloat16)


def to_dev(a, dtype=None) -> torch.Tensor:
    t = torch.from_numpy(np.ascontiguousarray(a)).to(DEVICE)
    return t if dtype is None else t.to(dtype)


def from_dev(t: torch.Tensor) -> np.ndarray:
    if t.dtype == torch.bfloat16:
        bits = t.detach().view(torch.int16).cpu().numpy().view(np.uint16)
        return bf16_bits_to_f32(bits)
    if t.dtype == torch.uint16:
        return t.detach().view(torch.int16).cpu().numpy().view(np.uint16)
    return t.detach().cpu().numpy()


def bits_from_dev(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def rel_l2(actual, expected) -> float:
    a = np.asarray(actual, np.float64)
    e = np.asarray(expected, np.float64)
    denom = np.linalg.norm(e)
    if denom == 0:
        return float(np.linalg.norm(a))
    return float(np.linalg.norm(a - e) / denom)


def ulp_diff(a_bits: np.ndarray, b_bits: np.ndarray) -> np.ndarray:
    """Distance in bf16 units in the last place (same-sign finite values)."""

    def ordered(u):
        u = u.astype(np.int32)
        return np.where(u & 0x8000, 0x8000 - (u & 0x7FFF), 0x8000 + u)

    return np.abs(ordered(a_bits) - ordered(b_bits))


TINY = 1e-30  # below it f32 intermediates are subnormal; results only need to stay tiny


def assert_act_bits(got_bits: np.ndarray, want_f32: np.ndarray):
    """The activation is evaluated in f32 on the GPU (an erfc fit with
    fractional error < 1.2e-7, the hardware exp2 and reciprocal) and exactly
    in the oracle: identical bits except where the exact value sits within a
    few f32 ulps of a bf16 rounding boundary, and then one bf16 ulp. Results
    below 1e-30 in magnitude (f32 subnormal intermediates) must stay below it."""

    got_bits = got_bits.reshape(-1)
    want = np.asarray(want_f32, np.float32).reshape(-1)
    want_bits = f32_to_bf16_bits(want)
    got = (got_bits.astype(np.uint32) << 16).view(np.float32)
    tiny = np.abs(want) < TINY
    assert np.all(np.abs(got[tiny]) < TINY)
    d = ulp_diff(got_bits[~tiny], want_bits[~tiny])
    if d.size:
        i = int(np.argmax(d))
        assert d[i] <= 1, (d[i], float(got[~tiny][i]), float(want[~tiny][i]))
        assert np.mean(d > 0) < 1e-2


# Parity bars for bf16 outputs of the fp32-accumulating kernels against the
# oracle's float64 accumulation (the rounding points are the same; only
# results whose exact value sits next to a bf16 rounding boundary can differ,
# by one ulp).
BF16_REL_TOL = 2e-3
BF16_MIN_EQUAL = 0.99
# dA / dB reduce over every token (32,768 in the BERT step) in float32
# partials: about 1% of them land one ulp from the float64 oracle's value
BF16_MIN_EQUAL_TOKEN_SUM = 0.97


def assert_bf16_close(got: np.ndarray, want: np.ndarray, tol: float = BF16_REL_TOL,
                      min_equal: float | None = BF16_MIN_EQUAL, what: str = ""):
    """rel-L2 within ``tol`` and, when ``min_equal`` is given, at least that
    fraction of elements equal to the oracle's bf16 value. Outputs so small
    that the allowed fraction is under one element (fewer than 100 at 99%)
    may still differ in one element: a single rounding-boundary case there
    is the same event the fraction allows on larger outputs."""

    err = rel_l2(got, want)
    assert err < tol, (what, err)
    if min_equal is not None and np.size(want):
        same = np.asarray(got, np.float32) == np.asarray(want, np.float32)
        eq = float(np.mean(same))
        allowed = max(1, int(np.floor((1.0 - min_equal) * same.size)))
        assert eq >= min_equal or int(same.size - same.sum()) <= allowed, (what, eq)
