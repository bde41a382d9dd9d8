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
