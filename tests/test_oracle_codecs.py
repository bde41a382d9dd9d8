"""Pin the oracle's bf16 / fp8 codecs (CPU)."""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle.codecs import (
    E4M3FN,
    E5M2,
    bf16_bits_to_f32,
    f32_to_bf16_bits,
    fp8_decode,
    fp8_encode,
)

GOLDEN = Path(__file__).resolve().parent / "golden" / "codec_vectors.npz"


def _same_or_both_nan(a_codes, b_codes, fmt):
    a = fp8_decode(a_codes, fmt)
    b = fp8_decode(b_codes, fmt)
    return (a_codes == b_codes) | (np.isnan(a) & np.isnan(b))


def test_golden_vectors_bf16():
    g = np.load(GOLDEN, allow_pickle=False)
    got = f32_to_bf16_bits(g["x"])
    nan = np.isnan(g["x"])
    assert np.array_equal(got[~nan], g["bf16"][~nan])
    assert np.isnan(bf16_bits_to_f32(got[nan])).all()


@pytest.mark.parametrize("fmt", [E4M3FN, E5M2])
def test_golden_vectors_fp8(fmt):
    g = np.load(GOLDEN, allow_pickle=False)
    got = fp8_encode(g["x"], fmt)
    assert _same_or_both_nan(got, g[fmt], fmt).all()
    dec = g[f"dec_{fmt}"]
    mine = fp8_decode(np.arange(256, dtype=np.uint8), fmt)
    assert np.array_equal(np.isnan(mine), np.isnan(dec))
    assert np.array_equal(mine[~np.isnan(mine)], dec[~np.isnan(dec)])


@pytest.mark.parametrize("fmt,td", [(E4M3FN, torch.float8_e4m3fn), (E5M2, torch.float8_e5m2)])
def test_fp8_encode_matches_torch_on_every_bf16_value(fmt, td):
    x = bf16_bits_to_f32(np.arange(65536, dtype=np.uint32).astype(np.uint16))
    want = torch.from_numpy(x.copy()).to(td).view(torch.uint8).numpy()
    assert _same_or_both_nan(fp8_encode(x, fmt), want, fmt).all()


@pytest.mark.parametrize("fmt,td", [(E4M3FN, torch.float8_e4m3fn), (E5M2, torch.float8_e5m2)])
def test_fp8_encode_matches_torch_on_random_f32(fmt, td):
    rng = np.random.Generator(np.random.PCG64(11))
    x = rng.integers(0, 2**32, size=1_000_000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    want = torch.from_numpy(x.copy()).to(td).view(torch.uint8).numpy()
    assert _same_or_both_nan(fp8_encode(x, fmt), want, fmt).all()


def test_bf16_matches_torch_on_random_f32():
    rng = np.random.Generator(np.random.PCG64(12))
    x = rng.integers(0, 2**32, size=1_000_000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    want = torch.from_numpy(x.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    got = f32_to_bf16_bits(x)
    ok = ~np.isnan(x)
    assert np.array_equal(got[ok], want[ok])


def test_fp8_closed_form_values():
    """OCP FP8 spec values, independent of any conversion routine."""

    e4 = fp8_decode(np.arange(256, dtype=np.uint8), E4M3FN)
    assert e4[0x7E] == 448.0 and e4[0x01] == 2.0 ** -9 and e4[0x08] == 2.0 ** -6
    assert np.isnan(e4[0x7F]) and np.isnan(e4[0xFF]) and e4[0x80] == 0.0
    assert np.isfinite(e4[[c for c in range(256) if c & 0x7F != 0x7F]]).all()
    e5 = fp8_decode(np.arange(256, dtype=np.uint8), E5M2)
    assert e5[0x7B] == 57344.0 and e5[0x01] == 2.0 ** -16 and e5[0x04] == 2.0 ** -14
    assert e5[0x7C] == np.inf and e5[0xFC] == -np.inf and np.isnan(e5[0x7D])
    # round trip of every finite code
    for fmt, table in ((E4M3FN, e4), (E5M2, e5)):
        finite = np.isfinite(table)
        codes = np.arange(256, dtype=np.uint8)[finite]
        back = fp8_encode(table[finite], fmt)
        zero = table[finite] == 0
        assert np.array_equal(back[~zero], codes[~zero])


def test_fp8_ties_round_to_even():
    # e4m3: 1 + 1/16 lies halfway between 1.0 (mantissa 000) and 1.125 (001)
    assert fp8_encode(np.float32(1.0625), E4M3FN) == 0x38
    assert fp8_encode(np.float32(1.1875), E4M3FN) == 0x3A  # between 001 and 010 -> 010
    # overflow: 464 is the tie between 448 and the NaN slot -> 448; above -> NaN
    assert fp8_encode(np.float32(464.0), E4M3FN) == 0x7E
    assert fp8_encode(np.float32(465.0), E4M3FN) == 0x7F
    assert fp8_encode(np.float32(61440.0), E5M2) == 0x7C
    assert fp8_encode(np.float32(61439.0), E5M2) == 0x7B
    # half the smallest subnormal rounds to zero (even), just above rounds up
    assert fp8_encode(np.float32(2.0 ** -10), E4M3FN) == 0x00
    assert fp8_encode(np.nextafter(np.float32(2.0 ** -10), np.float32(1)), E4M3FN) == 0x01
    assert fp8_encode(np.float32(-0.0), E5M2) == 0x80


def test_bf16_rne_closed_form():
    # 1 + 2^-8 is the tie between 1.0 and 1 + 2^-7: even -> 1.0
    assert f32_to_bf16_bits(np.float32(1.0 + 2.0 ** -8)) == 0x3F80
    assert f32_to_bf16_bits(np.float32(1.0 + 3 * 2.0 ** -8)) == 0x3F82
    assert f32_to_bf16_bits(np.float32(np.finfo(np.float32).max)) == 0x7F80  # overflow -> inf
