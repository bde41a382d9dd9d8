"""Pin the oracle's INT4 packer / unpacker with hand-built known answers (CPU)."""

from __future__ import annotations

import numpy as np

from oracle import int4 as oint4
from oracle.codecs import bf16_bits_to_f32, bf16_round


def test_hand_built_row():
    # max |w| = 7 -> scale exactly 1.0 -> q = w; -1 is nibble 0xF; odd K pads.
    w = np.array([[1.0, -1.0, 0.0, 7.0, -7.0]], np.float32)
    packed, scales = oint4.pack_int4(w)
    assert scales.tolist() == [0x3F80]
    assert packed.tolist() == [[0xF1, 0x70, 0x09]]
    assert oint4.dequant_int4(packed, scales, 5).tolist() == w.tolist()


def test_zero_row_gets_unit_scale_and_zero_nibbles():
    packed, scales = oint4.pack_int4(np.zeros((2, 6), np.float32))
    assert scales.tolist() == [0x3F80, 0x3F80]
    assert not packed.any()


def test_ties_round_half_to_even():
    # scale 1.0 (max 7); 2.5 -> 2, 3.5 -> 4, -2.5 -> -2, 0.5 -> 0, 1.5 -> 2
    w = np.array([[7.0, 2.5, 3.5, -2.5, 0.5, 1.5]], np.float32)
    packed, scales = oint4.pack_int4(w)
    q = oint4.unpack_nibbles(packed, 6)
    assert q.tolist() == [[7, 2, 4, -2, 0, 2]]


def test_scale_is_bf16_of_max_over_seven():
    w = np.array([[0.3, -1.1, 0.9]], np.float32)
    _, scales = oint4.pack_int4(w)
    m = np.float32(bf16_round(np.float32(1.1)))
    assert bf16_bits_to_f32(scales)[0] == bf16_round(np.float32(m / np.float32(7.0)))


def test_unpack_every_byte_value():
    packed = np.arange(256, dtype=np.uint8)[None, :]
    q = oint4.unpack_nibbles(packed, 512)[0]
    for b in range(256):
        lo, hi = b & 0xF, b >> 4
        assert q[2 * b] == (lo if lo < 8 else lo - 16)
        assert q[2 * b + 1] == (hi if hi < 8 else hi - 16)


def test_dequant_is_one_rounding_of_exact_product():
    rng = np.random.Generator(np.random.PCG64(3))
    scales = rng.integers(0, 0x7F80, size=64, dtype=np.uint16)
    packed = rng.integers(0, 256, size=(64, 40), dtype=np.uint8)
    got = oint4.dequant_int4(packed, scales, 80)
    q = oint4.unpack_nibbles(packed, 80).astype(np.float64)
    exact = q * bf16_bits_to_f32(scales).astype(np.float64)[:, None]
    assert np.array_equal(got, bf16_round(exact.astype(np.float32)))


def test_round_trip_error_bound():
    rng = np.random.Generator(np.random.PCG64(4))
    w = (rng.standard_normal((128, 256)) * 0.02).astype(np.float32)
    for group in (None, 64):
        packed, scales = oint4.pack_int4(w, group)
        deq = oint4.dequant_int4(packed, scales, 256, group)
        s = bf16_bits_to_f32(scales)
        s_full = s[:, None] if group is None else np.repeat(s, group, axis=1)
        # half a step, plus the bf16 roundings of w, of the quotient (which can
        # move it across a half-integer: |t| <= 7.03) and of q*s (|q| <= 7); a bf16
        # rounding moves a value by at most 2^-8 of its magnitude
        bound = s_full * (0.5 + 14.1 * 2.0 ** -8) + np.abs(w) * 2.0 ** -8
        assert (np.abs(deq - w) <= bound).all()
        assert (np.abs(oint4.unpack_nibbles(packed, 256)) <= 7).all()


def test_group_scheme_equals_rows_of_groups():
    """Group-G packing == the reference's per-row packer on rows of length G."""

    rng = np.random.Generator(np.random.PCG64(5))
    w = rng.standard_normal((12, 128)).astype(np.float32)
    packed_g, scales_g = oint4.pack_int4(w, 32)
    packed_r, scales_r = oint4.pack_int4(w.reshape(12 * 4, 32))
    assert np.array_equal(scales_g.reshape(-1), scales_r)
    assert np.array_equal(packed_g.reshape(-1), packed_r.reshape(-1))


def test_stacked_weights_pack_per_layer():
    rng = np.random.Generator(np.random.PCG64(6))
    w = rng.standard_normal((3, 8, 10)).astype(np.float32)
    packed, scales = oint4.pack_int4(w)
    assert packed.shape == (3, 8, 5) and scales.shape == (3, 8)
    for i in range(3):
        p, s = oint4.pack_int4(w[i])
        assert np.array_equal(p, packed[i]) and np.array_equal(s, scales[i])


def test_reference_test_sizes():
    """The reference test packs a [6, 8] weight into 24 bytes of uint8 and
    uint16 scales (tests/models/test_adapters.py:82-84)."""

    packed, scales = oint4.pack_int4(np.ones((6, 8), np.float32))
    assert packed.dtype == np.uint8 and packed.size == 6 * 4
    assert scales.dtype == np.uint16
