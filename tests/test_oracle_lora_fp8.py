"""Pin the oracle's INT4-LoRA and FP8 linears against closed forms, brute
force and finite differences (CPU)."""

from __future__ import annotations

import numpy as np

from oracle import fp8 as ofp8
from oracle import int4 as oint4
from oracle import lora as olora
from oracle.codecs import E4M3FN, E5M2, FLT_MIN, bf16_bits_to_f32, bf16_round, f32_to_bf16_bits


def _case(m=5, k=8, n=6, r=2, seed=0):
    g = np.random.Generator(np.random.PCG64(seed))
    x = bf16_round(g.standard_normal((m, k)))
    w = (g.standard_normal((n, k)) * 0.3).astype(np.float32)
    a = (g.standard_normal((r, k)) * 0.3).astype(np.float32)
    b = (g.standard_normal((n, r)) * 0.3).astype(np.float32)
    packed, scales = oint4.pack_int4(w)
    bias = f32_to_bf16_bits(g.standard_normal(n).astype(np.float32))
    return x, packed, scales, a, b, bias


def test_forward_brute_force_loops():
    """Element-by-element loops with the documented rounding points."""

    x, packed, scales, a, b, bias = _case()
    alpha, r = 3.0, 2
    y, h = olora.lora_forward(x, packed, scales, a, b, alpha=alpha, rank=r, bias_bits=bias)
    w = oint4.dequant_int4(packed, scales, x.shape[1])
    ab, bb = bf16_round(a), bf16_round(b)
    c = float(bf16_round(np.float32(alpha / r)))
    m, k = x.shape
    n = w.shape[0]
    for i in range(m):
        hh = [float(bf16_round(np.float32(sum(float(x[i, t]) * float(ab[j, t]) for t in range(k)))))
              for j in range(r)]
        assert np.allclose(hh, h[i])
        for o in range(n):
            base = bf16_round(np.float32(sum(float(x[i, t]) * float(w[o, t]) for t in range(k))))
            ad = bf16_round(np.float32(sum(hh[j] * float(bb[o, j]) for j in range(r))))
            yy = bf16_round(np.float32(base + bf16_round(np.float32(ad * c))))
            yy = bf16_round(np.float32(yy + bf16_bits_to_f32(bias[o])))
            assert yy == y[i, o]


def test_zero_adapter_equals_base_projection():
    """lora_b = 0 (the reference's init) leaves exactly the base projection."""

    x, packed, scales, a, _, bias = _case(seed=1)
    y, _ = olora.lora_forward(x, packed, scales, a, np.zeros((6, 2), np.float32), alpha=4.0,
                              rank=2, bias_bits=bias)
    w = oint4.dequant_int4(packed, scales, 8)
    base = bf16_round(bf16_round(x.astype(np.float64) @ w.T.astype(np.float64)) +
                      bf16_bits_to_f32(bias))
    assert np.array_equal(y, base)


def test_forward_close_to_merged_weight():
    """Adapted output ~ x W_merged^T + bias (tests/models/test_adapters.py:77-94)."""

    x, packed, scales, a, b, bias = _case(m=16, k=32, n=24, r=4, seed=2)
    y, _ = olora.lora_forward(x, packed, scales, a, b, alpha=8.0, rank=4, bias_bits=bias,
                              compute="f32")
    merged = olora.merged_weight(packed, scales, a, b, alpha=8.0, rank=4, input_size=32)
    np.testing.assert_allclose(y, x @ merged.T + bf16_bits_to_f32(bias), rtol=2e-3, atol=2e-3)


def test_backward_matches_finite_differences():
    """The transpose rules (float64 mode) against central differences of
    L = sum(g * y) in x, A and B."""

    m, k, n, r = 4, 8, 6, 3
    x, packed, scales, a, b, _ = _case(m, k, n, r, seed=3)
    x = x.astype(np.float64)
    a = a.astype(np.float64)
    b = b.astype(np.float64)
    gy = np.random.Generator(np.random.PCG64(9)).standard_normal((m, n))
    kw = dict(alpha=2.5, rank=r, compute="f64")

    def loss(xx, aa, bb):
        y, _ = olora.lora_forward(xx, packed, scales, aa, bb, **kw)
        return float((gy * y).sum())

    _, h = olora.lora_forward(x, packed, scales, a, b, **kw)
    dx, da, db = olora.lora_backward(gy, x, packed, scales, a, b, h, **kw)
    eps = 1e-6
    for arr, grad, which in ((x, dx, 0), (a, da, 1), (b, db, 2)):
        num = np.zeros_like(arr)
        for idx in np.ndindex(arr.shape):
            plus = [x.copy(), a.copy(), b.copy()]
            minus = [x.copy(), a.copy(), b.copy()]
            plus[which][idx] += eps
            minus[which][idx] -= eps
            num[idx] = (loss(*plus) - loss(*minus)) / (2 * eps)
        np.testing.assert_allclose(grad, num, rtol=1e-6, atol=1e-8)


def test_bf16_backward_gradients_are_bf16_values():
    x, packed, scales, a, b, _ = _case(seed=4)
    gy = bf16_round(np.random.Generator(np.random.PCG64(5)).standard_normal((5, 6)))
    _, h = olora.lora_forward(x, packed, scales, a, b, alpha=4.0, rank=2)
    dx, da, db = olora.lora_backward(gy, x, packed, scales, a, b, h, alpha=4.0, rank=2)
    for t in (dx, da, db):
        assert np.array_equal(bf16_round(t), t)
    assert da.dtype == np.float32 and db.dtype == np.float32


def test_promoted_forward_brute_force_loops():
    """No policy, bf16 activations, fp32 masters: element-by-element loops
    with bf16 rounding of the base product only, float32 elsewhere."""

    x, packed, scales, a, b, bias = _case(seed=6)
    alpha, r = 3.0, 2
    y, h = olora.lora_forward(x, packed, scales, a, b, alpha=alpha, rank=r, bias_bits=bias,
                              compute="promoted")
    assert y.dtype == np.float32 and h.dtype == np.float32
    w = oint4.dequant_int4(packed, scales, x.shape[1])
    c = np.float32(alpha / r)
    m, k = x.shape
    n = w.shape[0]
    for i in range(m):
        hh = [np.float32(sum(float(x[i, t]) * float(a[j, t]) for t in range(k))) for j in range(r)]
        assert np.array_equal(np.asarray(hh, np.float32), h[i])
        for o in range(n):
            base = bf16_round(np.float32(sum(float(x[i, t]) * float(w[o, t]) for t in range(k))))
            ad = np.float32(sum(float(hh[j]) * float(b[o, j]) for j in range(r)))
            yy = np.float32(np.float32(base) + np.float32(ad * c))
            yy = np.float32(yy + bf16_bits_to_f32(bias[o]))
            assert yy == y[i, o]


def test_promoted_zero_adapter_equals_bf16_base():
    """lora_b = 0 and no bias: the float32 output holds exactly the bf16
    base product, the same values as under the bf16 policy."""

    x, packed, scales, a, _, _ = _case(seed=7)
    zero = np.zeros((6, 2), np.float32)
    y_p, _ = olora.lora_forward(x, packed, scales, a, zero, alpha=4.0, rank=2, compute="promoted")
    y_b, _ = olora.lora_forward(x, packed, scales, a, zero, alpha=4.0, rank=2)
    assert np.array_equal(y_p, y_b)


def test_promoted_backward_matches_float64_transpose():
    """The promoted backward against the float64 transpose (itself pinned by
    finite differences): dA and dB to float32 accuracy, dx to bf16
    accuracy, and dx holds bf16 values."""

    m, k, n, r = 7, 16, 12, 3
    x, packed, scales, a, b, _ = _case(m, k, n, r, seed=8)
    gy = np.random.Generator(np.random.PCG64(10)).standard_normal((m, n)).astype(np.float32)
    kw = dict(alpha=5.0, rank=r)
    _, h = olora.lora_forward(x, packed, scales, a, b, compute="promoted", **kw)
    dx, da, db = olora.lora_backward(gy, x, packed, scales, a, b, h, compute="promoted", **kw)
    _, h64 = olora.lora_forward(x, packed, scales, a, b, compute="f64", **kw)
    dx64, da64, db64 = olora.lora_backward(gy, x, packed, scales, a, b, h64, compute="f64", **kw)
    assert da.dtype == np.float32 and db.dtype == np.float32
    np.testing.assert_allclose(da, da64, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(db, db64, rtol=1e-5, atol=1e-6)
    assert np.array_equal(bf16_round(dx), dx)
    np.testing.assert_allclose(dx, dx64, rtol=2e-2, atol=2e-2)


def test_scaling_is_rounded_like_a_weak_scalar():
    assert olora.lora_scaling(32.0, 16) == 2.0
    assert olora.lora_scaling(1.0, 3) == bf16_round(np.float32(1 / 3))
    assert olora.lora_scaling(1.0, 3, "f32") == np.float32(1 / 3)


# ---------------------------------------------------------------------------
# FP8
# ---------------------------------------------------------------------------
def test_scale_closed_forms():
    assert ofp8.scale_from_amax(ofp8.amax(np.zeros((3, 3))), E4M3FN) == FLT_MIN
    assert ofp8.scale_from_amax(np.float32(448.0), E4M3FN) == 1.0
    assert ofp8.scale_from_amax(np.float32(57344.0 * 4), E5M2) == 4.0
    assert np.isnan(ofp8.scale_from_amax(ofp8.amax(np.array([1.0, np.nan])), E4M3FN))
    assert np.isinf(ofp8.scale_from_amax(ofp8.amax(np.array([1.0, -np.inf])), E4M3FN))
    # max |x| maps onto fmax
    x = np.array([[0.5, -3.0], [2.0, 1.0]], np.float32)
    q, s = ofp8.scaled_quantize(x, E4M3FN)
    assert s == np.float32(3.0) / np.float32(448.0)
    assert ofp8.fp8_decode(q, E4M3FN)[0, 1] == -448.0


def test_nonfinite_operands():
    """inf in an operand -> scale inf -> finite/inf = 0 and inf/inf = NaN."""

    q, s = ofp8.scaled_quantize(np.array([1.0, np.inf, -2.0], np.float32), E4M3FN)
    assert np.isinf(s)
    v = ofp8.fp8_decode(q, E4M3FN)
    assert v[0] == 0 and np.isnan(v[1]) and v[2] == 0


def test_dot_is_exact_on_representable_operands():
    """Operands whose scaled values are exact fp8 numbers: the scaled dot must
    equal the plain float64 product (no quantization error at all)."""

    g = np.random.Generator(np.random.PCG64(7))
    grid4 = ofp8.fp8_decode(np.arange(0, 0x7F, dtype=np.uint8), E4M3FN)  # finite >= 0
    grid5 = ofp8.fp8_decode(np.arange(0, 0x7C, dtype=np.uint8), E5M2)
    left = g.choice(grid4, size=(12, 32)) * g.choice([-1, 1], size=(12, 32))
    left[0, 0] = 448.0  # amax -> scale exactly 1
    right = g.choice(grid4, size=(32, 9)) * g.choice([-1, 1], size=(32, 9))
    right[0, 0] = -448.0
    out = ofp8.fp8_linear_forward(left, right)
    np.testing.assert_allclose(out, (left.astype(np.float64) @ right).astype(np.float32),
                               rtol=1e-6)
    gy = g.choice(grid5, size=(12, 9)) * g.choice([-1, 1], size=(12, 9))
    gy[0, 0] = 57344.0
    dl, dr = ofp8.fp8_linear_backward(left, right, gy, operand_round=lambda v: v)
    np.testing.assert_allclose(dl, (gy @ right.T).astype(np.float32), rtol=1e-6)
    np.testing.assert_allclose(dr, (left.T @ gy).astype(np.float32), rtol=1e-6)


def test_backward_scales_are_the_forward_ones():
    """The backward's re-quantization of left/right uses the same amax as the
    forward, so caching the forward codes is exact."""

    g = np.random.Generator(np.random.PCG64(8))
    left = bf16_round(g.standard_normal((16, 24)))
    right = bf16_round(g.standard_normal((24, 8)) * 0.02)
    ql, sl = ofp8.scaled_quantize(left, E4M3FN)
    qlt, slt = ofp8.scaled_quantize(left.T, E4M3FN)
    assert sl == slt and np.array_equal(ql.T, qlt)


def test_linear_matmul_flattens_leading_dims():
    g = np.random.Generator(np.random.PCG64(10))
    x = bf16_round(g.standard_normal((2, 3, 16)))
    right = bf16_round(g.standard_normal((16, 5)))
    out = ofp8.linear_matmul_fp8(x, right)
    flat = ofp8.linear_matmul_fp8(x.reshape(6, 16), right)
    assert out.shape == (2, 3, 5) and np.array_equal(out.reshape(6, 5), flat)
    assert np.array_equal(bf16_round(out), out)


# ---------------------------------------------------------------------------
# Delayed scaling (extension; the reference's roadmap, todo.org:1149-1154)
# ---------------------------------------------------------------------------
def _outliers(rng, shape):
    x = rng.standard_normal(shape).astype(np.float32)
    return np.where(rng.random(shape) < 1e-2, x * 50.0, x).astype(np.float32)


def test_saturating_cast_with_own_scale_is_the_dynamic_cast():
    rng = np.random.default_rng(11)
    for fmt in (E4M3FN, E5M2):
        for trial in range(4):
            t = bf16_round(_outliers(rng, (64, 96)) * (10.0 ** (trial - 2)))
            codes, s = ofp8.scaled_quantize(t, fmt)
            assert np.array_equal(ofp8.cast_saturating(t, s, fmt), codes)


def test_saturating_cast_closed_forms():
    for fmt, big in ((E4M3FN, 0x7E), (E5M2, 0x7B)):
        t = np.array([1e9, -1e9, np.inf, -np.inf, np.nan, 0.0, -0.0, 1.0], np.float32)
        c = ofp8.cast_saturating(t, np.float32(1.0), fmt)
        assert c[0] == big and c[1] == (0x80 | big)
        assert c[2] == big and c[3] == (0x80 | big)
        assert (c[4] & 0x7F) == 0x7F if fmt == E4M3FN else (c[4] & 0x7C) == 0x7C and (c[4] & 3) != 0
        assert c[5] == 0x00 and c[6] == 0x80
        # 1.0: exponent bias 7 (e4m3fn) / 15 (e5m2), zero mantissa
        assert c[7] == (0x38 if fmt == E4M3FN else 0x3C)


def test_delayed_update_closed_forms():
    hist = np.array([[0.0, 3.0, 0.0, 448.0],
                     [0.0, 5.0, np.nan, 1.0],
                     [0.0, 1.0, 2.0, 0.0]], np.float32)
    old = np.array([0.5, 0.25, 0.125, 2.0], np.float32)
    fmts = [E4M3FN, E4M3FN, E5M2, E4M3FN]
    new = ofp8.delayed_update(hist, old, fmts)
    assert new[0] == np.float32(0.5)                       # nothing recorded: kept
    assert new[1] == np.float32(np.float32(5.0) / np.float32(448.0))
    assert np.isnan(new[2])                                # a NaN was recorded
    assert new[3] == np.float32(1.0)                       # 448 / 448
    tiny = ofp8.delayed_update(np.array([[1e-45]], np.float32), np.ones(1, np.float32), [E4M3FN])
    assert tiny[0] == np.float32(FLT_MIN)
