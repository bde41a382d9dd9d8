"""Every fp8 GEMM plan, the BERT-base step's fp8 calls at full size, and the
INT4 + LoRA module under the fp8 policy, against the oracle (GPU).

The fp8 planner (``plan_fp8``) picks one of eleven tile configurations and a
split-K count per shape. Each configuration is forced here with the tuning
knobs, at several forced split counts (including a ragged last split), on
shapes whose M and N are cut by every tile edge, in all four operand-format
pairs, against ``oracle.fp8.scaled_dot_codes`` (float64 sums of the decoded
codes). A tile only changes which workgroup computes an output and a split
count only where the partial sums meet, so for one split count every tile
gives the same bits.

The full-size cases are the nine distinct GEMM calls of the BERT-base fp8
step at 8192 tokens (forward, input gradient and weight gradient of the
768 -> 768, 768 -> 3072 and 3072 -> 768 linears, precision.py:143-221),
with the planner's own choice, codes from quantizing normal data with
outliers (the step's inputs).

The module case is ``QuantizedLoRALinear`` under ``float8_mixed``: the
reference sends the base product and both adapter products through
``linear_matmul`` (adapters.py:158-182 -> precision.py:224-239), so the
forward and the gradients of x, A and B are compared with the same
composition of oracle pieces (``dequant_int4``, ``fp8_linear_forward``,
``fp8_linear_backward``) at the reference's bf16 rounding points.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import representax_amd as rx
from oracle import fp8 as ofp8
from oracle import int4 as oint4
from oracle.codecs import E4M3FN, E5M2, bf16_bits_to_f32, bf16_round
from representax_amd import ops
from tests.helpers import (assert_bf16_close, bf16_values,
                           from_dev, rel_l2, rng, to_dev, to_dev_bf16)

pytestmark = pytest.mark.gpu

FP8_CONFIGS = list(range(1, 12))
# BM x BN of each configuration (fp8_gemm.hip, RPX_FP8_CONFIGS)
FP8_TILE_SHAPES = {1: (128, 128), 2: (256, 128), 3: (256, 192), 4: (128, 192), 5: (256, 256),
                   6: (128, 128), 7: (128, 192), 8: (256, 96), 9: (128, 128), 10: (256, 128),
                   11: (256, 256)}
# fp8 outputs against the float64 oracle: the MFMA's sum of fp8 products is
# not a sequential float32 sum (5e-5 relative at K = 768 was measured), so
# float32 outputs are held to 2e-4 (the bar of the raw GEMM tests) and bf16
# outputs to rel-L2 2e-3 (the fp8 linear tests' bar), plus bit equality
# between the bf16 output and the rounded float32 output
FP8_F32_TOL = 2e-4
FP8_TOL = 2e-3
FORMAT_PAIRS = [(E4M3FN, E4M3FN), (E5M2, E4M3FN), (E4M3FN, E5M2), (E5M2, E5M2)]
# (m, n, k, split counts): k = 1280 is ten 128-deep slices (3 and 4 splits
# leave a short last split), k = 640 five
RAGGED = [(300, 200, 1280, (1, 3, 4)), (129, 385, 640, (1, 2, 5))]


def _finite_codes(g, shape, fmt):
    q = g.integers(0, 256, size=shape, dtype=np.uint8)
    q[~np.isfinite(ofp8.fp8_decode(q, fmt))] = 0x01
    return q


def _gemm(qa, fa, sa, qb, fb, sb, out_dtype):
    return ops.fp8_gemm(qa, fa, torch.tensor([sa], device="cuda"), qb, fb,
                        torch.tensor([sb], device="cuda"), out_dtype=out_dtype)


@pytest.mark.parametrize("fa,fb", FORMAT_PAIRS)
@pytest.mark.parametrize("cfg", FP8_CONFIGS)
def test_every_fp8_tile_and_split_matches_oracle(cfg, fa, fb):
    for m, n, k, splits in RAGGED:
        g = rng(cfg * 1000 + m + 7 * k)
        qa = _finite_codes(g, (m, k), fa)
        qb = _finite_codes(g, (n, k), fb)
        sa, sb = np.float32(0.0123), np.float32(3.7)
        want = ofp8.scaled_dot_codes(qa, sa, fa, qb.T, sb, fb)
        qad, qbd = to_dev(qa), to_dev(qb)
        for s in splits:
            with ops.tuning(fp8_tile=cfg, fp8_splits=s):
                ws_bytes = ops.nat.query("rpx_fp8_gemm_workspace", m, n, k)
                f32 = _gemm(qad, fa, sa, qbd, fb, sb, torch.float32)
                b16 = _gemm(qad, fa, sa, qbd, fb, sb, torch.bfloat16)
            torch.cuda.synchronize()
            # the forced split count is the one the launch used: s partial
            # tiles of BM x BN floats per output tile
            bm, bn = FP8_TILE_SHAPES[cfg]
            tiles = -(-m // bm) * -(-n // bn)
            assert ws_bytes == (0 if s == 1 else 4 * s * tiles * bm * bn), (cfg, s, ws_bytes)
            # codes span the whole fp8 range (heavy cancellation): only the
            # MFMA's float32 accumulation order differs from the float64 sum
            assert rel_l2(from_dev(f32), want) < FP8_F32_TOL, (cfg, s, m, n, k)
            assert torch.equal(b16.view(torch.int16), f32.to(torch.bfloat16).view(torch.int16))


@pytest.mark.parametrize("fa,fb", [(E4M3FN, E4M3FN), (E5M2, E4M3FN)])
def test_fp8_tiles_agree_bit_for_bit_per_split_count(fa, fb):
    m, n, k = 300, 200, 1280
    g = rng(4242)
    qa = to_dev(_finite_codes(g, (m, k), fa))
    qb = to_dev(_finite_codes(g, (n, k), fb))
    for s in (1, 3):
        first = None
        for cfg in FP8_CONFIGS:
            with ops.tuning(fp8_tile=cfg, fp8_splits=s):
                got = _gemm(qa, fa, 0.5, qb, fb, 0.25, torch.float32)
            torch.cuda.synchronize()
            if first is None:
                first = (cfg, got)
            else:
                assert torch.equal(got, first[1]), (s, cfg, first[0])


def _quantized(g, shape, fmt, outliers=False, std=1.0):
    """Codes and scale of normal data (0.1% outliers x 50 when asked), as
    the step's dynamic quantize makes them: a pool of 2^16 values is
    quantized by the oracle and the matrix drawn from its codes (the
    oracle's encoder takes tens of seconds on a whole 8192 x 3072 tensor)."""

    v = g.standard_normal(1 << 16).astype(np.float32) * std
    if outliers:
        mask = g.random(v.shape) < 1e-3
        v = np.where(mask, v * 50, v).astype(np.float32)
    pool, s = ofp8.scaled_quantize(bf16_values(v), fmt)
    return pool[g.integers(0, pool.size, size=shape)], s


# The step's nine distinct GEMM calls (M, N, K, format of A, format of B):
# forward x . W^T, input gradient g . W, weight gradient x^T . g, for the
# 768 -> 768 (q/k/v/o), 768 -> 3072 (FFN up) and 3072 -> 768 (FFN down)
# linears at 8192 tokens. The 768 x 768 weight gradient is the planner's
# three-split plan.
STEP_CALLS = [
    ("qkvo_fwd", 8192, 768, 768, E4M3FN, E4M3FN),
    ("qkvo_dx", 8192, 768, 768, E5M2, E4M3FN),
    ("qkvo_dw", 768, 768, 8192, E4M3FN, E5M2),
    ("up_fwd", 8192, 3072, 768, E4M3FN, E4M3FN),
    ("up_dx", 8192, 768, 3072, E5M2, E4M3FN),
    ("up_dw", 768, 3072, 8192, E4M3FN, E5M2),
    ("down_fwd", 8192, 768, 3072, E4M3FN, E4M3FN),
    ("down_dx", 8192, 3072, 768, E5M2, E4M3FN),
    ("down_dw", 3072, 768, 8192, E4M3FN, E5M2),
]


@pytest.mark.parametrize("call", range(len(STEP_CALLS)))
def test_fp8_step_calls_full_size_match_oracle(call):
    name, m, n, k, fa, fb = STEP_CALLS[call]
    g = rng(500 + call)
    qa, sa = _quantized(g, (m, k), fa, outliers=fa == E4M3FN)
    qb, sb = _quantized(g, (n, k), fb, std=0.02 if fb == E4M3FN else 1.0)
    want = ofp8.scaled_dot_codes(qa, sa, fa, qb.T, sb, fb)
    qad, qbd = to_dev(qa), to_dev(qb)
    ws_bytes = ops.nat.query("rpx_fp8_gemm_workspace", m, n, k)
    f32 = _gemm(qad, fa, sa, qbd, fb, sb, torch.float32)
    b16 = _gemm(qad, fa, sa, qbd, fb, sb, torch.bfloat16)
    torch.cuda.synchronize()
    if name == "qkvo_dw":
        # the planner's three splits: 3 x 36 partial tiles of 128 x 128 floats
        assert ws_bytes == 4 * 3 * 36 * 128 * 128, ws_bytes
    assert rel_l2(from_dev(f32), want) < FP8_F32_TOL, name
    assert_bf16_close(from_dev(b16), bf16_round(want), tol=FP8_TOL, min_equal=None, what=name)
    assert torch.equal(b16.view(torch.int16), f32.to(torch.bfloat16).view(torch.int16))


def _weight_grad_krows(qx, s_x, qg, s_g, right_t):
    """d_right of the fp8 linear backward through the K-row kernel (the
    tokens-major codes of the input and the gradient as they are): [N, K]
    when right_t, else [K, N]."""

    m, k = qx.shape
    n = qg.shape[1]
    dummy = torch.zeros((k, n), dtype=torch.uint8, device="cuda")
    _, d_right = ops.fp8_linear_backward_gemms(
        qg, torch.tensor([s_g], device="cuda"), qx, torch.tensor([s_x], device="cuda"), dummy,
        torch.tensor([1.0], device="cuda"), k=k, dtype=torch.bfloat16, right_transposed=right_t,
        need_left=False)
    return d_right.t() if right_t else d_right


def _weight_grad_rowmajor(qx, s_x, qg, s_g, right_t):
    """The same product through the row-major kernel on transposed copies."""

    xt, gt = qx.t().contiguous(), qg.t().contiguous()
    sx, sg = torch.tensor([s_x], device="cuda"), torch.tensor([s_g], device="cuda")
    if right_t:
        return ops.fp8_gemm(gt, E5M2, sx, xt, E4M3FN, sg, out_dtype=torch.bfloat16)
    return ops.fp8_gemm(xt, E4M3FN, sx, gt, E5M2, sg, out_dtype=torch.bfloat16)


# (tokens, K, N, split counts): N and K multiples of 16 but not of 128, the
# tokens ten and five 128-deep slices
KROWS_RAGGED = [(1280, 208, 400, (1, 3, 4)), (640, 96, 144, (1, 2, 5))]


@pytest.mark.parametrize("right_t", [True, False])
@pytest.mark.parametrize("cfg", [0, 1, 6, 9])
def test_weight_gradient_krows_plans(cfg, right_t):
    """The weight gradient read along the tokens from row-major codes (the
    128 x 128 configurations, forced split counts, edge tiles): the oracle's
    product, and bit for bit the row-major kernel's on transposed copies
    under the same plan (cfg 0: the planner's, checked against the oracle
    only)."""

    for m, k, n, splits in KROWS_RAGGED:
        g = rng(cfg * 100 + m + k + n)
        qx = _finite_codes(g, (m, k), E4M3FN)
        qg = _finite_codes(g, (m, n), E5M2)
        s_x, s_g = np.float32(0.0123), np.float32(3.7)
        if right_t:
            want = ofp8.scaled_dot_codes(np.ascontiguousarray(qg.T), s_x, E5M2, qx, s_g, E4M3FN)
        else:
            want = ofp8.scaled_dot_codes(np.ascontiguousarray(qx.T), s_x, E4M3FN, qg, s_g, E5M2)
        qxd, qgd = to_dev(qx), to_dev(qg)
        for sp in splits:
            with ops.tuning(fp8_tile=cfg, fp8_splits=sp):
                got = _weight_grad_krows(qxd, s_x, qgd, s_g, right_t)
                ref = _weight_grad_rowmajor(qxd, s_x, qgd, s_g, right_t) if cfg else None
            torch.cuda.synchronize()
            assert_bf16_close(from_dev(got), bf16_round(want), tol=FP8_TOL, min_equal=None,
                              what=f"cfg {cfg} splits {sp} {m}x{k}x{n}")
            if ref is not None:
                assert torch.equal(got, ref), (cfg, sp, m, k, n, right_t)


@pytest.mark.parametrize("m,k,n", [(200, 40, 30), (256, 24, 136), (384, 128, 100)])
def test_weight_gradient_krows_generic_shapes(m, k, n):
    """Shapes the pipelined K-row kernel does not take (tokens not a multiple
    of 128, or K, N not multiples of 16) go to the generic kernel."""

    g = rng(m * 3 + k + n)
    qx = _finite_codes(g, (m, k), E4M3FN)
    qg = _finite_codes(g, (m, n), E5M2)
    s_x, s_g = np.float32(0.05), np.float32(2.0)
    for right_t in (True, False):
        got = _weight_grad_krows(to_dev(qx), s_x, to_dev(qg), s_g, right_t)
        torch.cuda.synchronize()
        if right_t:
            want = ofp8.scaled_dot_codes(np.ascontiguousarray(qg.T), s_x, E5M2, qx, s_g, E4M3FN)
        else:
            want = ofp8.scaled_dot_codes(np.ascontiguousarray(qx.T), s_x, E4M3FN, qg, s_g, E5M2)
        assert_bf16_close(from_dev(got), bf16_round(want), tol=FP8_TOL, min_equal=None,
                          what=f"{m}x{k}x{n} right_t={right_t}")


@pytest.mark.parametrize("k,n", [(768, 768), (768, 3072), (3072, 768)])
def test_weight_gradient_krows_step_shapes(k, n):
    """The step's three weight gradients at 8192 tokens, from the tokens-major
    codes: the oracle's product, and bit for bit the row-major kernel's (the
    planners agree on these shapes: three-stage 128 x 128 tiles, three splits
    for 768 x 768, unsplit otherwise)."""

    m = 8192
    g = rng(900 + k + n)
    qx, s_x = _quantized(g, (m, k), E4M3FN, outliers=True)
    qg, s_g = _quantized(g, (m, n), E5M2)
    want = ofp8.scaled_dot_codes(np.ascontiguousarray(qg.T), s_x, E5M2, qx, s_g, E4M3FN)
    qxd, qgd = to_dev(qx), to_dev(qg)
    got = _weight_grad_krows(qxd, s_x, qgd, s_g, True)
    ref = _weight_grad_rowmajor(qxd, s_x, qgd, s_g, True)
    torch.cuda.synchronize()
    assert_bf16_close(from_dev(got), bf16_round(want), tol=FP8_TOL, min_equal=None,
                      what=f"dW {n}x{k}")
    assert torch.equal(got, ref)


def _fp8_adapter_oracle(x, packed, scales, a, b, bias_bits, alpha, rank, k, gy):
    """The fp8-policy forward and backward of QuantizedLoRALinear from the
    oracle's pieces, at the reference's bf16 rounding points
    (adapters.py:162-181 with linear_matmul's fp8 branch and its custom VJP).
    Returns y, dx, dA, dB."""

    w_b = oint4.dequant_int4(packed, scales, k)
    a_b, b_b = bf16_values(a), bf16_values(b)
    c = float(bf16_values(np.float32(alpha / rank)))  # the weak scalar in bf16
    base = bf16_round(ofp8.fp8_linear_forward(x, w_b.T))
    hidden = bf16_round(ofp8.fp8_linear_forward(x, a_b.T))
    adapter = bf16_round(ofp8.fp8_linear_forward(hidden, b_b.T))
    y = bf16_round(base + bf16_round(adapter * np.float32(c)))
    if bias_bits is not None:
        y = bf16_round(y + bf16_bits_to_f32(bias_bits))
    g_ad = bf16_round(gy * np.float32(c))
    d_hidden, d_bt = ofp8.fp8_linear_backward(hidden, b_b.T, g_ad)
    dx_base, _ = ofp8.fp8_linear_backward(x, w_b.T, gy)
    dx_lora, d_at = ofp8.fp8_linear_backward(x, a_b.T, d_hidden)
    dx = bf16_round(dx_base + dx_lora)
    return y, dx, d_at.T, d_bt.T


@pytest.mark.parametrize("m,k,n,r,bias", [(512, 256, 192, 16, True), (300, 384, 640, 8, False)])
def test_quantized_lora_float8_policy_matches_oracle(m, k, n, r, bias):
    """All three adapter products through the fp8 path, forward and the
    gradients of x, A and B, against the oracle composition."""

    g = rng(31 + m + r)
    lin = rx.Linear.init(k, n, key=1, scale=0.05, bias=bias, device="cuda")
    layer = rx.QuantizedLoRALinear.from_linear(lin, rank=r, alpha=2.0 * r, key=2)
    with torch.no_grad():
        layer.lora_b.copy_(torch.from_numpy((g.standard_normal((n, r)) * 0.05).astype(np.float32)))
    x = bf16_values(g.standard_normal((m, k)))
    gy = bf16_values(g.standard_normal((m, n)))
    xd = to_dev_bf16(x).requires_grad_(True)
    policy = rx.resolve_precision_policy(rx.PrecisionConfig.float8_mixed())
    with rx.precision_context(policy):
        y = layer(xd)
    y.backward(to_dev_bf16(gy))
    torch.cuda.synchronize()
    assert y.dtype == torch.bfloat16 and xd.grad.dtype == torch.bfloat16
    packed = layer.packed_weight.cpu().numpy()
    scales = layer.scale_bits.view(torch.int16).cpu().numpy().view(np.uint16)
    bias_bits = None if layer.bias_bits is None else \
        layer.bias_bits.view(torch.int16).cpu().numpy().view(np.uint16)
    a = layer.lora_a.detach().cpu().numpy()
    b = layer.lora_b.detach().cpu().numpy()
    y_o, dx_o, da_o, db_o = _fp8_adapter_oracle(x, packed, scales, a, b, bias_bits, 2.0 * r, r,
                                                k, gy)
    assert_bf16_close(from_dev(y.detach()), y_o, what="y")
    assert_bf16_close(from_dev(xd.grad), dx_o, what="dx")
    # dA and dB: float32 masters holding the bf16 gradients of the compute
    # view. Each is an fp8 product over every token with an e5m2 operand, so
    # it carries the fp8 MFMA's summation (94% of the elements measured
    # bit-equal to the float64 oracle's): the fp8 bar, rel-L2 2e-3
    da = layer.lora_a.grad.cpu().numpy()
    db = layer.lora_b.grad.cpu().numpy()
    assert np.array_equal(bf16_values(da), da) and np.array_equal(bf16_values(db), db)
    assert_bf16_close(da, da_o, tol=FP8_TOL, min_equal=None, what="dA")
    assert_bf16_close(db, db_o, tol=FP8_TOL, min_equal=None, what="dB")
