"""FP8 amax / cast / GEMM / linear: HIP kernels vs the oracle (GPU)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import fp8 as ofp8
from oracle.codecs import E4M3FN, E5M2, bf16_bits_to_f32
from representax_amd import _native as nat
from representax_amd import ops
from tests.helpers import bf16_values, from_dev, rel_l2, rng, to_dev, to_dev_bf16

pytestmark = pytest.mark.gpu

# rel-L2 bound for fp8 GEMM outputs and gradients: the fp8 products are exact
# in float32, so only the accumulation order (and the final bf16 rounding)
# separates the kernels from the oracle
FP8_TOL = 2e-3


def _all_bf16_values() -> np.ndarray:
    return bf16_bits_to_f32(np.arange(65536, dtype=np.uint32).astype(np.uint16))


@pytest.mark.parametrize("fmt", ["e4m3fn", "e5m2"])
def test_hardware_convert_matches_integer_encoder_everywhere(fmt):
    """The cast kernels convert with the gfx950 packed fp8/bf8 instruction in
    range; it must agree with the integer encoder (pinned to the oracle on the
    host) on every one of the 2^32 f32 bit patterns."""

    bad, first = ops.fp8_encode_selfcheck(fmt, 0, 1 << 31)
    assert bad == 0, f"{bad} mismatches, first pattern {first:#010x}" if first is not None else bad


@pytest.mark.parametrize("fmt", ["e4m3fn", "e5m2"])
def test_cast_every_bf16_value_bit_exact(fmt):
    """All 65536 bf16 patterns x a sweep of scales: codes must match exactly."""

    vals = _all_bf16_values().reshape(256, 256)
    g = rng(3)
    scales = [1.0, 1.17549435e-38, 2.0 ** -126, 0.1, 3.0, 1e-3, 7.5e5]
    scales += list((10.0 ** g.uniform(-6, 6, size=12)).astype(np.float32))
    xd = to_dev_bf16(vals)
    for s in scales:
        sd = torch.tensor([s], dtype=torch.float32, device="cuda")
        out, out_t = ops.fp8_cast(xd, sd, fmt, rowmajor=True, transposed=True)
        torch.cuda.synchronize()
        want = ofp8.cast_with_scale(vals, np.float32(s), fmt)
        got = out.cpu().numpy()
        assert np.array_equal(got, want), (fmt, s)
        assert np.array_equal(out_t.cpu().numpy(), want.T)


@pytest.mark.parametrize("fmt", ["e4m3fn", "e5m2"])
def test_cast_random_f32_bit_exact(fmt):
    g = rng(4)
    bits = g.integers(0, 2**32, size=(512, 1024), dtype=np.uint64).astype(np.uint32)
    vals = bits.view(np.float32)
    vals = np.where(np.isfinite(vals), vals, np.float32(1.0)).astype(np.float32)
    for s in (np.float32(1e-30), np.float32(1.0), np.float32(3.1e30)):
        sd = torch.tensor([s], dtype=torch.float32, device="cuda")
        out, _ = ops.fp8_cast(to_dev(vals), sd, fmt)
        want = ofp8.cast_with_scale(vals, s, fmt)
        assert np.array_equal(out.cpu().numpy(), want), (fmt, s)


@pytest.mark.parametrize("rows,cols", [(300, 200), (37, 96), (129, 136), (8, 8), (1000, 8)])
@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_cast_ragged_tiles_both_outputs_bit_exact(rows, cols, dtype):
    """Tiles cut by the matrix edge: rows not a multiple of 8 or 128, columns
    not a multiple of 128; row-major and transposed codes."""

    g = rng(rows * 7 + cols)
    vals = (g.standard_normal((rows, cols)) * 3.0).astype(np.float32)
    if dtype == "bf16":
        vals = bf16_values(vals)
        xd = to_dev_bf16(vals)
    else:
        xd = to_dev(vals)
    for fmt in ("e4m3fn", "e5m2"):
        s = np.float32(0.037)
        sd = torch.tensor([s], dtype=torch.float32, device="cuda")
        out, out_t = ops.fp8_cast(xd, sd, fmt, rowmajor=True, transposed=True)
        want = ofp8.cast_with_scale(vals, s, fmt)
        assert np.array_equal(out.cpu().numpy(), want), (fmt, rows, cols)
        assert np.array_equal(out_t.cpu().numpy(), want.T), (fmt, rows, cols)


@pytest.mark.parametrize("fmt", ["e4m3fn", "e5m2"])
def test_scale_matches_oracle(fmt):
    g = rng(5)
    x = bf16_values(g.standard_normal((8192, 768)))
    mask = g.random(x.shape) < 1e-3
    x = bf16_values(np.where(mask, x * 50, x))
    cases = {
        "outliers": x,
        "zeros": np.zeros((64, 96), np.float32),
        "tiny": np.full((10, 10), 1e-39, np.float32),
        "ragged": bf16_values(g.standard_normal((3, 7))),
    }
    for name, arr in cases.items():
        s = ops.fp8_scale(to_dev_bf16(arr), fmt)
        want = ofp8.scale_from_amax(ofp8.amax(bf16_values(arr)), fmt)
        assert from_dev(s)[0] == want, name
    nan_case = np.ones((4, 4), np.float32)
    nan_case[2, 3] = np.nan
    assert np.isnan(from_dev(ops.fp8_scale(to_dev(nan_case), fmt))[0])
    inf_case = np.ones((4, 4), np.float32)
    inf_case[0, 0] = -np.inf
    assert np.isinf(from_dev(ops.fp8_scale(to_dev(inf_case), fmt))[0])


@pytest.mark.parametrize(
    "m,n,k,fa,fb",
    [(256, 256, 256, E4M3FN, E4M3FN), (512, 384, 768, E5M2, E4M3FN),
     (768, 3072, 1024, E4M3FN, E5M2), (100, 70, 200, E4M3FN, E4M3FN), (64, 96, 8192, E5M2, E5M2),
     (1000, 770, 384, E4M3FN, E4M3FN), (300, 1000, 640, E5M2, E4M3FN)],
)
def test_fp8_gemm_matches_oracle(m, n, k, fa, fb):
    g = rng(m + n + k)
    qa = g.integers(0, 256, size=(m, k), dtype=np.uint8)
    qb = g.integers(0, 256, size=(n, k), dtype=np.uint8)
    # keep codes finite: drop NaN / inf patterns
    for q, f in ((qa, fa), (qb, fb)):
        vals = ofp8.fp8_decode(q, f)
        q[~np.isfinite(vals)] = 0x01
    sa, sb = np.float32(0.0123), np.float32(3.7)
    want = ofp8.scaled_dot_codes(qa, sa, fa, qb.T, sb, fb)
    got = ops.fp8_gemm(to_dev(qa), fa, torch.tensor([sa], device="cuda"), to_dev(qb), fb,
                       torch.tensor([sb], device="cuda"), out_dtype=torch.float32)
    torch.cuda.synchronize()
    # products are exact; only the MFMA's float32 accumulation differs from the
    # float64 sum (codes span the whole fp8 range, so cancellation is heavy)
    assert rel_l2(from_dev(got), want) < 2e-4


@pytest.mark.parametrize(
    "m,n,k,fa",
    [(8192, 768, 768, E4M3FN), (768, 768, 8192, E5M2), (1000, 770, 384, E4M3FN),
     (130, 4100, 128, E5M2), (300, 1000, 640, E4M3FN), (8192, 3072, 768, E4M3FN)],
)
def test_fp8_gemm_bf16_output_is_rounded_f32_output(m, n, k, fa):
    # the bf16 epilogue (staged through LDS, whole-row stores, edge tiles) must
    # write exactly the round-to-nearest-even of what the fp32 epilogue writes
    g = torch.Generator(device="cuda").manual_seed(m * 7 + n)
    qa = torch.randint(0, 256, (m, k), dtype=torch.uint8, device="cuda", generator=g)
    qb = torch.randint(0, 256, (n, k), dtype=torch.uint8, device="cuda", generator=g)
    qa[(qa & 0x7F) >= 0x78] = 0x11  # finite codes in both formats
    qb[(qb & 0x7F) >= 0x78] = 0x22
    sa = torch.tensor([0.03], device="cuda")
    sb = torch.tensor([0.5], device="cuda")
    f32 = ops.fp8_gemm(qa, fa, sa, qb, E4M3FN, sb, out_dtype=torch.float32)
    b16 = ops.fp8_gemm(qa, fa, sa, qb, E4M3FN, sb, out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    assert torch.isfinite(f32).all()
    assert torch.equal(b16.view(torch.int16), f32.to(torch.bfloat16).view(torch.int16))


def _fp8_case(m, k, n, seed):
    g = rng(seed)
    x = g.standard_normal((m, k))
    mask = g.random(x.shape) < 1e-3
    x = bf16_values(np.where(mask, x * 50, x))
    w = bf16_values(g.standard_normal((n, k)) * 0.02)
    gy = bf16_values(g.standard_normal((m, n)))
    return x, w, gy


@pytest.mark.parametrize("m,k,n", [(1024, 768, 768), (2048, 768, 3072), (2048, 3072, 768),
                                   (50, 40, 30)])
def test_fp8_linear_forward_backward(m, k, n):
    x, w, gy = _fp8_case(m, k, n, seed=m + k + n)
    right = w.T  # linear_matmul(value, weight.T)
    y_o = bf16_values(ofp8.fp8_linear_forward(x, right))
    dl_o, dr_o = ofp8.fp8_linear_backward(x, right, gy)
    xd = to_dev_bf16(x)
    wd = to_dev_bf16(w)
    y, scales, codes = ops.fp8_linear_forward(xd, wd.t(), save_codes=True)
    dl, dr = ops.fp8_linear_backward(xd, wd.t(), to_dev_bf16(gy), scales)
    dl_c, dr_c = ops.fp8_linear_backward_codes(codes, scales, to_dev_bf16(gy), k=k,
                                               dtype=torch.bfloat16, right_transposed=True)
    torch.cuda.synchronize()
    # the saved-codes backward is the same computation as re-quantizing
    assert torch.equal(dl, dl_c) and torch.equal(dr, dr_c)
    s = from_dev(scales)
    assert s[0] == ofp8.scale_from_amax(ofp8.amax(x), E4M3FN)
    assert s[1] == ofp8.scale_from_amax(ofp8.amax(w), E4M3FN)
    assert dr.shape == (k, n)
    assert rel_l2(from_dev(y), y_o) < FP8_TOL
    assert rel_l2(from_dev(dl), dl_o) < FP8_TOL
    assert rel_l2(from_dev(dr), dr_o) < FP8_TOL


def test_fp8_linear_bert_ffn_full_size():
    m, k, n = 8192, 768, 3072
    x, w, gy = _fp8_case(m, k, n, seed=77)
    right = w.T
    y_o = bf16_values(ofp8.fp8_linear_forward(x, right, acc=np.float32))
    dl_o, dr_o = ofp8.fp8_linear_backward(x, right, gy, acc=np.float32)
    xd, wd = to_dev_bf16(x), to_dev_bf16(w)
    y, scales, codes = ops.fp8_linear_forward(xd, wd.t(), save_codes=True)
    dl, dr = ops.fp8_linear_backward_codes(codes, scales, to_dev_bf16(gy), k=k,
                                           dtype=torch.bfloat16, right_transposed=True)
    torch.cuda.synchronize()
    errs = [rel_l2(from_dev(y), y_o), rel_l2(from_dev(dl), dl_o), rel_l2(from_dev(dr), dr_o)]
    assert max(errs) < FP8_TOL, errs


@pytest.mark.parametrize("m,k,n", [(300, 200, 136), (1000, 8, 40), (129, 96, 8),
                                   (2100 * 128 + 5, 8, 16)])
def test_fused_quantize_scales_and_codes_bit_exact(m, k, n):
    """The linear's own quantize (amax tile partials, then every cast block
    reducing them to the scale): scales and the saved codes (left row-major
    [M, K], right [K, N]) equal the oracle's, on ragged tiles and on an
    operand of more than 2048 tiles (partials beyond the ones each thread
    loads up front)."""

    x, w, _ = _fp8_case(m, k, n, seed=m + 3 * k + n)
    _, scales, codes = ops.fp8_linear_forward(to_dev_bf16(x), to_dev_bf16(w).t(), save_codes=True)
    torch.cuda.synchronize()
    s = from_dev(scales)
    s_x = ofp8.scale_from_amax(ofp8.amax(x), E4M3FN)
    s_w = ofp8.scale_from_amax(ofp8.amax(w), E4M3FN)
    assert s[0] == s_x and s[1] == s_w
    assert np.array_equal(codes[0].cpu().numpy(), ofp8.cast_with_scale(x, s_x, E4M3FN))
    assert np.array_equal(codes[1].cpu().numpy(), ofp8.cast_with_scale(w, s_w, E4M3FN).T)


def _kernel_names(fn):
    with torch.profiler.profile(activities=[torch.profiler.ProfilerActivity.CUDA]) as prof:
        out = fn()
        torch.cuda.synchronize()
    return out, [e.key for e in prof.key_averages()]


@pytest.mark.parametrize("m,k,n,paired", [(8192, 768, 768, True), (16384, 768, 768, True),
                                          (8192, 768, 3072, True), (8192, 3072, 768, True),
                                          (8192, 700, 768, None)])
def test_paired_backward_equals_two_launches(m, k, n, paired):
    """The backward's input and weight gradients in one launch (the default
    where both products' plans allow it: the BERT-base linears at 8192
    tokens) equal the two separate launches bit for bit."""

    x, w, gy = _fp8_case(m, k, n, seed=m + 5 * k + n)
    _, scales, codes = ops.fp8_linear_forward(to_dev_bf16(x), to_dev_bf16(w).t(),
                                              save_codes=True)
    gd = to_dev_bf16(gy)
    lib = nat.load()
    old = lib.rpx_get_tuning(nat.TUNE_FP8_PAIR)
    got = {}
    try:
        for v in (-1, 0):
            assert lib.rpx_set_tuning(nat.TUNE_FP8_PAIR, v) == 0
            got[v] = _kernel_names(lambda: ops.fp8_linear_backward_codes(
                codes, scales, gd, k=k, dtype=torch.bfloat16, right_transposed=True))
    finally:
        lib.rpx_set_tuning(nat.TUNE_FP8_PAIR, old)
    ran = {v: any("k_fp8_gemm_pair" in name for name in got[v][1]) for v in got}
    assert not ran[0]
    if paired is not None:
        assert ran[-1] == paired
    (dl1, dr1), (dl0, dr0) = got[-1][0], got[0][0]
    assert torch.equal(dl1, dl0) and torch.equal(dr1, dr0)


@pytest.mark.parametrize("m,k,n", [(8192, 768, 768), (300, 200, 256)])
def test_backward_gemms_from_gradient_codes(m, k, n):
    """rpx_fp8_linear_backward_gemms on gradient codes quantized by the
    caller equals the backward that quantizes the gradient itself, for each
    subset of outputs and both right-operand layouts."""

    x, w, gy = _fp8_case(m, k, n, seed=m + 7 * k + n)
    _, scales, codes = ops.fp8_linear_forward(to_dev_bf16(x), to_dev_bf16(w).t(), save_codes=True)
    gd = to_dev_bf16(gy)
    s_g = ops.fp8_scale(gd, E5M2)
    qg, _ = ops.fp8_cast(gd, s_g, E5M2, rowmajor=True)
    for right_t in (True, False):
        for need_l, need_r in ((True, True), (True, False), (False, True)):
            want = ops.fp8_linear_backward_codes(codes, scales, gd, k=k, dtype=torch.bfloat16,
                                                 right_transposed=right_t, need_left=need_l,
                                                 need_right=need_r)
            got = ops.fp8_linear_backward_gemms(qg, s_g, codes[0], scales[0:1], codes[1],
                                                scales[1:2], k=k, dtype=torch.bfloat16,
                                                right_transposed=right_t, need_left=need_l,
                                                need_right=need_r)
            torch.cuda.synchronize()
            for a, b in zip(got, want):
                assert (a is None) == (b is None)
                if a is not None:
                    assert a.shape == b.shape and torch.equal(a, b), (right_t, need_l, need_r)


def test_fp8_linear_natural_right_layout():
    """right given as a row-major [K, N] matrix (not a transposed view)."""

    m, k, n = 256, 384, 512
    x, w, gy = _fp8_case(m, k, n, seed=9)
    right = np.ascontiguousarray(w.T)
    y_o = bf16_values(ofp8.fp8_linear_forward(x, right))
    dl_o, dr_o = ofp8.fp8_linear_backward(x, right, gy)
    rd = to_dev_bf16(right)
    y, scales, codes = ops.fp8_linear_forward(to_dev_bf16(x), rd, save_codes=True)
    dl, dr = ops.fp8_linear_backward_codes(codes, scales, to_dev_bf16(gy), k=k,
                                           dtype=torch.bfloat16, right_transposed=False)
    torch.cuda.synchronize()
    assert dr.shape == (k, n) and dr.is_contiguous()
    for got, want in ((y, y_o), (dl, dl_o), (dr, dr_o)):
        assert rel_l2(from_dev(got), want) < FP8_TOL


def test_fp8_autograd_function_gradients():
    """Fp8LinearFn through torch autograd equals the explicit backward."""

    m, k, n = 512, 256, 384
    x, w, gy = _fp8_case(m, k, n, seed=10)
    xd = to_dev_bf16(x).requires_grad_(True)
    wd = to_dev_bf16(w).requires_grad_(True)
    y = ops.Fp8LinearFn.apply(xd, wd.t(), torch.bfloat16)
    y.backward(to_dev_bf16(gy))
    dl_o, dr_o = ofp8.fp8_linear_backward(x, w.T, gy)
    assert rel_l2(from_dev(xd.grad), dl_o) < FP8_TOL
    assert rel_l2(from_dev(wd.grad), dr_o.T) < FP8_TOL
