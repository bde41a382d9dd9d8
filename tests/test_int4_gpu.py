"""INT4 codec and INT4+LoRA linear: HIP kernels vs the oracle (GPU)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import int4 as oint4
from oracle import lora as olora
from oracle.codecs import bf16_bits_to_f32, f32_to_bf16_bits
from representax_amd import ops
from tests.helpers import (BF16_MIN_EQUAL_TOKEN_SUM, BF16_REL_TOL, assert_bf16_close,
                           bits_from_dev, bf16_values, from_dev, rel_l2, rng, to_dev,
                           to_dev_bf16)

pytestmark = pytest.mark.gpu

# bf16 rel-L2 bound for GEMM outputs and gradients (accumulation order only)
TOL = BF16_REL_TOL


def _scale_patterns(count: int, seed: int) -> np.ndarray:
    g = rng(seed)
    special = np.array(
        [0x0000, 0x8000, 0x0001, 0x007F, 0x0080, 0x3F80, 0xBF80, 0x3C23, 0x7F7F, 0x4000, 0x3E00,
         0x0100, 0x3A83, 0x3D4D],
        dtype=np.uint16,
    )
    finite = g.integers(0, 0x7F80, size=count - special.size, dtype=np.uint16)
    sign = g.integers(0, 2, size=finite.size, dtype=np.uint16) << 15
    return np.concatenate([special, finite | sign])


@pytest.mark.parametrize("group", [None, 64])
def test_dequant_exhaustive_bytes(group):
    """Every byte value (both nibbles) against many scale patterns, bit-exact."""

    n = 2048
    k = 512  # each row holds all 256 byte values
    packed = np.tile(np.arange(256, dtype=np.uint8), (n, 1))
    if group is None:
        scales = _scale_patterns(n, 11)
    else:
        scales = _scale_patterns(n * (k // group), 12).reshape(n, k // group)
    out = ops.int4_dequant(to_dev(packed), to_dev(scales.view(np.int16)).view(torch.uint16), k,
                           group)
    torch.cuda.synchronize()
    got = bits_from_dev(out)
    want = oint4.dequant_int4_bits(packed, scales, k, group)
    assert np.array_equal(got, want)


@pytest.mark.parametrize(
    "n,k,group",
    [(6, 8, None), (5, 7, None), (33, 130, None), (3072, 768, None), (3072, 768, 64), (64, 256, 32),
     (17, 96, 48)],
)
def test_pack_and_dequant_match_oracle(n, k, group):
    g = rng(100 + n + k)
    w = (g.standard_normal((n, k)) * 0.02).astype(np.float32)
    if n > 4:
        w[1] = 0.0  # zero row -> scale 1.0, zero nibbles
        w[2, : min(k, 4)] = [0.5, -0.5, 0.25, 1.25][: min(k, 4)]
    packed_d, scales_d = ops.int4_pack(to_dev(w), group)
    torch.cuda.synchronize()
    packed_o, scales_o = oint4.pack_int4(w, group)
    assert np.array_equal(packed_d.cpu().numpy(), packed_o)
    assert np.array_equal(bits_from_dev(scales_d), scales_o)
    deq = ops.int4_dequant(packed_d, scales_d, k, group)
    assert np.array_equal(bits_from_dev(deq), oint4.dequant_int4_bits(packed_o, scales_o, k, group))


def test_pack_from_bf16_weights():
    g = rng(7)
    w = bf16_values(g.standard_normal((64, 128)) * 0.05)
    packed_d, scales_d = ops.int4_pack(to_dev_bf16(w))
    packed_o, scales_o = oint4.pack_int4(w)
    assert np.array_equal(packed_d.cpu().numpy(), packed_o)
    assert np.array_equal(bits_from_dev(scales_d), scales_o)


def _lora_case(m, k, n, r, group, seed, bias=True):
    g = rng(seed)
    x = bf16_values(g.standard_normal((m, k)))
    w = (g.standard_normal((n, k)) * 0.02).astype(np.float32)
    a = (g.standard_normal((r, k)) * 0.02).astype(np.float32)
    b = (g.standard_normal((n, r)) * 0.02).astype(np.float32)
    bias_v = (g.standard_normal(n) * 0.1).astype(np.float32) if bias else None
    gy = bf16_values(g.standard_normal((m, n)))
    packed, scales = oint4.pack_int4(w, group)
    bias_bits = None if bias_v is None else f32_to_bf16_bits(bias_v)
    return x, packed, scales, a, b, bias_bits, gy


LORA_SHAPES = [
    # (m, k, n, r, group): fused MFMA path
    (256, 128, 192, 16, None),
    (300, 256, 320, 16, 64),
    (512, 768, 3072, 16, None),
    (96, 512, 256, 32, 128),
    (64, 192, 128, 8, None),
    # generic path (the reference test's 8->6, rank 2; odd sizes)
    (4, 8, 6, 2, None),
    (37, 100, 52, 3, None),
    (20, 96, 100, 72, None),
]


@pytest.mark.parametrize("m,k,n,r,group", LORA_SHAPES)
def test_int4lora_forward_backward(m, k, n, r, group):
    x, packed, scales, a, b, bias_bits, gy = _lora_case(m, k, n, r, group, seed=m * 7 + k)
    alpha = 2.0 * r
    y_o, h_o = olora.lora_forward(x, packed, scales, a, b, alpha=alpha, rank=r,
                                  bias_bits=bias_bits, group_size=group)
    dx_o, da_o, db_o = olora.lora_backward(gy, x, packed, scales, a, b, h_o, alpha=alpha, rank=r,
                                           group_size=group)
    xd = to_dev_bf16(x)
    pd = to_dev(packed)
    sd = to_dev(scales.view(np.int16)).view(torch.uint16)
    ad = to_dev_bf16(a)
    bd = to_dev_bf16(b)
    biasd = None if bias_bits is None else to_dev(bias_bits.view(np.int16)).view(torch.uint16)
    y, h = ops.int4lora_forward(xd, pd, sd, ad, bd, scaling=alpha / r, group_size=group,
                                bias_bits=biasd)
    dx, da, db = ops.int4lora_backward(to_dev_bf16(gy), xd, pd, sd, ad, bd, h, scaling=alpha / r,
                                       group_size=group)
    torch.cuda.synchronize()
    assert_bf16_close(from_dev(h), h_o, what="h")
    assert_bf16_close(from_dev(y), y_o, what="y")
    assert_bf16_close(from_dev(dx), dx_o, what="dx")
    assert_bf16_close(from_dev(da), da_o, min_equal=BF16_MIN_EQUAL_TOKEN_SUM, what="dA")
    assert_bf16_close(from_dev(db), db_o, min_equal=BF16_MIN_EQUAL_TOKEN_SUM, what="dB")
    # dA / dB are float32 holding bf16-rounded values (reference: f32(bf16(.)))
    assert np.array_equal(bf16_values(from_dev(da)), from_dev(da))
    assert np.array_equal(bf16_values(from_dev(db)), from_dev(db))


def test_int4lora_fp32_policy_generic():
    """fp32 compute (no precision context): every op in float32."""

    m, k, n, r = 16, 64, 48, 4
    x, packed, scales, a, b, bias_bits, gy = _lora_case(m, k, n, r, None, seed=5)
    x = np.random.default_rng(1).standard_normal((m, k)).astype(np.float32)
    gy = np.random.default_rng(2).standard_normal((m, n)).astype(np.float32)
    y_o, h_o = olora.lora_forward(x, packed, scales, a, b, alpha=8.0, rank=r, bias_bits=bias_bits,
                                  compute="f32")
    dx_o, da_o, db_o = olora.lora_backward(gy, x, packed, scales, a, b, h_o, alpha=8.0, rank=r,
                                           compute="f32")
    pd = to_dev(packed)
    sd = to_dev(scales.view(np.int16)).view(torch.uint16)
    biasd = to_dev(bias_bits.view(np.int16)).view(torch.uint16)
    y, h = ops.int4lora_forward(to_dev(x), pd, sd, to_dev(a), to_dev(b), scaling=2.0,
                                bias_bits=biasd)
    dx, da, db = ops.int4lora_backward(to_dev(gy), to_dev(x), pd, sd, to_dev(a), to_dev(b), h,
                                       scaling=2.0)
    torch.cuda.synchronize()
    for got, want in ((y, y_o), (h, h_o), (dx, dx_o), (da, da_o), (db, db_o)):
        assert rel_l2(from_dev(got), want) < 1e-5


def test_int4lora_full_bert_ffn_shape():
    """BERT-base FFN up-projection at the benchmark size: x [4096, 768], W 768->3072."""

    m, k, n, r = 4096, 768, 3072, 16
    x, packed, scales, a, b, bias_bits, gy = _lora_case(m, k, n, r, None, seed=2024)
    y_o, h_o = olora.lora_forward(x, packed, scales, a, b, alpha=32.0, rank=r, bias_bits=bias_bits)
    dx_o, da_o, db_o = olora.lora_backward(gy, x, packed, scales, a, b, h_o, alpha=32.0, rank=r)
    xd = to_dev_bf16(x)
    pd = to_dev(packed)
    sd = to_dev(scales.view(np.int16)).view(torch.uint16)
    ad, bd = to_dev_bf16(a), to_dev_bf16(b)
    biasd = to_dev(bias_bits.view(np.int16)).view(torch.uint16)
    y, h = ops.int4lora_forward(xd, pd, sd, ad, bd, scaling=2.0, bias_bits=biasd)
    dx, da, db = ops.int4lora_backward(to_dev_bf16(gy), xd, pd, sd, ad, bd, h, scaling=2.0)
    torch.cuda.synchronize()
    for name, got, want in (("y", y, y_o), ("h", h, h_o), ("dx", dx, dx_o)):
        assert_bf16_close(from_dev(got), want, what=name)
    for name, got, want in (("dA", da, da_o), ("dB", db, db_o)):
        assert_bf16_close(from_dev(got), want, min_equal=BF16_MIN_EQUAL_TOKEN_SUM, what=name)


def test_merge_matches_oracle():
    n, k, r = 96, 128, 8
    g = rng(9)
    w = (g.standard_normal((n, k)) * 0.02).astype(np.float32)
    a = (g.standard_normal((r, k)) * 0.1).astype(np.float32)
    b = (g.standard_normal((n, r)) * 0.1).astype(np.float32)
    packed, scales = oint4.pack_int4(w)
    got = ops.int4_merge(to_dev(packed), to_dev(scales.view(np.int16)).view(torch.uint16),
                         to_dev(a), to_dev(b), alpha=16.0, rank=r, input_size=k)
    want = olora.merged_weight(packed, scales, a, b, alpha=16.0, rank=r, input_size=k)
    np.testing.assert_allclose(got.cpu().numpy(), want, rtol=1e-5, atol=1e-6)


def test_invalid_arguments_raise_before_launch():
    pd = torch.zeros((4, 4), dtype=torch.uint8, device="cuda")
    sd = torch.zeros(4, dtype=torch.uint16, device="cuda")
    with pytest.raises(ValueError):
        ops.int4_dequant(pd, sd, 8, group_size=3)
    x = torch.zeros((2, 8), dtype=torch.bfloat16, device="cuda")
    a = torch.zeros((9, 8), dtype=torch.bfloat16, device="cuda")
    b = torch.zeros((4, 9), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError):
        ops.int4lora_forward(x, pd, sd, a, b, scaling=1.0)


def test_cpu_tensor_is_rejected():
    with pytest.raises(RuntimeError):
        ops.int4_dequant(torch.zeros((4, 4), dtype=torch.uint8),
                         torch.zeros(4, dtype=torch.uint16), 8)


@pytest.mark.parametrize(
    "m,k,n,r,group,bias",
    [(1, 2048, 6144, 32, None, False), (4, 6144, 2048, 32, None, True),
     (16, 2048, 2048, 32, 64, False), (17, 1024, 640, 16, None, True),
     (64, 2048, 1024, 32, 64, True), (33, 384, 200, 8, 128, False), (2, 128, 70, 3, None, True),
     (9, 256, 48, 16, None, True), (40, 256, 300, 24, 64, False)],
)
def test_skinny_forward_matches_oracle(m, k, n, r, group, bias):
    """M <= 64 runs the split-K skinny kernels (rotating nothing: parity only),
    including one adapter block and one K split (K = 256), where every
    block finishes its own tile and the only adapter block sums h alone."""

    x, packed, scales, a, b, bias_bits, _ = _lora_case(m, k, n, r, group, seed=m + n, bias=bias)
    y_o, h_o = olora.lora_forward(x, packed, scales, a, b, alpha=float(r), rank=r,
                                  bias_bits=bias_bits, group_size=group)
    biasd = None if bias_bits is None else to_dev(bias_bits.view(np.int16)).view(torch.uint16)
    y, h = ops.int4lora_forward(to_dev_bf16(x), to_dev(packed),
                                to_dev(scales.view(np.int16)).view(torch.uint16), to_dev_bf16(a),
                                to_dev_bf16(b), scaling=1.0, group_size=group, bias_bits=biasd)
    torch.cuda.synchronize()
    assert_bf16_close(from_dev(h), h_o, what="h")
    assert_bf16_close(from_dev(y), y_o, what="y")


SKINNY_TILE_IDS = list(range(1, 16))


@pytest.mark.parametrize("tile", SKINNY_TILE_IDS)
@pytest.mark.parametrize("m,k,n,r,group", [(3, 1024, 200, 32, 64), (40, 640, 136, 16, None)])
def test_skinny_every_tile_shape_matches_oracle(tile, m, k, n, r, group):
    """Each row-tile x K-split shape of the one-launch skinny kernel, including
    ragged last tiles and last splits."""

    x, packed, scales, a, b, bias_bits, _ = _lora_case(m, k, n, r, group, seed=tile + m, bias=True)
    y_o, h_o = olora.lora_forward(x, packed, scales, a, b, alpha=2.0 * r, rank=r,
                                  bias_bits=bias_bits, group_size=group)
    biasd = to_dev(bias_bits.view(np.int16)).view(torch.uint16)
    with ops.tuning(skinny_tile=tile):
        y, h = ops.int4lora_forward(to_dev_bf16(x), to_dev(packed),
                                    to_dev(scales.view(np.int16)).view(torch.uint16),
                                    to_dev_bf16(a), to_dev_bf16(b), scaling=2.0, group_size=group,
                                    bias_bits=biasd)
    torch.cuda.synchronize()
    assert_bf16_close(from_dev(h), h_o, what="h")
    assert_bf16_close(from_dev(y), y_o, what="y")


@pytest.mark.parametrize("m,k,n,r,group", [(3, 1024, 200, 32, 64), (16, 640, 136, 48, None),
                                           (9, 256, 70, 5, 128), (1, 4096, 80, 64, 64),
                                           (2, 6144, 2048, 32, 64), (4, 384, 33, 8, None)])
@pytest.mark.parametrize("one", [0, 1])
def test_skinny_two_launch_matches_oracle(one, m, k, n, r, group):
    """The M <= 16 row-block path, forced: two launches, or the one-launch
    form (M <= 4 with the rank a multiple of 8; the others fall back to two
    launches) that hands the adapter partials to the weight blocks as tagged
    words. Ragged last row blocks, ranks that are not multiples of 8 and
    ranks above 32, several K slices."""

    x, packed, scales, a, b, bias_bits, _ = _lora_case(m, k, n, r, group, seed=m + r, bias=True)
    b = b * 50.0  # the adapter term comparable to the base product
    y_o, h_o = olora.lora_forward(x, packed, scales, a, b, alpha=2.0 * r, rank=r,
                                  bias_bits=bias_bits, group_size=group)
    biasd = to_dev(bias_bits.view(np.int16)).view(torch.uint16)
    with ops.tuning(skinny2=1, skinny2_one=one):
        y, h = ops.int4lora_forward(to_dev_bf16(x), to_dev(packed),
                                    to_dev(scales.view(np.int16)).view(torch.uint16),
                                    to_dev_bf16(a), to_dev_bf16(b), scaling=2.0, group_size=group,
                                    bias_bits=biasd)
    torch.cuda.synchronize()
    assert_bf16_close(from_dev(h), h_o, what="h")
    assert_bf16_close(from_dev(y), y_o, what="y")


def test_skinny_one_launch_consecutive_calls_match_oracle():
    """Twelve back-to-back calls with different inputs (more calls than
    slots of arrival words, so slots are reused): each result matches the
    oracle, so no call reads an h published by an earlier one."""

    k, n, r = 4096, 320, 32
    base = _lora_case(4, k, n, r, 64, seed=5, bias=True)
    _, packed, scales, a, b, bias_bits, _ = base
    b = b * 50.0  # the adapter term comparable to the base product
    pd = to_dev(packed)
    sd = to_dev(scales.view(np.int16)).view(torch.uint16)
    ad, bd = to_dev_bf16(a), to_dev_bf16(b)
    biasd = to_dev(bias_bits.view(np.int16)).view(torch.uint16)
    xs, outs = [], []
    for i in range(12):
        m = 1 + i % 4
        x = bf16_values(rng(100 + i).standard_normal((m, k)))
        xs.append(x)
        outs.append(ops.int4lora_forward(to_dev_bf16(x), pd, sd, ad, bd, scaling=1.0,
                                         group_size=64, bias_bits=biasd))
    torch.cuda.synchronize()
    for x, (y, h) in zip(xs, outs):
        y_o, h_o = olora.lora_forward(x, packed, scales, a, b, alpha=float(r), rank=r,
                                      bias_bits=bias_bits, group_size=64)
        assert_bf16_close(from_dev(h), h_o, what="h")
        assert_bf16_close(from_dev(y), y_o, what="y")


@pytest.mark.parametrize("m,k", [(8, 2048), (2, 2048), (1, 4096)])
def test_skinny_graph_replays_and_repeats_are_bit_identical(m, k):
    """The arrival words of the M > 4 one-launch kernel (M = 8: per-tile
    split counters) return to their resting value after each call, and the
    M <= 4 one-launch form (M = 2 and 1) tags its partials per launch: eager
    repeats and graph replays give the same bits."""

    n, r = 1536, 32
    x, packed, scales, a, b, bias_bits, _ = _lora_case(m, k, n, r, 64, seed=91, bias=False)
    xd, pd = to_dev_bf16(x), to_dev(packed)
    sd = to_dev(scales.view(np.int16)).view(torch.uint16)
    ad, bd = to_dev_bf16(a), to_dev_bf16(b)

    def call():
        return ops.int4lora_forward(xd, pd, sd, ad, bd, scaling=1.0, group_size=64)

    y0, h0 = call()
    y1, h1 = call()
    torch.cuda.synchronize()
    assert torch.equal(y0, y1) and torch.equal(h0, h1)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        call()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        yg, hg = call()
    for _ in range(4):
        yg.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(yg, y0) and torch.equal(hg, h0)
        # eager work between replays reuses the allocator's blocks
        ye, _ = call()
        torch.cuda.synchronize()
        assert torch.equal(ye, y0)


@pytest.mark.parametrize("m,k,n,r,group", [(1, 2048, 6144, 32, 64), (4, 6144, 2048, 32, 64),
                                           (2, 2048, 2048, 64, None), (3, 1024, 1000, 24, 64),
                                           (1, 8192, 512, 40, 64), (4, 512, 96, 8, None)])
def test_skinny_one_launch_h_equals_two_launches(m, k, n, r, group):
    """The one-launch form sums the same partials in the same order as the
    two-launch form's finishing launch: h is bit-identical; y matches the
    oracle."""

    x, packed, scales, a, b, bias_bits, _ = _lora_case(m, k, n, r, group, seed=7 * m + r, bias=True)
    b = b * 50.0
    args = (to_dev_bf16(x), to_dev(packed), to_dev(scales.view(np.int16)).view(torch.uint16),
            to_dev_bf16(a), to_dev_bf16(b))
    biasd = to_dev(bias_bits.view(np.int16)).view(torch.uint16)
    out = {}
    for one in (0, 1):
        with ops.tuning(skinny2_one=one):
            out[one] = ops.int4lora_forward(*args, scaling=2.0, group_size=group, bias_bits=biasd)
    torch.cuda.synchronize()
    assert torch.equal(out[0][1].view(torch.uint16), out[1][1].view(torch.uint16))
    y_o, h_o = olora.lora_forward(x, packed, scales, a, b, alpha=2.0 * r, rank=r,
                                  bias_bits=bias_bits, group_size=group)
    assert_bf16_close(from_dev(out[1][0]), y_o, what="y")
    assert_bf16_close(from_dev(out[1][1]), h_o, what="h")


def test_skinny_one_launch_graph_replays_follow_new_inputs():
    """A graph of one M = 1 one-launch call replayed with new x each time
    (the launch's parameters, slot included, stay the same): every replay
    equals the two-launch form on the same x, so no replay takes the
    partials its previous replay left in the slot."""

    m, k, n, r = 1, 2048, 1536, 32
    x, packed, scales, a, b, _, _ = _lora_case(m, k, n, r, 64, seed=301, bias=False)
    b = b * 50.0
    xd, pd = to_dev_bf16(x), to_dev(packed)
    sd = to_dev(scales.view(np.int16)).view(torch.uint16)
    ad, bd = to_dev_bf16(a), to_dev_bf16(b)

    def call():
        return ops.int4lora_forward(xd, pd, sd, ad, bd, scaling=1.0, group_size=64)

    with ops.tuning(skinny2_one=1):
        call()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            call()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            yg, hg = call()
    for i in range(6):
        xi = bf16_values(rng(400 + i).standard_normal((m, k)))
        xd.copy_(to_dev_bf16(xi))
        graph.replay()
        torch.cuda.synchronize()
        with ops.tuning(skinny2_one=0):
            y0, h0 = call()
        torch.cuda.synchronize()
        assert torch.equal(hg.view(torch.uint16), h0.view(torch.uint16)), i
        y_o, _ = olora.lora_forward(xi, packed, scales, a, b, alpha=float(r), rank=r,
                                    group_size=64)
        assert_bf16_close(from_dev(yg), y_o, what="y")
    assert ops.check_device_errors() == 0


@pytest.mark.parametrize("group", [None, 64])
def test_int4lora_empty_batch(group):
    """Zero tokens: empty outputs and all-zero adapter gradients, as the
    reference's dense product over an empty batch gives; the empty tensors'
    null data pointers are accepted."""

    k, n, r = 256, 192, 16
    _, packed, scales, a, b, bias_bits, _ = _lora_case(1, k, n, r, group, seed=44)
    pd = to_dev(packed)
    sd = to_dev(scales.view(np.int16)).view(torch.uint16)
    ad = to_dev_bf16(a)
    bd = to_dev_bf16(b)
    biasd = to_dev(bias_bits.view(np.int16)).view(torch.uint16)
    x = torch.empty((0, k), dtype=torch.bfloat16, device="cuda")
    gy = torch.empty((0, n), dtype=torch.bfloat16, device="cuda")
    y, h = ops.int4lora_forward(x, pd, sd, ad, bd, scaling=2.0, group_size=group, bias_bits=biasd)
    dx, da, db = ops.int4lora_backward(gy, x, pd, sd, ad, bd, h, scaling=2.0, group_size=group)
    dz, dgate, da2, db2 = ops.int4lora_backward_act(gy, x, pd, sd, ad, bd, h, activation="gelu",
                                                    z=torch.empty((0, k), dtype=torch.bfloat16,
                                                                  device="cuda"),
                                                    scaling=2.0, group_size=group)
    torch.cuda.synchronize()
    assert y.shape == (0, n) and h.shape == (0, r) and dx.shape == (0, k) and dz.shape == (0, k)
    assert dgate is None
    for t, shape in ((da, (r, k)), (db, (n, r)), (da2, (r, k)), (db2, (n, r))):
        assert t.shape == shape and t.dtype == torch.float32
        assert torch.count_nonzero(t).item() == 0


def test_module_empty_batch_gradients_are_zero():
    import representax_amd as rx

    lin = rx.Linear.init(256, 192, key=1, scale=0.02, bias=True, device="cuda")
    layer = rx.QuantizedLoRALinear.from_linear(lin, rank=16, alpha=32.0, key=3)
    x = torch.empty((0, 256), dtype=torch.bfloat16, device="cuda", requires_grad=True)
    bf = rx.resolve_precision_policy(rx.PrecisionConfig.bfloat16_mixed())
    with rx.precision_context(bf):
        y = layer(x)
    y.sum().backward()
    torch.cuda.synchronize()
    assert y.shape == (0, 192)
    assert x.grad.shape == (0, 256)
    assert torch.count_nonzero(layer.lora_a.grad).item() == 0
    assert torch.count_nonzero(layer.lora_b.grad).item() == 0


@pytest.mark.parametrize("m,k,n,r,group,bias", [(64, 256, 192, 16, None, True),
                                                (300, 512, 320, 8, 64, False),
                                                (5, 100, 52, 3, None, True)])
def test_promoted_forward_backward_matches_oracle(m, k, n, r, group, bias):
    """No precision policy on bf16 activations with float32 masters: the
    bf16 base product (MFMA GEMM where the shape allows it, generic kernel
    otherwise), the float32 adapter and output, and their transpose."""

    x, packed, scales, a, b, bias_bits, _ = _lora_case(m, k, n, r, group, seed=m + 5 * r,
                                                       bias=bias)
    b = b * 20.0
    gy = rng(77 + m).standard_normal((m, n)).astype(np.float32)
    alpha = 3.0 * r
    y_o, h_o = olora.lora_forward(x, packed, scales, a, b, alpha=alpha, rank=r,
                                  bias_bits=bias_bits, group_size=group, compute="promoted")
    pd = to_dev(packed)
    sd = to_dev(scales.view(np.int16)).view(torch.uint16)
    biasd = None if bias_bits is None else to_dev(bias_bits.view(np.int16)).view(torch.uint16)
    xd = to_dev_bf16(x)
    y, h = ops.int4lora_forward_promoted(xd, pd, sd, to_dev(a), to_dev(b), scaling=alpha / r,
                                         group_size=group, bias_bits=biasd)
    dx, da, db = ops.int4lora_backward_promoted(to_dev(gy), xd, pd, sd, to_dev(a), to_dev(b), h,
                                                scaling=alpha / r, group_size=group)
    torch.cuda.synchronize()
    assert y.dtype == torch.float32 and h.dtype == torch.float32 and dx.dtype == torch.bfloat16
    dx_o, da_o, db_o = olora.lora_backward(gy, x, packed, scales, a, b, from_dev(h), alpha=alpha,
                                           rank=r, group_size=group, compute="promoted")
    assert rel_l2(from_dev(h), h_o) < 1e-5
    assert rel_l2(from_dev(y), y_o) < TOL
    assert rel_l2(from_dev(dx), dx_o) < TOL
    assert rel_l2(from_dev(da), da_o) < 1e-4
    assert rel_l2(from_dev(db), db_o) < 1e-4


def test_module_without_policy_promotes_to_float32():
    """QuantizedLoRALinear called on bf16 activations with no precision
    context (the reference's inference setting) returns float32 and sends
    float32 gradients to the masters."""

    import representax_amd as rx

    lin = rx.Linear.init(256, 192, key=1, scale=0.02, bias=True, device="cuda")
    layer = rx.QuantizedLoRALinear.from_linear(lin, rank=8, alpha=16.0, key=3)
    with torch.no_grad():
        layer.lora_b.normal_(0.0, 0.5)
    x = to_dev_bf16(bf16_values(rng(5).standard_normal((48, 256)))).requires_grad_(True)
    y = layer(x)
    assert y.dtype == torch.float32
    gy = torch.from_numpy(rng(6).standard_normal((48, 192)).astype(np.float32)).cuda()
    y.backward(gy)
    torch.cuda.synchronize()
    assert x.grad.dtype == torch.bfloat16 and layer.lora_a.grad.dtype == torch.float32
    packed = layer.packed_weight.cpu().numpy()
    scales = layer.scale_bits.view(torch.int16).cpu().numpy().view(np.uint16)
    bias = layer.bias_bits.view(torch.int16).cpu().numpy().view(np.uint16)
    a = layer.lora_a.detach().cpu().numpy()
    b = layer.lora_b.detach().cpu().numpy()
    xh = from_dev(x.detach())
    y_o, h_o = olora.lora_forward(xh, packed, scales, a, b, alpha=16.0, rank=8, bias_bits=bias,
                                  compute="promoted")
    dx_o, da_o, db_o = olora.lora_backward(gy.cpu().numpy(), xh, packed, scales, a, b, h_o,
                                           alpha=16.0, rank=8, compute="promoted")
    assert rel_l2(from_dev(y.detach()), y_o) < TOL
    assert rel_l2(from_dev(x.grad), dx_o) < TOL
    assert rel_l2(layer.lora_a.grad.cpu().numpy(), da_o) < 1e-4
    assert rel_l2(layer.lora_b.grad.cpu().numpy(), db_o) < 1e-4


@pytest.mark.parametrize("form", ["skinny", "skinny_one"])
def test_skinny_slots_recover_after_expired_waits(form):
    """Force the one-launch kernels' bounded waits to expire from the host (a
    one-poll spin limit; every kernel still exits normally), then run more
    calls than there are slots with the default limit: each equals the
    result taken before, bit for bit, so no expired call left its slot
    dirty (M > 4) or handed its late partials to a later call (M <= 4).
    Expired calls are reported through the device error word."""

    if form == "skinny":
        m, k, knobs = 8, 2048, dict(skinny2=0)
    else:
        m, k, knobs = 2, 4096, dict(skinny2=1, skinny2_one=1)
    n, r = 1536, 32
    x, packed, scales, a, b, _, _ = _lora_case(m, k, n, r, 64, seed=123, bias=False)
    b = b * 50.0
    xd, pd = to_dev_bf16(x), to_dev(packed)
    sd = to_dev(scales.view(np.int16)).view(torch.uint16)
    ad, bd = to_dev_bf16(a), to_dev_bf16(b)

    def call():
        return ops.int4lora_forward(xd, pd, sd, ad, bd, scaling=1.0, group_size=64)

    with ops.tuning(**knobs):
        assert ops.check_device_errors() == 0
        y0, h0 = call()
        torch.cuda.synchronize()
        y_o, h_o = olora.lora_forward(x, packed, scales, a, b, alpha=float(r), rank=r,
                                      group_size=64)
        assert_bf16_close(from_dev(y0), y_o, what="y")
        with ops.tuning(spin_limit=1):
            forced = [call() for _ in range(12)]
        torch.cuda.synchronize()
        expired = 0
        try:
            ops.check_device_errors()
        except ops.nat.DeviceError:
            expired = 1
        nan_calls = sum(int(torch.isnan(y.float()).any().item()) for y, _ in forced)
        # a call whose wait expired holds NaN; one that did not equals y0
        assert expired == (nan_calls > 0)
        for y, h in forced:
            if not torch.isnan(y.float()).any():
                assert torch.equal(y, y0)
        for _ in range(20):
            y1, h1 = call()
            torch.cuda.synchronize()
            assert torch.equal(y1, y0) and torch.equal(h1, h0)
        assert ops.check_device_errors() == 0


@pytest.mark.parametrize("rank_blocks", [16, 100, 384, 2048])
@pytest.mark.parametrize("m,k,n,r,group", [(700, 320, 448, 16, 64), (1000, 256, 192, 32, None)])
def test_backward_every_token_split(rank_blocks, m, k, n, r, group):
    """dA / dB under every token-split plan the rank-r reduction can take (one
    to many token chunks per tile, ragged last chunk), against the oracle."""

    x, packed, scales, a, b, bias_bits, gy = _lora_case(m, k, n, r, group, seed=m + rank_blocks)
    alpha = 2.0 * r
    _, h_o = olora.lora_forward(x, packed, scales, a, b, alpha=alpha, rank=r, group_size=group)
    dx_o, da_o, db_o = olora.lora_backward(gy, x, packed, scales, a, b, h_o, alpha=alpha, rank=r,
                                           group_size=group)
    xd = to_dev_bf16(x)
    pd = to_dev(packed)
    sd = to_dev(scales.view(np.int16)).view(torch.uint16)
    ad = to_dev_bf16(a)
    bd = to_dev_bf16(b)
    with ops.tuning(rank_blocks=rank_blocks):
        _, h = ops.int4lora_forward(xd, pd, sd, ad, bd, scaling=alpha / r, group_size=group)
        dx, da, db = ops.int4lora_backward(to_dev_bf16(gy), xd, pd, sd, ad, bd, h,
                                           scaling=alpha / r, group_size=group)
    torch.cuda.synchronize()
    assert_bf16_close(from_dev(dx), dx_o, what="dx")
    assert_bf16_close(from_dev(da), da_o, min_equal=BF16_MIN_EQUAL_TOKEN_SUM, what="dA")
    assert_bf16_close(from_dev(db), db_o, min_equal=BF16_MIN_EQUAL_TOKEN_SUM, what="dB")
    assert np.array_equal(bf16_values(from_dev(da)), from_dev(da))
    assert np.array_equal(bf16_values(from_dev(db)), from_dev(db))
