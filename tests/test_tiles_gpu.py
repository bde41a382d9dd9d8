"""Every GEMM tile shape the planners can pick, with every epilogue, and the
train-step linears at their full sizes, against the oracle (GPU).

The INT4 fused forward GEMM and the bf16 input-gradient GEMM each have
several tile shapes; the planners pick them by grid size and by the scale
footprint (group 64 at K = 6144 selects the 256-row INT4 tile). Each tile is
forced here with the tuning knobs on ragged shapes (edges in M, N and the
output width), with the plain, GELU, SiLU-gated and add epilogues, and its
result is compared with the oracle and, bit for bit, with every other tile:
a tile only changes which workgroup computes an output, not the order of
its K accumulation.

The full-size cases are the linears of the BERT-base step (32,768 tokens,
group 64, rank 16) and of the Qwen3-VL-2B-shaped step (4096 of its 16,384
tokens, group 64, rank 32). dA and dB are checked over the whole batch; y,
h and dx over a seeded subset of 512 rows (they are row-separable), so the
float64 oracle finishes in seconds.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import act as oact
from oracle import int4 as oint4
from oracle import lora as olora
from oracle.codecs import f32_to_bf16_bits
from representax_amd import ops
from tests.helpers import (BF16_MIN_EQUAL_TOKEN_SUM, assert_act_bits, assert_bf16_close,
                           bf16_values, bits_from_dev, from_dev, rng, to_dev, to_dev_bf16)

pytestmark = pytest.mark.gpu

INT4_TILES = [3, 10, 11, 1, 12, 7, 17]  # 64x128, 128x128 two / three stages, 256x128 three /
                                         # two stages, 256x256; B dequantized once per
                                         # workgroup: 256x192
BF16_TILES = [6, 9, 5, 4, 13, 8]  # 64x128, 128x96, 128x128, 256x128 two / three stages, 256x256
NO_ACT_TILES = {7, 8}           # sweep-only shapes without activation epilogues


def _params(g, n, k, r, group, bias, b_scale=20.0):
    w = (g.standard_normal((n, k)) * 0.02).astype(np.float32)
    packed, scales = oint4.pack_int4(w, group)
    a = (g.standard_normal((r, k)) * 0.05).astype(np.float32)
    b = (g.standard_normal((n, r)) * 0.05 * b_scale).astype(np.float32)
    bias_bits = f32_to_bf16_bits((g.standard_normal(n) * 0.5).astype(np.float32)) if bias else None
    return dict(packed=packed, scales=scales, a=a, b=b, bias=bias_bits, alpha=2.0 * r, r=r,
                group=group)


def _dev(p):
    return dict(packed=to_dev(p["packed"]),
                scales=to_dev(p["scales"].view(np.int16)).view(torch.uint16),
                a=to_dev_bf16(p["a"]), b=to_dev_bf16(p["b"]),
                bias=None if p["bias"] is None else to_dev(p["bias"].view(np.int16)).view(torch.uint16),
                scaling=float(p["alpha"] / p["r"]), group=p["group"])


def _forward(d, x, activation, gate):
    if activation == "none":
        y, h = ops.int4lora_forward(x, d["packed"], d["scales"], d["a"], d["b"],
                                    scaling=d["scaling"], group_size=d["group"],
                                    bias_bits=d["bias"])
        return y, y, h
    return ops.int4lora_forward_act(x, d["packed"], d["scales"], d["a"], d["b"],
                                    activation=activation, scaling=d["scaling"],
                                    group_size=d["group"], bias_bits=d["bias"], gate=gate)


# (m, k, n, r, group): M, N and K ragged against every tile (300 rows; 320 and
# 704 columns are not multiples of 128 or 256), ranks 16 / 32 / 64 (one, two
# and four 16-rank epilogue blocks), per-row and group scales
FWD_SHAPES = [(300, 704, 320, 16, 64), (300, 512, 448, 32, None), (264, 256, 200, 64, 32)]


@pytest.mark.parametrize("activation", ["none", "gelu", "silu_mul"])
@pytest.mark.parametrize("m,k,n,r,group", FWD_SHAPES)
def test_int4_forward_every_tile(activation, m, k, n, r, group):
    g = rng(1000 + m + n + r)
    p = _params(g, n, k, r, group, bias=True)
    d = _dev(p)
    x = bf16_values(g.standard_normal((m, k)))
    gate = bf16_values(g.standard_normal((m, n)) * 2.0)
    xd = to_dev_bf16(x)
    gated = to_dev_bf16(gate) if activation == "silu_mul" else None
    z_o, h_o = olora.lora_forward(x, p["packed"], p["scales"], p["a"], p["b"], alpha=p["alpha"],
                                  rank=r, bias_bits=p["bias"], group_size=group)
    results = {}
    for tile in INT4_TILES:
        if activation != "none" and tile in NO_ACT_TILES:
            continue
        with ops.tuning(int4_tile=tile):
            results[tile] = _forward(d, xd, activation, gated)
    torch.cuda.synchronize()
    first = None
    for tile, (y, z, h) in results.items():
        assert_bf16_close(from_dev(z), z_o, what=f"tile {tile} z")
        assert_bf16_close(from_dev(h), h_o, what=f"tile {tile} h")
        if activation != "none":
            want = oact.act_forward(activation, from_dev(z),
                                    gate if activation == "silu_mul" else None)
            assert_act_bits(bits_from_dev(y), want)
        if first is None:
            first = (tile, y, z)
        else:
            assert torch.equal(z, first[2]), (tile, first[0])
            assert torch.equal(y, first[1]), (tile, first[0])


def _backward(d, gy, x, h, activation, z, gate):
    if activation == "none":
        dx, d_a, d_b = ops.int4lora_backward(gy, x, d["packed"], d["scales"], d["a"], d["b"], h,
                                             scaling=d["scaling"], group_size=d["group"])
        return dx, None, d_a, d_b
    return ops.int4lora_backward_act(gy, x, d["packed"], d["scales"], d["a"], d["b"], h,
                                     activation=activation, z=z, gate=gate, scaling=d["scaling"],
                                     group_size=d["group"])


# (m, k, n, r, group) of the linear whose input gradient is computed: the dx
# GEMM's output is [m, k] (k ragged against 96, 128 and 256) and it reduces
# over n
BWD_SHAPES = [(300, 704, 320, 16, 64), (300, 448, 512, 32, None), (264, 192, 256, 64, 32)]


@pytest.mark.parametrize("activation", ["none", "gelu", "silu_mul", "add"])
@pytest.mark.parametrize("m,k,n,r,group", BWD_SHAPES)
def test_bf16_dx_every_tile(activation, m, k, n, r, group):
    g = rng(2000 + m + k + r)
    p = _params(g, n, k, r, group, bias=False)
    d = _dev(p)
    x = bf16_values(g.standard_normal((m, k)))
    z = bf16_values(g.standard_normal((m, k)) * 2.0)
    gate = bf16_values(g.standard_normal((m, k)) * 2.0)
    gy = bf16_values(g.standard_normal((m, n)))
    xd, gyd, zd = to_dev_bf16(x), to_dev_bf16(gy), to_dev_bf16(z)
    gated = to_dev_bf16(gate) if activation == "silu_mul" else None
    _, h = ops.int4lora_forward(xd, d["packed"], d["scales"], d["a"], d["b"],
                                scaling=d["scaling"], group_size=group)
    torch.cuda.synchronize()
    dx_o, da_o, db_o = olora.lora_backward(gy, x, p["packed"], p["scales"], p["a"], p["b"],
                                           from_dev(h), alpha=p["alpha"], rank=r,
                                           group_size=group)
    results = {}
    for tile in BF16_TILES:
        if activation != "none" and tile in NO_ACT_TILES:
            continue
        with ops.tuning(bf16_tile=tile):
            results[tile] = _backward(d, gyd, xd, h, activation, zd, gated)
            if activation != "none":
                # the plain input gradient on the same tile, for the
                # activation's exact backward
                results[tile] = results[tile] + (_backward(d, gyd, xd, h, "none", None, None)[0],)
    torch.cuda.synchronize()
    first = None
    for tile, res in results.items():
        out, dgate, d_a, d_b = res[:4]
        dx = out if activation == "none" else res[4]
        assert_bf16_close(from_dev(dx), dx_o, what=f"tile {tile} dx")
        assert_bf16_close(from_dev(d_a), da_o, min_equal=BF16_MIN_EQUAL_TOKEN_SUM,
                          what=f"tile {tile} dA")
        assert_bf16_close(from_dev(d_b), db_o, min_equal=BF16_MIN_EQUAL_TOKEN_SUM,
                          what=f"tile {tile} dB")
        if activation != "none":
            want_dz, want_dg = oact.act_backward(activation, from_dev(dx), z,
                                                 gate if activation == "silu_mul" else None)
            assert_act_bits(bits_from_dev(out), want_dz)
            if activation == "silu_mul":
                assert_act_bits(bits_from_dev(dgate), want_dg)
        if first is None:
            first = (tile, out, dgate)
        else:
            assert torch.equal(out, first[1]), (tile, first[0])
            if dgate is not None:
                assert torch.equal(dgate, first[2]), (tile, first[0])


# Row-blocks per band of the tile order, forced: powers of two, bands that do
# not divide the tile rows (3, 5: a short last band) and one wider than the
# grid (64: clamped to the tile rows)
BANDS = [1, 2, 3, 5, 64]


@pytest.mark.parametrize("tile", [3, 10, 1])
def test_int4_forward_every_band(tile):
    """The tile order only moves tiles between workgroups: every band gives
    the same bits, and those match the oracle."""

    m, k, n, r, group = 1100, 512, 704, 16, 64
    g = rng(4000 + tile)
    p = _params(g, n, k, r, group, bias=True)
    d = _dev(p)
    x = bf16_values(g.standard_normal((m, k)))
    xd = to_dev_bf16(x)
    z_o, h_o = olora.lora_forward(x, p["packed"], p["scales"], p["a"], p["b"], alpha=p["alpha"],
                                  rank=r, bias_bits=p["bias"], group_size=group)
    results = {}
    for band in BANDS:
        with ops.tuning(int4_tile=tile, gemm_band=band):
            results[band] = _forward(d, xd, "none", None)
    torch.cuda.synchronize()
    assert_bf16_close(from_dev(results[1][0]), z_o, what=f"tile {tile} band 1 y")
    assert_bf16_close(from_dev(results[1][2]), h_o, what=f"tile {tile} band 1 h")
    for band, (y, _, _) in results.items():
        assert torch.equal(y, results[1][0]), (tile, band)


@pytest.mark.parametrize("tile", [6, 5, 4])
def test_bf16_dx_every_band(tile):
    m, k, n, r, group = 1100, 704, 512, 16, 64
    g = rng(4100 + tile)
    p = _params(g, n, k, r, group, bias=False)
    d = _dev(p)
    x = bf16_values(g.standard_normal((m, k)))
    gy = bf16_values(g.standard_normal((m, n)))
    xd, gyd = to_dev_bf16(x), to_dev_bf16(gy)
    _, h = ops.int4lora_forward(xd, d["packed"], d["scales"], d["a"], d["b"],
                                scaling=d["scaling"], group_size=group)
    torch.cuda.synchronize()
    dx_o, _, _ = olora.lora_backward(gy, x, p["packed"], p["scales"], p["a"], p["b"], from_dev(h),
                                     alpha=p["alpha"], rank=r, group_size=group)
    results = {}
    for band in BANDS:
        with ops.tuning(bf16_tile=tile, gemm_band=band):
            results[band] = _backward(d, gyd, xd, h, "none", None, None)[0]
    torch.cuda.synchronize()
    assert_bf16_close(from_dev(results[1]), dx_o, what=f"tile {tile} band 1 dx")
    for band, dx in results.items():
        assert torch.equal(dx, results[1]), (tile, band)


# Full-size linears of the two train steps: (m, k, n, r, group, activation)
FULL = [
    # BERT-base, 64 x 256 tokens: Q/K/V/O, FFN up (with GELU), FFN down
    pytest.param(32768, 768, 768, 16, 64, "none", id="bert-qkvo"),
    pytest.param(32768, 768, 3072, 16, 64, "gelu", id="bert-ffn-up"),
    pytest.param(32768, 3072, 768, 16, 64, "none", id="bert-ffn-down"),
    # Qwen3-VL-2B-shaped text tower, 4096 tokens: q/o, k/v, gate/up, down
    pytest.param(4096, 2048, 2048, 32, 64, "none", id="qwen3-q-o"),
    pytest.param(4096, 2048, 1024, 32, 64, "none", id="qwen3-k-v"),
    pytest.param(4096, 2048, 6144, 32, 64, "silu_mul", id="qwen3-gate-up"),
    pytest.param(4096, 6144, 2048, 32, 64, "none", id="qwen3-down"),
]


@pytest.mark.parametrize("m,k,n,r,group,activation", FULL)
def test_train_step_linears_full_size(m, k, n, r, group, activation):
    """Forward (with the step's activation epilogue) and backward at the
    sizes the train steps run, on the tiles the planners pick there."""

    g = rng(3000 + k + n)
    p = _params(g, n, k, r, group, bias=True, b_scale=10.0)
    d = _dev(p)
    x = bf16_values(g.standard_normal((m, k)))
    gate = bf16_values(g.standard_normal((m, n)) * 2.0) if activation == "silu_mul" else None
    gy = bf16_values(g.standard_normal((m, n)))
    xd, gyd = to_dev_bf16(x), to_dev_bf16(gy)
    y, z, h = _forward(d, xd, activation, None if gate is None else to_dev_bf16(gate))
    dx, _, d_a, d_b = _backward(d, gyd, xd, h, "none", None, None)
    torch.cuda.synchronize()
    rows = np.sort(rng(4000 + m).choice(m, size=min(m, 512), replace=False))
    z_o, h_o = olora.lora_forward(x[rows], p["packed"], p["scales"], p["a"], p["b"],
                                  alpha=p["alpha"], rank=r, bias_bits=p["bias"], group_size=group)
    hg = from_dev(h)
    assert_bf16_close(from_dev(z)[rows], z_o, what="y")
    assert_bf16_close(hg[rows], h_o, what="h")
    if activation != "none":
        want = oact.act_forward(activation, from_dev(z)[rows],
                                None if gate is None else gate[rows])
        assert_act_bits(bits_from_dev(y)[rows], want)
    dx_o, da_o, db_o = olora.lora_backward(gy, x, p["packed"], p["scales"], p["a"], p["b"], hg,
                                           alpha=p["alpha"], rank=r, group_size=group,
                                           dx_rows=rows)
    assert_bf16_close(from_dev(dx)[rows], dx_o, what="dx")
    assert_bf16_close(from_dev(d_a), da_o, min_equal=BF16_MIN_EQUAL_TOKEN_SUM, what="dA")
    assert_bf16_close(from_dev(d_b), db_o, min_equal=BF16_MIN_EQUAL_TOKEN_SUM, what="dB")


# The input gradient read from the packed weight (no bf16 W_b^T): output
# widths k that are multiples of 128, reductions n over whole 64-row slices
# (n = 64: a single slice), ragged M, per-row and group-64 scales, ranks
# 16 / 32 / 64
PACKED_DX_TILES = [16, 15, 14]  # 64x128, 128x128, 256x128
PACKED_DX_SHAPES = [(300, 768, 320, 16, 64), (300, 384, 512, 32, None), (264, 256, 192, 64, 64),
                    (100, 128, 64, 16, None)]


@pytest.mark.parametrize("activation", ["none", "gelu", "silu_mul", "add"])
@pytest.mark.parametrize("m,k,n,r,group", PACKED_DX_SHAPES)
def test_packed_dx_every_tile(activation, m, k, n, r, group):
    """dx = g . W_b from the packed weight, dequantized in the GEMM, on every
    tile: the oracle's values, and bit for bit the input gradient computed
    from a bf16 W_b^T (the K accumulation order is the same)."""

    g = rng(5000 + m + k + n + r)
    p = _params(g, n, k, r, group, bias=False)
    d = _dev(p)
    x = bf16_values(g.standard_normal((m, k)))
    z = bf16_values(g.standard_normal((m, k)) * 2.0)
    gate = bf16_values(g.standard_normal((m, k)) * 2.0)
    gy = bf16_values(g.standard_normal((m, n)))
    xd, gyd, zd = to_dev_bf16(x), to_dev_bf16(gy), to_dev_bf16(z)
    gated = to_dev_bf16(gate) if activation == "silu_mul" else None
    _, h = ops.int4lora_forward(xd, d["packed"], d["scales"], d["a"], d["b"],
                                scaling=d["scaling"], group_size=group)
    with ops.tuning(dx_packed=0):
        want = _backward(d, gyd, xd, h, activation, zd, gated)
    results = {}
    for tile in PACKED_DX_TILES:
        with ops.tuning(bf16_tile=tile, dx_packed=1):
            results[tile] = _backward(d, gyd, xd, h, activation, zd, gated)
    torch.cuda.synchronize()
    if activation == "none":
        dx_o, da_o, db_o = olora.lora_backward(gy, x, p["packed"], p["scales"], p["a"], p["b"],
                                               from_dev(h), alpha=p["alpha"], rank=r,
                                               group_size=group)
        assert_bf16_close(from_dev(want[0]), dx_o, what="bf16 W_b^T dx")
    for tile, res in results.items():
        if activation == "none":
            assert_bf16_close(from_dev(res[0]), dx_o, what=f"tile {tile} dx")
        for i, name in enumerate(("out", "dgate", "dA", "dB")):
            if want[i] is None:
                assert res[i] is None
            else:
                assert torch.equal(res[i], want[i]), (tile, name)


@pytest.mark.parametrize("dx_packed,cases", [
    (1, [(300, 704, 320, 16, 64), (200, 256, 128, 16, 32)]),
    (-1, [(300, 768, 320, 16, 64)])])
def test_packed_dx_falls_back_where_not_allowed(dx_packed, cases):
    """Shapes the packed form does not take (an output width that is not a
    multiple of 128, 32-column groups), and every shape under the planner's
    default, run the bf16 W_b^T form unchanged."""

    for (m, k, n, r, group) in cases:
        g = rng(5100 + k + (group or 0))
        p = _params(g, n, k, r, group, bias=False)
        d = _dev(p)
        x = to_dev_bf16(bf16_values(g.standard_normal((m, k))))
        gy = to_dev_bf16(bf16_values(g.standard_normal((m, n))))
        _, h = ops.int4lora_forward(x, d["packed"], d["scales"], d["a"], d["b"],
                                    scaling=d["scaling"], group_size=group)
        with ops.tuning(dx_packed=0):
            want = _backward(d, gy, x, h, "none", None, None)
        with ops.tuning(dx_packed=dx_packed):
            got = _backward(d, gy, x, h, "none", None, None)
        torch.cuda.synchronize()
        assert torch.equal(got[0], want[0]) and torch.equal(got[2], want[2])
        assert torch.equal(got[3], want[3])
