"""Pin the oracle's FFN activations and fused blocks against torch's float64
routines, closed forms, symmetry identities and finite differences (CPU)."""

from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

from oracle import act as oact
from oracle import int4 as oint4
from oracle.codecs import bf16_round

GRID = np.concatenate([np.linspace(-12.0, 12.0, 4001), [0.0, 1e-30, -1e-30, 3.5e-8, -40.0, 40.0]])


def test_gelu_and_silu_match_torch_float64():
    t = torch.from_numpy(GRID)
    np.testing.assert_allclose(oact.gelu(GRID), F.gelu(t, approximate="none").numpy(),
                               rtol=1e-12, atol=1e-15)
    np.testing.assert_allclose(oact.silu(GRID), F.silu(t).numpy(), rtol=1e-12, atol=1e-15)


def test_closed_forms_and_symmetries():
    assert oact.gelu(0.0) == 0.0 and oact.silu(0.0) == 0.0
    z = GRID[np.abs(GRID) <= 8]
    # Phi(-z) = 1 - Phi(z)  =>  gelu(-z) = gelu(z) - z; same for silu
    np.testing.assert_allclose(oact.gelu(-z), oact.gelu(z) - z, atol=1e-13)
    np.testing.assert_allclose(oact.silu(-z), oact.silu(z) - z, atol=1e-13)
    assert abs(oact.gelu(10.0) - 10.0) < 1e-20 and abs(oact.gelu(-10.0)) < 1e-20
    assert oact.gelu_grad(0.0) == 0.5 and oact.silu_grad(0.0) == 0.5
    # gelu'(z) + gelu'(-z) = 1 (the z phi(z) terms cancel)
    np.testing.assert_allclose(oact.gelu_grad(z) + oact.gelu_grad(-z), 1.0, atol=1e-13)


def test_gelu_keeps_its_tail():
    """Phi through erfc: gelu(-10) = -10 Phi(-10) = -7.62e-23 (1 + erf would
    cancel to zero), gelu'(-10) from the same tail."""

    assert abs(oact.gelu(-10.0) / (-10.0 * 7.619853024160527e-24) - 1.0) < 1e-12
    np.testing.assert_allclose(oact.normal_cdf(-10.0), 7.619853024160527e-24, rtol=1e-12)


def test_derivatives_match_central_differences():
    z = np.linspace(-6.0, 6.0, 241)
    h = 1e-6
    np.testing.assert_allclose(oact.gelu_grad(z), (oact.gelu(z + h) - oact.gelu(z - h)) / (2 * h),
                               atol=1e-8)
    np.testing.assert_allclose(oact.silu_grad(z), (oact.silu(z + h) - oact.silu(z - h)) / (2 * h),
                               atol=1e-8)


def test_act_rounds_once_to_bf16():
    g = np.random.Generator(np.random.PCG64(3))
    z = bf16_round(g.standard_normal(1000) * 3)
    gate = bf16_round(g.standard_normal(1000) * 3)
    np.testing.assert_array_equal(oact.act_forward("gelu", z), bf16_round(oact.gelu(z)))
    np.testing.assert_array_equal(oact.act_forward("silu_mul", z, gate),
                                  bf16_round(oact.silu(gate) * z))
    d = bf16_round(g.standard_normal(1000))
    dsum, none = oact.act_backward("add", d, z)
    assert none is None
    np.testing.assert_array_equal(dsum, bf16_round(d.astype(np.float64) + z))
    du, dg = oact.act_backward("silu_mul", d, z, gate)
    np.testing.assert_array_equal(du, bf16_round(d * oact.silu(gate)))
    np.testing.assert_array_equal(dg, bf16_round(d * z * oact.silu_grad(gate)))


def _linear(g, n, k, r, alpha, compute):
    w = (g.standard_normal((n, k)) * 0.3).astype(np.float32)
    packed, scales = oint4.pack_int4(w)
    return dict(packed=packed, scale_bits=scales,
                lora_a=(g.standard_normal((r, k)) * 0.3).astype(np.float32),
                lora_b=(g.standard_normal((n, r)) * 0.3).astype(np.float32),
                alpha=alpha, rank=r, compute=compute)


def _fd_check(forward, backward_dx, x, seed):
    """Central differences of sum(y * G) in x against the backward's dx."""

    g = np.random.Generator(np.random.PCG64(seed))
    y = forward(x)
    gy = g.standard_normal(y.shape)
    dx = backward_dx(gy)
    h = 1e-6
    for idx in [(0, 0), (1, 3), (2, 5)]:
        xp, xm = x.copy(), x.copy()
        xp[idx] += h
        xm[idx] -= h
        num = (np.sum(forward(xp) * gy) - np.sum(forward(xm) * gy)) / (2 * h)
        assert abs(num - dx[idx]) < 1e-5 * max(1.0, abs(num)), (idx, num, dx[idx])


def test_gelu_mlp_backward_matches_finite_differences():
    g = np.random.Generator(np.random.PCG64(5))
    m, k, f, r = 3, 6, 10, 2
    up = _linear(g, f, k, r, 3.0, "f64")
    down = _linear(g, k, f, r, 3.0, "f64")
    x = g.standard_normal((m, k))

    def fwd(xv):
        return oact.gelu_mlp_forward(xv, up, down)[0]

    def bwd(gy):
        _, z, act, h_up, h_down = oact.gelu_mlp_forward(x, up, down)
        return oact.gelu_mlp_backward(gy, x, up, down, z, act, h_up, h_down)[0]

    _fd_check(fwd, bwd, x, 6)


def test_swiglu_mlp_backward_matches_finite_differences():
    g = np.random.Generator(np.random.PCG64(7))
    m, k, f, r = 3, 6, 10, 2
    gate = _linear(g, f, k, r, 3.0, "f64")
    up = _linear(g, f, k, r, 3.0, "f64")
    down = _linear(g, k, f, r, 3.0, "f64")
    x = g.standard_normal((m, k))

    def fwd(xv):
        return oact.swiglu_mlp_forward(xv, gate, up, down)[0]

    def bwd(gy):
        _, gg, u, act, h_gate, h_up, h_down = oact.swiglu_mlp_forward(x, gate, up, down)
        return oact.swiglu_mlp_backward(gy, x, gate, up, down, gg, u, act, h_gate, h_up,
                                        h_down)[0]

    _fd_check(fwd, bwd, x, 8)
