"""Activation epilogues (GELU, SiLU-gated product) fused into the INT4 + LoRA
GEMMs, and the fused FFN blocks, against the oracle (GPU)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from tests.helpers import (BF16_REL_TOL, assert_act_bits, bf16_values, bits_from_dev, from_dev,
                           rel_l2, rng, to_dev, to_dev_bf16)
from oracle import act as oact
from oracle import int4 as oint4
from oracle import lora as olora
from oracle.codecs import f32_to_bf16_bits
from representax_amd import ops

pytestmark = pytest.mark.gpu

TOL = BF16_REL_TOL


def _linear(g, n, k, r, group, bias, b_scale=1.0):
    w = (g.standard_normal((n, k)) * 0.02).astype(np.float32)
    packed, scales = oint4.pack_int4(w, group)
    a = (g.standard_normal((r, k)) * 0.05).astype(np.float32)
    b = (g.standard_normal((n, r)) * 0.05 * b_scale).astype(np.float32)
    bias_bits = f32_to_bf16_bits((g.standard_normal(n) * 0.5).astype(np.float32)) if bias else None
    return dict(packed=packed, scale_bits=scales, lora_a=a, lora_b=b, alpha=2.0 * r, rank=r,
                bias_bits=bias_bits, group_size=group)


def _dev(p):
    return dict(packed=to_dev(p["packed"]),
                scale_bits=to_dev(p["scale_bits"].view(np.int16)).view(torch.uint16),
                a=to_dev_bf16(p["lora_a"]), b=to_dev_bf16(p["lora_b"]),
                bias=None if p["bias_bits"] is None
                else to_dev(p["bias_bits"].view(np.int16)).view(torch.uint16),
                scaling=float(p["alpha"] / p["rank"]), group=p["group_size"])


# (m, k, n, r, group): the fused GEMM path, a ragged tile, the skinny path
# (elementwise activation after the skinny kernels) and the generic path
SHAPES = [(512, 256, 384, 16, 64), (300, 128, 200, 8, None), (8, 256, 192, 16, 64),
          (37, 100, 52, 3, None), (256, 128, 256, 48, 64)]


@pytest.mark.parametrize("activation", ["gelu", "silu_mul"])
@pytest.mark.parametrize("m,k,n,r,group", SHAPES)
def test_forward_act_matches_oracle(activation, m, k, n, r, group):
    g = rng(m + n + (7 if activation == "gelu" else 9))
    p = _linear(g, n, k, r, group, bias=True, b_scale=20.0)
    x = bf16_values(g.standard_normal((m, k)))
    gate = bf16_values(g.standard_normal((m, n)) * 2.0)
    d = _dev(p)
    y, z, h = ops.int4lora_forward_act(
        to_dev_bf16(x), d["packed"], d["scale_bits"], d["a"], d["b"], activation=activation,
        scaling=d["scaling"], group_size=group, bias_bits=d["bias"],
        gate=to_dev_bf16(gate) if activation == "silu_mul" else None)
    torch.cuda.synchronize()
    z_o, h_o = olora.lora_forward(x, p["packed"], p["scale_bits"], p["lora_a"], p["lora_b"],
                                  alpha=p["alpha"], rank=r, bias_bits=p["bias_bits"],
                                  group_size=group)
    assert rel_l2(from_dev(z), z_o) < TOL
    assert rel_l2(from_dev(h), h_o) < TOL
    # the activation of the GPU's own z, rounded once
    zg = from_dev(z)
    want = oact.act_forward(activation, zg, gate if activation == "silu_mul" else None)
    assert_act_bits(bits_from_dev(y), want)
    # z equals the plain forward's y bit for bit
    y_plain, _ = ops.int4lora_forward(to_dev_bf16(x), d["packed"], d["scale_bits"], d["a"], d["b"],
                                      scaling=d["scaling"], group_size=group, bias_bits=d["bias"])
    torch.cuda.synchronize()
    assert torch.equal(y_plain, z)


# (m, k, n, r, group) of the down projection: k is the activation width
BWD_SHAPES = [(512, 384, 256, 16, 64), (300, 192, 128, 8, None), (8, 256, 192, 16, 64),
              (37, 100, 52, 3, None), (256, 256, 128, 48, 64)]


@pytest.mark.parametrize("activation", ["gelu", "silu_mul", "add"])
@pytest.mark.parametrize("m,k,n,r,group", BWD_SHAPES)
def test_backward_act_matches_oracle(activation, m, k, n, r, group):
    g = rng(m + k + (11 if activation == "gelu" else 13))
    p = _linear(g, n, k, r, group, bias=False)
    x = bf16_values(g.standard_normal((m, k)))  # the activation output
    z = bf16_values(g.standard_normal((m, k)) * 2.0)
    gate = bf16_values(g.standard_normal((m, k)) * 2.0)
    gy = bf16_values(g.standard_normal((m, n)))
    d = _dev(p)
    xd, gyd = to_dev_bf16(x), to_dev_bf16(gy)
    _, h = ops.int4lora_forward(xd, d["packed"], d["scale_bits"], d["a"], d["b"],
                                scaling=d["scaling"], group_size=group)
    dz, dgate, d_a, d_b = ops.int4lora_backward_act(
        gyd, xd, d["packed"], d["scale_bits"], d["a"], d["b"], h, activation=activation,
        z=to_dev_bf16(z), gate=to_dev_bf16(gate) if activation == "silu_mul" else None,
        scaling=d["scaling"], group_size=group)
    dx, d_a2, d_b2 = ops.int4lora_backward(gyd, xd, d["packed"], d["scale_bits"], d["a"], d["b"],
                                           h, scaling=d["scaling"], group_size=group)
    torch.cuda.synchronize()
    # the LoRA gradients are the plain backward's
    assert torch.equal(d_a, d_a2) and torch.equal(d_b, d_b2)
    # the activation's backward of the GPU's own (rounded) input gradient
    dxg = from_dev(dx)
    want_dz, want_dg = oact.act_backward(activation, dxg, z,
                                         gate if activation == "silu_mul" else None)
    assert_act_bits(bits_from_dev(dz), want_dz)
    if activation == "silu_mul":
        assert_act_bits(bits_from_dev(dgate), want_dg)
    else:
        assert dgate is None
    # and the input gradient itself against the oracle
    dx_o, _, _ = olora.lora_backward(gy, x, p["packed"], p["scale_bits"], p["lora_a"],
                                     p["lora_b"], from_dev(h), alpha=p["alpha"], rank=r,
                                     group_size=group)
    assert rel_l2(dxg, dx_o) < TOL


@pytest.mark.parametrize("m,k,n,r,group", [(256, 128, 192, 8, 64), (37, 100, 52, 3, None)])
def test_shared_input_projections_match_separate_linears(m, k, n, r, group):
    """q / k / v of one input: outputs and LoRA gradients equal the separate
    linears' bit for bit; the input gradient equals the bf16 sum of theirs in
    projection order, bit for bit (fused GEMM and generic paths)."""

    g = rng(m + 3 * n)
    ps = [_linear(g, n, k, r, group, bias=True, b_scale=10.0) for _ in range(3)]
    dv = [_dev(p) for p in ps]
    x = to_dev_bf16(bf16_values(g.standard_normal((m, k))))
    gys = [to_dev_bf16(bf16_values(g.standard_normal((m, n)))) for _ in range(3)]
    views, leaves = [], []
    for d in dv:
        views += [d["a"].clone().requires_grad_(True), d["b"].clone().requires_grad_(True)]
        leaves += [d["packed"], d["scale_bits"], d["bias"], d["scaling"], d["group"]]
    xd = x.clone().requires_grad_(True)
    outs = ops.Int4LoRASharedInputFn.apply(xd, 3, *views, *leaves)
    grads = torch.autograd.grad(outs, [xd] + views, gys)
    dx_sum = None
    for i, d in enumerate(dv):
        y, h = ops.int4lora_forward(x, d["packed"], d["scale_bits"], d["a"], d["b"],
                                    scaling=d["scaling"], group_size=d["group"], bias_bits=d["bias"])
        assert torch.equal(outs[i], y)
        dx, d_a, d_b = ops.int4lora_backward(gys[i], x, d["packed"], d["scale_bits"], d["a"],
                                             d["b"], h, scaling=d["scaling"], group_size=d["group"])
        assert torch.equal(grads[1 + 2 * i], d_a.to(torch.bfloat16))
        assert torch.equal(grads[2 + 2 * i], d_b.to(torch.bfloat16))
        dx_sum = dx if dx_sum is None else (dx_sum.float() + dx.float()).to(torch.bfloat16)
    torch.cuda.synchronize()
    assert torch.equal(grads[0], dx_sum)


def _mlp_params(g, k, f, r, group, names):
    return {nm: _linear(g, f if nm != "down" else k, k if nm != "down" else f, r, group,
                        bias=nm != "gate", b_scale=10.0) for nm in names}


@pytest.mark.parametrize("m,k,f,r,group", [(256, 128, 512, 8, 64), (40, 128, 256, 4, None)])
def test_gelu_mlp_forward_backward_matches_oracle(m, k, f, r, group):
    g = rng(m + f)
    ps = _mlp_params(g, k, f, r, group, ["up", "down"])
    x = bf16_values(g.standard_normal((m, k)))
    gy = bf16_values(g.standard_normal((m, k)))
    up, down = _dev(ps["up"]), _dev(ps["down"])
    xd = to_dev_bf16(x).requires_grad_(True)
    views = [up["a"].clone().requires_grad_(True), up["b"].clone().requires_grad_(True),
             down["a"].clone().requires_grad_(True), down["b"].clone().requires_grad_(True)]
    y = ops.Int4LoRAGeluMLPFn.apply(
        xd, *views, up["packed"], up["scale_bits"], up["bias"], up["scaling"], up["group"],
        down["packed"], down["scale_bits"], down["bias"], down["scaling"], down["group"])
    grads = torch.autograd.grad(y, [xd] + views, to_dev_bf16(gy))
    torch.cuda.synchronize()
    y_o, z_o, act_o, h_up, h_down = oact.gelu_mlp_forward(x, ps["up"], ps["down"])
    want = oact.gelu_mlp_backward(gy, x, ps["up"], ps["down"], z_o, act_o, h_up, h_down)
    assert rel_l2(from_dev(y), y_o) < TOL
    for got, exp in zip(grads, want):
        assert rel_l2(from_dev(got.float()), exp) < 2 * TOL


@pytest.mark.parametrize("m,k,f,r,group", [(256, 128, 512, 8, 64), (40, 128, 256, 4, None)])
def test_swiglu_mlp_forward_backward_matches_oracle(m, k, f, r, group):
    g = rng(m + f + 1)
    ps = _mlp_params(g, k, f, r, group, ["gate", "up", "down"])
    x = bf16_values(g.standard_normal((m, k)))
    gy = bf16_values(g.standard_normal((m, k)))
    dv = {nm: _dev(ps[nm]) for nm in ("gate", "up", "down")}
    xd = to_dev_bf16(x).requires_grad_(True)
    views = []
    for nm in ("gate", "up", "down"):
        views += [dv[nm]["a"].clone().requires_grad_(True), dv[nm]["b"].clone().requires_grad_(True)]
    leaves = []
    for nm in ("gate", "up", "down"):
        leaves += [dv[nm]["packed"], dv[nm]["scale_bits"], dv[nm]["bias"], dv[nm]["scaling"],
                   dv[nm]["group"]]
    y = ops.Int4LoRASwiGLUMLPFn.apply(xd, *views, *leaves)
    grads = torch.autograd.grad(y, [xd] + views, to_dev_bf16(gy))
    torch.cuda.synchronize()
    out = oact.swiglu_mlp_forward(x, ps["gate"], ps["up"], ps["down"])
    want = oact.swiglu_mlp_backward(gy, x, ps["gate"], ps["up"], ps["down"], *out[1:])
    assert rel_l2(from_dev(y), out[0]) < TOL
    for got, exp in zip(grads, want):
        assert rel_l2(from_dev(got.float()), exp) < 2 * TOL
