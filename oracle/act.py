"""FFN activations next to the INT4 + LoRA linears, and the fused blocks
built from them (numpy restatement; test infrastructure).

* GELU, exact (erf) form: ``activate(value, "gelu")`` ->
  ``jax.nn.gelu(value, approximate=False)``,
  ``src/representax/models/components.py:153-167``, used by BertMLP at
  ``src/representax/models/bert/model.py:243-249``.
* SiLU-gated product ``jax.nn.silu(gate(x)) * up(x)``,
  ``src/representax/models/qwen3_vl/text.py:200-203``.

Rounding reading: the activation is evaluated exactly (float64 here) from
the bf16 linear outputs and rounded once to bf16; the backward forms the
JAX transpose of the same expressions, ``dz = d * gelu'(z)``,
``d_up = d * silu(gate)``, ``d_gate = d * up * silu'(gate)``, each rounded
once from the bf16 incoming gradient ``d``. This is how XLA evaluates a
fused elementwise chain under its default excess precision; whether the
reference's backend rounds the intermediates instead is not fixed by any
reference test (parity unpinned for the rounding of intermediates; the
functions themselves are pinned by the tests against closed forms, symmetry
identities, finite differences and torch's float64 routines).
"""

from __future__ import annotations

import numpy as np
from scipy.special import erfc

from .lora import _rounder, lora_backward, lora_forward

_INV_SQRT2 = 1.0 / np.sqrt(2.0)
_INV_SQRT_2PI = 1.0 / np.sqrt(2.0 * np.pi)


def normal_cdf(z):
    """``Phi(z) = erfc(-z / sqrt 2) / 2`` (float64; no cancellation for z < 0)."""

    return 0.5 * erfc(-np.asarray(z, dtype=np.float64) * _INV_SQRT2)


def gelu(z):
    """``z * Phi(z)`` with the standard normal CDF ``Phi`` (float64)."""

    z = np.asarray(z, dtype=np.float64)
    return z * normal_cdf(z)


def gelu_grad(z):
    """``d/dz [z Phi(z)] = Phi(z) + z phi(z)`` (float64)."""

    z = np.asarray(z, dtype=np.float64)
    return normal_cdf(z) + z * np.exp(-0.5 * z * z) * _INV_SQRT_2PI


def sigmoid(g):
    g = np.asarray(g, dtype=np.float64)
    return 1.0 / (1.0 + np.exp(-g))


def silu(g):
    """``g * sigmoid(g)`` (float64)."""

    g = np.asarray(g, dtype=np.float64)
    return g * sigmoid(g)


def silu_grad(g):
    """``sigmoid(g) (1 + g sigmoid(-g))`` (float64)."""

    g = np.asarray(g, dtype=np.float64)
    return sigmoid(g) * (1.0 + g * sigmoid(-g))


def act_forward(activation: str, z, gate=None, compute: str = "bf16") -> np.ndarray:
    """Output of the activation from compute-dtype ``z`` (and ``gate``),
    rounded once to the compute dtype ("f64" keeps float64)."""

    rnd = _rounder(compute)
    if activation == "gelu":
        return rnd(gelu(z))
    if activation == "silu_mul":
        return rnd(silu(gate) * np.asarray(z, np.float64))
    raise ValueError(activation)


def act_backward(activation: str, d, z, gate=None, compute: str = "bf16"):
    """``(dz, dgate or None)`` from the incoming gradient ``d``."""

    rnd = _rounder(compute)
    d = np.asarray(d, np.float64)
    if activation == "gelu":
        return rnd(d * gelu_grad(z)), None
    if activation == "add":
        # an input gradient added to the one accumulated so far (a shared input)
        return rnd(d + np.asarray(z, np.float64)), None
    if activation == "silu_mul":
        z = np.asarray(z, np.float64)
        return rnd(d * silu(gate)), rnd(d * z * silu_grad(gate))
    raise ValueError(activation)


def gelu_mlp_forward(x, up: dict, down: dict):
    """``down(gelu(up(x)))``: returns ``(y, z, act, h_up, h_down)``. ``up`` /
    ``down`` hold the lora_forward keyword arguments plus ``packed``,
    ``scale_bits``, ``lora_a``, ``lora_b``."""

    z, h_up = _linear(x, up)
    act = act_forward("gelu", z, compute=up.get("compute", "bf16"))
    y, h_down = _linear(act, down)
    return y, z, act, h_up, h_down


def gelu_mlp_backward(g, x, up: dict, down: dict, z, act, h_up, h_down):
    """``(dx, dA_up, dB_up, dA_down, dB_down)``."""

    d_act, da_down, db_down = _linear_backward(g, act, down, h_down)
    dz, _ = act_backward("gelu", d_act, z, compute=up.get("compute", "bf16"))
    dx, da_up, db_up = _linear_backward(dz, x, up, h_up)
    return dx, da_up, db_up, da_down, db_down


def swiglu_mlp_forward(x, gate: dict, up: dict, down: dict):
    """``down(silu(gate(x)) * up(x))``: returns
    ``(y, g, u, act, h_gate, h_up, h_down)``."""

    g, h_gate = _linear(x, gate)
    u, h_up = _linear(x, up)
    act = act_forward("silu_mul", u, g, compute=up.get("compute", "bf16"))
    y, h_down = _linear(act, down)
    return y, g, u, act, h_gate, h_up, h_down


def swiglu_mlp_backward(grad, x, gate: dict, up: dict, down: dict, g, u, act, h_gate, h_up,
                        h_down):
    """``(dx, dA_gate, dB_gate, dA_up, dB_up, dA_down, dB_down)``; the two
    input-gradient contributions add in bf16."""

    d_act, da_down, db_down = _linear_backward(grad, act, down, h_down)
    compute = up.get("compute", "bf16")
    du, dg = act_backward("silu_mul", d_act, u, g, compute=compute)
    dx_up, da_up, db_up = _linear_backward(du, x, up, h_up)
    dx_gate, da_gate, db_gate = _linear_backward(dg, x, gate, h_gate)
    dx = _rounder(compute)(np.asarray(dx_up, np.float64) + np.asarray(dx_gate, np.float64))
    return dx, da_gate, db_gate, da_up, db_up, da_down, db_down


def _split(p: dict):
    kw = {k: v for k, v in p.items() if k not in ("packed", "scale_bits", "lora_a", "lora_b")}
    return (p["packed"], p["scale_bits"], p["lora_a"], p["lora_b"]), kw


def _linear(x, p: dict):
    args, kw = _split(p)
    return lora_forward(x, *args, **kw)


def _linear_backward(g, x, p: dict, h):
    args, kw = _split(p)
    kw.pop("bias_bits", None)
    return lora_backward(g, x, *args, h, **kw)
