"""Feed-forward blocks over INT4 + LoRA projections with the activation fused
into the projections' GEMM epilogues.

``gelu_mlp`` is BertMLP's ``output(activate(input(hidden), "gelu"))``
(src/representax/models/bert/model.py:243-249, activate at
src/representax/models/components.py:153-167); ``swiglu_mlp`` is the Qwen3
text MLP's ``down(silu(gate(x)) * up(x))``
(src/representax/models/qwen3_vl/text.py:200-203). The activation runs in
float32 on the projections' bf16 outputs and is rounded once to bf16, the
reading in which XLA evaluates a fused elementwise chain with its default
excess precision. Under the fp8 policy, or with another compute dtype, the
blocks are composed from the separate projections.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from . import ops
from .adapters import QuantizedLoRALinear
from .precision import activation_inputs, active_compute_dtype, active_policy, compute_parameter


def _fusable(value: torch.Tensor, *linears: QuantizedLoRALinear) -> bool:
    policy = active_policy()
    if policy is not None and policy.matrix_dtype == torch.float8_e4m3fn:
        return False
    if active_compute_dtype(value.dtype) != torch.bfloat16:
        return False
    return all(isinstance(l, QuantizedLoRALinear) and l.packed_weight.ndim == 2 for l in linears)


def _leaves(layer: QuantizedLoRALinear) -> tuple:
    return (layer.packed_weight, layer.scale_bits, layer.bias_bits, layer.scaling,
            layer.group_size)


def _views(layer: QuantizedLoRALinear) -> tuple:
    return compute_parameter(layer.lora_a), compute_parameter(layer.lora_b)


def gelu_mlp(value: torch.Tensor, up: torch.nn.Module, down: torch.nn.Module) -> torch.Tensor:
    """``down(gelu(up(value)))`` with the exact (erf) GELU."""

    if not _fusable(value, up, down):
        return down(F.gelu(up(value)))
    x = activation_inputs(value).to(torch.bfloat16)
    lead = x.shape[:-1]
    y = ops.Int4LoRAGeluMLPFn.apply(x.reshape(-1, up.input_size), *_views(up), *_views(down),
                                    *_leaves(up), *_leaves(down))
    return y.reshape(*lead, down.output_size)


def swiglu_mlp(value: torch.Tensor, gate: torch.nn.Module, up: torch.nn.Module,
               down: torch.nn.Module) -> torch.Tensor:
    """``down(silu(gate(value)) * up(value))``."""

    if not _fusable(value, gate, up, down):
        return down(F.silu(gate(value)) * up(value))
    x = activation_inputs(value).to(torch.bfloat16)
    lead = x.shape[:-1]
    y = ops.Int4LoRASwiGLUMLPFn.apply(x.reshape(-1, up.input_size), *_views(gate), *_views(up),
                                      *_views(down), *_leaves(gate), *_leaves(up), *_leaves(down))
    return y.reshape(*lead, down.output_size)


__all__ = ["gelu_mlp", "swiglu_mlp"]
