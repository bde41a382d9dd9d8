"""Feed-forward blocks over INT4 + LoRA projections with the activation fused
into the projections' GEMM epilogues, and projections of one shared input
whose input gradients are summed in the dx GEMMs' epilogues.

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
    if not all(isinstance(l, QuantizedLoRALinear) and l.packed_weight.ndim == 2 for l in linears):
        return False
    # bf16 adapter views; float32 masters without a policy promote the
    # adapter term to float32 (the module's own path handles that)
    return all(compute_parameter(l.lora_a).dtype == torch.bfloat16 for l in linears)


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


def shared_input_projections(value: torch.Tensor, linears) -> list[torch.Tensor]:
    """``[linear(value) for linear in linears]`` (e.g. the q / k / v
    projections of attention, bert/model.py and qwen3_vl/text.py). When all
    are INT4 + LoRA, the backward adds each input gradient to the running
    sum inside its dx GEMM instead of in separate passes."""

    linears = list(linears)
    if not _fusable(value, *linears):
        return [layer(value) for layer in linears]
    x = activation_inputs(value).to(torch.bfloat16)
    lead = x.shape[:-1]
    views, leaves = [], []
    for layer in linears:
        views += list(_views(layer))
        leaves += list(_leaves(layer))
    if not torch.is_grad_enabled() or not (x.requires_grad or any(v.requires_grad for v in views)):
        # inference: every projection in one call (one pair of launches for
        # all of them at small M, where a call is launch-latency bound)
        x2d = x.reshape(-1, linears[0].input_size)
        outs = ops.int4lora_forward_multi(
            x2d, [(l.packed_weight, l.scale_bits, views[2 * i], views[2 * i + 1], l.scaling,
                   l.group_size, l.bias_bits) for i, l in enumerate(linears)], need_h=False)
        return [y.reshape(*lead, layer.output_size) for (y, _), layer in zip(outs, linears)]
    outs = ops.Int4LoRASharedInputFn.apply(x.reshape(-1, linears[0].input_size), len(linears),
                                           *views, *leaves)
    return [y.reshape(*lead, layer.output_size) for y, layer in zip(outs, linears)]


__all__ = ["gelu_mlp", "shared_input_projections", "swiglu_mlp"]
