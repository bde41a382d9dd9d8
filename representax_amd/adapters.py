"""Low-rank adapters over packed INT4 base weights
(mirror of src/representax/models/adapters.py).

``QuantizedLoRALinear`` keeps the reference's leaves, names and dtypes:

* ``packed_weight``  uint8  ``[*, N, ceil(K/2)]`` (buffer, frozen)
* ``scale_bits``     uint16 ``[*, N]`` bf16 bit patterns (buffer, frozen);
  ``[*, N, K/G]`` when built with ``group_size=G`` (an extension)
* ``bias_bits``      uint16 ``[*, N]`` or None (buffer, frozen)
* ``lora_a``         float32 ``[*, r, K]`` (parameter)
* ``lora_b``         float32 ``[*, N, r]`` (parameter)

and static ``input_size``, ``output_size``, ``rank``, ``alpha``. Its forward
and backward run in the fused HIP kernels of ``librepresentax_amd``.
"""

from __future__ import annotations

import copy
import re
from typing import Any, TypeVar

import torch

from . import ops
from .components import Linear
from .sharding import activation_out_sharding, constrain_activation, replicate
from .precision import (
    active_compute_dtype,
    active_policy,
    activation_inputs,
    compute_parameter,
    linear_matmul,
)

ModelT = TypeVar("ModelT", bound=torch.nn.Module)


def _bits_from_bfloat16(value: torch.Tensor) -> torch.Tensor:
    """bf16 bit patterns of ``value`` rounded to bf16 (adapters.py:30-31)."""

    return value.to(torch.bfloat16).view(torch.uint16)


def _bfloat16_from_bits(value: torch.Tensor) -> torch.Tensor:
    """bf16 tensor from bit patterns (adapters.py:34-35)."""

    return value.view(torch.bfloat16)


def _pack_int4_rows(weight: torch.Tensor, group_size: int | None = None):
    """Per-output-row (or per-group) symmetric INT4 pack on the device
    (adapters.py:38-65)."""

    return ops.int4_pack(weight, group_size)


def _unpack_int4_rows(packed: torch.Tensor, scale_bits: torch.Tensor, input_size: int,
                      group_size: int | None = None) -> torch.Tensor:
    """bf16 dequantized weight (adapters.py:68-79), bit-exact."""

    return ops.int4_dequant(packed, scale_bits, input_size, group_size)


def _seeded_generator(key: Any, device: torch.device) -> torch.Generator:
    g = torch.Generator(device=device)
    if isinstance(key, torch.Generator):
        g.manual_seed(int(key.initial_seed()))
    else:
        g.manual_seed(int(key))
    return g


def _split_keys(key: Any, count: int) -> list[int]:
    """Independent per-match seeds from one key (the role of jax.random.split)."""

    base = int(key.initial_seed()) if isinstance(key, torch.Generator) else int(key)
    g = torch.Generator()
    g.manual_seed(base)
    return [int(v) for v in torch.randint(0, 2**62, (count,), generator=g)]


class QuantizedLoRALinear(torch.nn.Module):
    """Packed INT4 base projection with bf16 compute and fp32 LoRA masters
    (adapters.py:82-93)."""

    def __init__(self, *, packed_weight: torch.Tensor, scale_bits: torch.Tensor,
                 bias_bits: torch.Tensor | None, lora_a: torch.Tensor, lora_b: torch.Tensor,
                 input_size: int, output_size: int, rank: int, alpha: float,
                 group_size: int | None = None) -> None:
        super().__init__()
        self.register_buffer("packed_weight", packed_weight)
        self.register_buffer("scale_bits", scale_bits)
        self.register_buffer("bias_bits", bias_bits)
        self.lora_a = torch.nn.Parameter(lora_a)
        self.lora_b = torch.nn.Parameter(lora_b)
        self.input_size = int(input_size)
        self.output_size = int(output_size)
        self.rank = int(rank)
        self.alpha = float(alpha)
        self.group_size = None if group_size in (None, input_size) else int(group_size)

    @classmethod
    def from_linear(cls, linear: Linear, *, rank: int, alpha: float, key: Any,
                    initialization_scale: float | None = None,
                    group_size: int | None = None) -> "QuantizedLoRALinear":
        """Quantize one native projection and add a zero-output adapter
        (adapters.py:95-139)."""

        weight = linear.weight.detach()
        if rank <= 0 or rank > min(weight.shape[-2:]):
            raise ValueError("adapter rank must fit both linear dimensions")
        if alpha <= 0:
            raise ValueError("adapter alpha must be positive")
        packed, scales = _pack_int4_rows(weight, group_size)
        scale = weight.shape[-1] ** -0.5 if initialization_scale is None else initialization_scale
        gen = _seeded_generator(key, weight.device)
        lora_a = scale * torch.randn((*weight.shape[:-2], rank, weight.shape[-1]),
                                     generator=gen, dtype=torch.float32, device=weight.device)
        lora_b = torch.zeros((*weight.shape[:-2], weight.shape[-2], rank), dtype=torch.float32,
                             device=weight.device)
        bias = None if linear.bias is None else _bits_from_bfloat16(linear.bias.detach())
        return cls(packed_weight=packed, scale_bits=scales, bias_bits=bias, lora_a=lora_a,
                   lora_b=lora_b, input_size=weight.shape[-1], output_size=weight.shape[-2],
                   rank=rank, alpha=alpha, group_size=group_size)

    @property
    def scaling(self) -> float:
        return self.alpha / self.rank

    def base_weight(self) -> torch.Tensor:
        """bf16 base materialized at its use boundary (adapters.py:141-148)."""

        return _unpack_int4_rows(replicate(self.packed_weight), replicate(self.scale_bits),
                                 self.input_size, self.group_size)

    def merged_weight(self) -> torch.Tensor:
        """float32 ``base + (B @ A) * alpha / r`` (adapters.py:150-156)."""

        if self.packed_weight.ndim == 2:
            return ops.int4_merge(self.packed_weight, self.scale_bits, self.lora_a.detach(),
                                  self.lora_b.detach(), alpha=self.alpha, rank=self.rank,
                                  input_size=self.input_size, group_size=self.group_size)
        return torch.stack([self[i].merged_weight() for i in range(self.packed_weight.shape[0])])

    def __getitem__(self, index: int) -> "QuantizedLoRALinear":
        """One layer of a stacked ``[L, N, K]`` adapter, sharing storage."""

        if self.packed_weight.ndim <= 2:
            raise IndexError("adapter is not stacked")
        view = QuantizedLoRALinear.__new__(QuantizedLoRALinear)
        torch.nn.Module.__init__(view)
        view.register_buffer("packed_weight", self.packed_weight[index])
        view.register_buffer("scale_bits", self.scale_bits[index])
        view.register_buffer("bias_bits", None if self.bias_bits is None else self.bias_bits[index])
        view.lora_a = torch.nn.Parameter(self.lora_a[index])
        view.lora_b = torch.nn.Parameter(self.lora_b[index])
        view.input_size, view.output_size = self.input_size, self.output_size
        view.rank, view.alpha, view.group_size = self.rank, self.alpha, self.group_size
        return view

    def forward(self, value: torch.Tensor) -> torch.Tensor:
        """``y = x W_b^T + (x A^T) B^T * alpha/r (+ bias)`` (adapters.py:158-182).

        Under a bf16 (or fp32) policy the whole projection is one fused HIP
        call; under the fp8 policy the three products go through
        ``linear_matmul`` like the reference's. Without a policy, bf16
        activations meet the float32 masters and the adapter term and the
        output are promoted to float32 (the reference's ``jnp.matmul``).
        """

        if self.packed_weight.ndim != 2:
            raise ValueError("call a stacked adapter one layer at a time (adapter[i])")
        value = activation_inputs(value)
        compute_dtype = active_compute_dtype(value.dtype)
        policy = active_policy()
        if policy is not None and policy.matrix_dtype == torch.float8_e4m3fn:
            return self._forward_fp8(value, compute_dtype)
        a = compute_parameter(self.lora_a)
        b = compute_parameter(self.lora_b)
        x = value.to(compute_dtype)
        lead = x.shape[:-1]
        x2d = x.reshape(-1, self.input_size)
        if x2d.dtype == torch.bfloat16 and a.dtype == torch.float32:
            # no policy: jnp.matmul promotes the bf16 activations against the
            # float32 masters, so the adapter term and the output are float32
            y = ops.Int4LoRAPromotedFn.apply(x2d, a, b, self.packed_weight, self.scale_bits,
                                             self.bias_bits, self.scaling, self.group_size)
        elif torch.is_grad_enabled() and (x2d.requires_grad or a.requires_grad or b.requires_grad):
            y = ops.Int4LoRALinearFn.apply(x2d, a, b, self.packed_weight, self.scale_bits,
                                           self.bias_bits, self.scaling, self.group_size)
        else:
            # no backward will run: the fused call alone, h kept in its scratch
            y, _ = ops.int4lora_forward(x2d, self.packed_weight, self.scale_bits, a, b,
                                        scaling=self.scaling, group_size=self.group_size,
                                        bias_bits=self.bias_bits, need_h=False)
        return constrain_activation(y.reshape(*lead, self.output_size))

    def _forward_fp8(self, value: torch.Tensor, compute_dtype: torch.dtype) -> torch.Tensor:
        output = linear_matmul(value, self.base_weight().to(compute_dtype).transpose(-1, -2),
                               out_sharding=activation_out_sharding(value.ndim))
        hidden = linear_matmul(value, compute_parameter(self.lora_a).transpose(-1, -2))
        adapter = linear_matmul(hidden, compute_parameter(self.lora_b).transpose(-1, -2))
        c = torch.tensor(self.scaling, dtype=torch.float32).to(adapter.dtype).item()
        output = output + adapter * c
        if self.bias_bits is not None:
            output = output + _bfloat16_from_bits(replicate(self.bias_bits)).to(compute_dtype)
        return constrain_activation(output)

    def merge(self) -> Linear:
        """Conventional projection for export or inference (adapters.py:184-194)."""

        bias = None
        if self.bias_bits is not None:
            bias = _bfloat16_from_bits(self.bias_bits).to(torch.float32)
        return Linear(self.merged_weight(), bias)

    def extra_repr(self) -> str:
        return (f"input_size={self.input_size}, output_size={self.output_size}, "
                f"rank={self.rank}, alpha={self.alpha}, group_size={self.group_size}")


def _path_name(path: str) -> str:
    """torch module path -> the reference's ``jax.tree_util.keystr`` style:
    ``layers.0.attention.query`` -> ``.layers[0].attention.query``."""

    if not path:
        return ""
    out = []
    for part in path.split("."):
        out.append(f"[{part}]" if part.isdigit() else f".{part}")
    return "".join(out)


def matched_linear_paths(model: torch.nn.Module, target_pattern: str = ".*") -> list[str]:
    """Module paths of the ``Linear`` leaves that ``apply_quantized_lora``
    would replace (adapters.py:212-223)."""

    pattern = re.compile(target_pattern)
    return [
        name
        for name, module in model.named_modules()
        if isinstance(module, Linear) and pattern.search(_path_name(name))
    ]


def _set_module(root: torch.nn.Module, path: str, new: torch.nn.Module) -> torch.nn.Module:
    if not path:
        return new
    parent_path, _, leaf = path.rpartition(".")
    parent = root.get_submodule(parent_path) if parent_path else root
    if leaf.isdigit() and isinstance(parent, (torch.nn.ModuleList, torch.nn.Sequential)):
        parent[int(leaf)] = new
    else:
        setattr(parent, leaf, new)
    return root


def apply_quantized_lora(model: ModelT, *, rank: int, alpha: float, key: Any,
                         target_pattern: str = ".*", initialization_scale: float | None = None,
                         group_size: int | None = None, inplace: bool = False) -> ModelT:
    """Replace matching native ``Linear`` leaves (adapters.py:201-236).

    Like the reference this returns a new model unless ``inplace``; a pattern
    that matches nothing raises ``ValueError``.
    """

    matched = matched_linear_paths(model, target_pattern)
    if not matched:
        raise ValueError("adapter target_pattern matched no native Linear modules")
    if rank <= 0:
        raise ValueError("adapter rank must fit both linear dimensions")
    if alpha <= 0:
        raise ValueError("adapter alpha must be positive")
    target = model if inplace else copy.deepcopy(model)
    seeds = _split_keys(key, len(matched))
    for path, seed in zip(matched, seeds, strict=True):
        leaf = target.get_submodule(path) if path else target
        replacement = QuantizedLoRALinear.from_linear(
            leaf, rank=rank, alpha=alpha, key=seed, initialization_scale=initialization_scale,
            group_size=group_size)
        target = _set_module(target, path, replacement)
    return target


def merge_quantized_lora(model: ModelT) -> ModelT:
    """Replace every adapter with an ordinary merged ``Linear`` (adapters.py:239-251)."""

    target = copy.deepcopy(model)
    if isinstance(target, QuantizedLoRALinear):
        return target.merge()  # type: ignore[return-value]
    paths = [n for n, m in target.named_modules() if isinstance(m, QuantizedLoRALinear)]
    for path in paths:
        target = _set_module(target, path, target.get_submodule(path).merge())
    return target


def lora_parameter_filter(model: torch.nn.Module) -> dict[str, bool]:
    """``{parameter name: trainable}``: exactly the floating ``lora_a`` /
    ``lora_b`` leaves are selected (adapters.py:254-267)."""

    selected = {"lora_a", "lora_b"}
    return {
        name: p.is_floating_point() and name.rsplit(".", 1)[-1] in selected
        for name, p in model.named_parameters()
    }


def lora_parameters(model: torch.nn.Module) -> list[torch.nn.Parameter]:
    """The parameters selected by ``lora_parameter_filter``."""

    chosen = lora_parameter_filter(model)
    return [p for name, p in model.named_parameters() if chosen[name]]


__all__ = [
    "QuantizedLoRALinear",
    "apply_quantized_lora",
    "lora_parameter_filter",
    "lora_parameters",
    "matched_linear_paths",
    "merge_quantized_lora",
]
