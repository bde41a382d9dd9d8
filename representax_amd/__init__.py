"""MI355X-native implementation of representax's quantized-linear path.

Public API mirrors the reference (``representax.models.adapters``,
``representax.precision``, ``representax.config``): ``QuantizedLoRALinear``,
``apply_quantized_lora``, ``merge_quantized_lora``, ``lora_parameter_filter``,
``Linear``, ``linear_matmul``, ``precision_context``, ``PrecisionConfig``,
``QuantizedLoRAConfig``. The arithmetic runs in hand-written gfx950 HIP
kernels (``librepresentax_amd.so``, C ABI in ``include/representax_amd.h``).
"""

from .adapters import (
    QuantizedLoRALinear,
    apply_quantized_lora,
    lora_parameter_filter,
    lora_parameters,
    matched_linear_paths,
    merge_quantized_lora,
)
from .components import Linear
from .config import PrecisionConfig, QuantizedLoRAConfig
from .mlp import gelu_mlp, shared_input_projections, swiglu_mlp
from .precision import (
    FP32_POLICY,
    DelayedScaling,
    PrecisionPolicy,
    activation_inputs,
    active_compute_dtype,
    active_model_for_compute,
    compute_parameter,
    linear_matmul,
    model_for_compute,
    precision_context,
    resolve_precision_policy,
)
from .sharding import activation_out_sharding, constrain_activation, replicate

__all__ = [
    "DelayedScaling",
    "FP32_POLICY",
    "Linear",
    "PrecisionConfig",
    "PrecisionPolicy",
    "QuantizedLoRAConfig",
    "QuantizedLoRALinear",
    "activation_inputs",
    "activation_out_sharding",
    "active_compute_dtype",
    "active_model_for_compute",
    "apply_quantized_lora",
    "compute_parameter",
    "constrain_activation",
    "gelu_mlp",
    "linear_matmul",
    "lora_parameter_filter",
    "lora_parameters",
    "matched_linear_paths",
    "merge_quantized_lora",
    "model_for_compute",
    "precision_context",
    "replicate",
    "resolve_precision_policy",
    "shared_input_projections",
    "swiglu_mlp",
]
