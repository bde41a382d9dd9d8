"""The native projection that the adapter replaces
(mirror of src/representax/models/components.py:58-94)."""

from __future__ import annotations

import torch

from .precision import activation_inputs, compute_parameter, linear_matmul


def _generator(key) -> torch.Generator | None:
    if key is None or isinstance(key, torch.Generator):
        return key
    g = torch.Generator()
    g.manual_seed(int(key))
    return g


class Linear(torch.nn.Module):
    """Batched linear projection ``y = x W^T (+ b)`` with ``W [*, N, K]``.

    ``__call__`` follows components.py:81-94: inputs are cast to the activation
    dtype, the fp32 master weight to the compute dtype, and the product goes
    through ``linear_matmul`` (so the fp8 policy reaches the fp8 kernels).
    """

    def __init__(self, weight: torch.Tensor, bias: torch.Tensor | None = None) -> None:
        super().__init__()
        self.weight = torch.nn.Parameter(weight)
        self.bias = None if bias is None else torch.nn.Parameter(bias)

    @classmethod
    def init(cls, input_size: int, output_size: int, *, key, scale: float,
             dtype: torch.dtype = torch.float32, bias: bool = False,
             device: torch.device | str | None = None) -> "Linear":
        """``weight = scale * N(0, 1)`` of shape ``[output, input]``, zero bias
        (components.py:65-79). ``key`` is an int seed or a torch.Generator."""

        w = scale * torch.randn((output_size, input_size), generator=_generator(key), dtype=dtype)
        b = torch.zeros((output_size,), dtype=dtype) if bias else None
        if device is not None:
            w = w.to(device)
            b = None if b is None else b.to(device)
        return cls(w, b)

    @property
    def input_size(self) -> int:
        return self.weight.shape[-1]

    @property
    def output_size(self) -> int:
        return self.weight.shape[-2]

    def forward(self, value: torch.Tensor) -> torch.Tensor:
        value = activation_inputs(value)
        weight = compute_parameter(self.weight)
        output = linear_matmul(value, weight.transpose(-1, -2), fp8_owner=self)
        if self.bias is not None:
            output = output + compute_parameter(self.bias)
        return output


__all__ = ["Linear"]
