"""Config surface of the quantized-linear path
(mirror of src/representax/config.py:392-467)."""

from __future__ import annotations

import re
from typing import Literal

from pydantic import BaseModel, ConfigDict, Field, PositiveFloat, PositiveInt, field_validator

PrecisionDType = Literal["float32", "bfloat16"]
MatrixDType = Literal["float32", "bfloat16", "float8_e4m3fn"]


class FrozenConfig(BaseModel):
    model_config = ConfigDict(frozen=True, extra="forbid")


class PrecisionConfig(FrozenConfig):
    """Serializable execution dtypes at each numerical boundary (config.py:392-446)."""

    parameter_dtype: Literal["float32"] = Field(default="float32")
    compute_dtype: PrecisionDType = Field(default="float32")
    activation_dtype: PrecisionDType = Field(default="float32")
    matrix_dtype: MatrixDType | None = Field(default=None)
    accumulation_dtype: Literal["float32"] = Field(default="float32")
    loss_dtype: Literal["float32"] = Field(default="float32")
    # extension (the reference's roadmap, todo.org:1149-1154): "delayed" casts
    # fp8 operands with scales from an amax history, updated once per step
    fp8_scaling: Literal["dynamic", "delayed"] = Field(default="dynamic")
    amax_history_len: PositiveInt = Field(default=16)

    @classmethod
    def bfloat16_mixed(cls) -> "PrecisionConfig":
        """bf16 compute with fp32 master and objective state (config.py:420-424)."""

        return cls(compute_dtype="bfloat16", activation_dtype="bfloat16")

    @classmethod
    def float8_mixed(cls, fp8_scaling: Literal["dynamic", "delayed"] = "dynamic",
                     amax_history_len: int = 16) -> "PrecisionConfig":
        """Experimental fp8 matrices with bf16 everything else (config.py:426-435);
        ``fp8_scaling="delayed"`` is the extension above."""

        return cls(compute_dtype="bfloat16", activation_dtype="bfloat16",
                   matrix_dtype="float8_e4m3fn", fp8_scaling=fp8_scaling,
                   amax_history_len=amax_history_len)

    @property
    def resolved_matrix_dtype(self) -> MatrixDType:
        return self.matrix_dtype or self.compute_dtype

    @property
    def communication_dtype(self) -> PrecisionDType:
        return self.compute_dtype


class QuantizedLoRAConfig(FrozenConfig):
    """Four-bit frozen base weights plus trainable low-rank adapters
    (config.py:449-467). ``group_size`` is an extension: None keeps the
    reference's one scale per output row."""

    bits: Literal[4] = 4
    rank: PositiveInt
    alpha: PositiveFloat
    target_pattern: str = Field(default=".*", min_length=1)
    initialization_scale: PositiveFloat | None = None
    group_size: PositiveInt | None = None

    @field_validator("target_pattern")
    @classmethod
    def validate_target_pattern(cls, pattern: str) -> str:
        try:
            re.compile(pattern)
        except re.error as error:
            raise ValueError(f"invalid adapter target_pattern: {error}") from error
        return pattern


__all__ = ["PrecisionConfig", "QuantizedLoRAConfig"]
