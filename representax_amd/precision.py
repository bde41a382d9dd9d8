"""Numerical precision boundaries (mirror of src/representax/precision.py).

Same names and meaning as the reference, over torch dtypes. A policy is made
visible with ``precision_context``; ``linear_matmul`` routes projections
through the fp8 kernels when the policy's ``matrix_dtype`` is
``float8_e4m3fn`` (precision.py:224-239), and otherwise through an ordinary
matmul, as the reference does with ``jnp.matmul``.
"""

from __future__ import annotations

import math
from collections.abc import Iterator
from contextlib import contextmanager
from contextvars import ContextVar
from dataclasses import dataclass
from typing import Any

import torch

from . import ops


class DelayedScaling:
    """Persistent fp8 scale state with one coalesced update per step.

    The reference's roadmap item (todo.org:1149-1154, docs/precision.md:67-71;
    not built there): instead of a max|t| pass over every operand before its
    cast, each scaled tensor ("slot") is cast with the scale its slot holds
    and records its amax in the same pass; ``update()`` then recomputes every
    slot's scale from the last ``history_len`` recorded amaxes in one launch,
    ``max(amax / fmax, FLT_MIN)`` as in the dynamic rule. Casts saturate at
    the format's largest finite value, since the data may outgrow a scale
    set from past steps. Scales start at 1.0 and a slot whose history holds
    no nonzero amax keeps its scale. Call ``update()`` once per step, after
    the backward pass (the backward reuses the forward's scales).

    Device buffers (one set per model): ``scales`` / ``fmax`` float32
    [n_slots]; ``amax_pending`` uint32 [n_slots, pending words] (maxima
    recorded since the last update, spread over several cache lines per
    slot); ``amax_history`` uint32 [history_len, n_slots] (per-step maxima as
    ordered f32 bits); ``cursor`` int32 [1] (the history row the next update
    writes; it lives on the device so captured graphs advance it).
    """

    FMAX = {"e4m3fn": 448.0, "e5m2": 57344.0}
    _instances = 0

    def __init__(self, n_slots: int, history_len: int = 16,
                 device: torch.device | str = "cuda") -> None:
        if n_slots < 1 or history_len < 1:
            raise ValueError("delayed scaling needs at least one slot and one history row")
        self.n_slots = int(n_slots)
        self.history_len = int(history_len)
        self.scales = torch.ones(self.n_slots, dtype=torch.float32, device=device)
        self.fmax = torch.full((self.n_slots,), self.FMAX["e4m3fn"], dtype=torch.float32,
                               device=device)
        self.amax_history = torch.zeros((self.history_len, self.n_slots), dtype=torch.uint32,
                                        device=device)
        words = ops.fp8_delayed_pending_words() if torch.device(device).type == "cuda" else 2048
        self.amax_pending = torch.zeros((self.n_slots, words), dtype=torch.uint32, device=device)
        self.cursor = torch.zeros(1, dtype=torch.int32, device=device)
        self._next = 0
        DelayedScaling._instances += 1
        self._token = DelayedScaling._instances  # never reused within a process
        self._named: dict[str, dict[int, tuple[int, ...]]] = {}

    def allocate(self, formats: tuple[str, ...]) -> tuple[int, ...]:
        """Fresh slots, one per entry of ``formats`` ("e4m3fn" / "e5m2")."""

        if self._next + len(formats) > self.n_slots:
            raise ValueError(f"delayed scaling state has {self.n_slots} slots; "
                             f"{self._next + len(formats)} needed")
        slots = tuple(range(self._next, self._next + len(formats)))
        for sl, fmt in zip(slots, formats):
            self.fmax[sl] = self.FMAX[fmt]
        self._next += len(formats)
        return slots

    def slots_for(self, owner: object, formats: tuple[str, ...]) -> tuple[int, ...]:
        """The slots of ``owner`` (allocated on its first use): a module, or a
        name (a string such as the module's path).

        A module's assignment is stored on the module itself, keyed by this
        state, so copies of it (``model_for_compute`` deep-copies the model
        every step) keep using their original's slots, and no other module
        can inherit a dead module's scale history.
        """

        if isinstance(owner, str):
            table = self._named.setdefault(owner, {})
        else:
            table = getattr(owner, "_fp8_delayed_slots", None)
            if table is None:
                table = {}
                object.__setattr__(owner, "_fp8_delayed_slots", table)
        if self._token not in table:
            table[self._token] = self.allocate(formats)
        slots = table[self._token]
        if len(slots) != len(formats):
            raise ValueError("delayed-scale slots of this owner were allocated for other formats")
        return slots

    def update(self) -> None:
        ops.fp8_scale_update(self)

    @classmethod
    def for_model(cls, model: torch.nn.Module, history_len: int = 16,
                  device: torch.device | str = "cuda") -> "DelayedScaling":
        """State sized for every ``Linear`` of ``model`` (left, right and
        gradient slots each)."""

        from .components import Linear

        n = sum(1 for m in model.modules() if isinstance(m, Linear))
        return cls(max(3 * n, 1), history_len, device)


LINEAR_FORMATS = ("e4m3fn", "e4m3fn", "e5m2")  # left, right, gradient


@dataclass(frozen=True, slots=True)
class PrecisionPolicy:
    """Resolved dtypes for stored state, forward compute, and objectives
    (precision.py:19-34). ``fp8_state`` (an extension) selects delayed fp8
    scaling when set; None keeps the reference's dynamic scaling."""

    parameter_dtype: torch.dtype
    compute_dtype: torch.dtype
    activation_dtype: torch.dtype
    matrix_dtype: torch.dtype
    accumulation_dtype: torch.dtype
    loss_dtype: torch.dtype
    fp8_state: DelayedScaling | None = None

    @property
    def communication_dtype(self) -> torch.dtype:
        return self.compute_dtype


FP32_POLICY = PrecisionPolicy(
    parameter_dtype=torch.float32,
    compute_dtype=torch.float32,
    activation_dtype=torch.float32,
    matrix_dtype=torch.float32,
    accumulation_dtype=torch.float32,
    loss_dtype=torch.float32,
)

_DTYPES = {
    "float32": torch.float32,
    "bfloat16": torch.bfloat16,
    "float8_e4m3fn": torch.float8_e4m3fn,
}
_ACTIVE_PRECISION: ContextVar[PrecisionPolicy | None] = ContextVar(
    "representax_amd_precision", default=None
)


def resolve_precision_policy(config: Any, *, fp8_state: DelayedScaling | None = None
                             ) -> PrecisionPolicy:
    """Resolve a ``PrecisionConfig`` into torch dtypes (precision.py:57-67).
    A config with ``fp8_scaling="delayed"`` needs the model's
    ``DelayedScaling`` state."""

    delayed = getattr(config, "fp8_scaling", "dynamic") == "delayed"
    if delayed and config.resolved_matrix_dtype == "float8_e4m3fn" and fp8_state is None:
        raise ValueError("fp8_scaling='delayed' needs a DelayedScaling state (fp8_state=...)")
    return PrecisionPolicy(
        parameter_dtype=_DTYPES[config.parameter_dtype],
        compute_dtype=_DTYPES[config.compute_dtype],
        activation_dtype=_DTYPES[config.activation_dtype],
        matrix_dtype=_DTYPES[config.resolved_matrix_dtype],
        accumulation_dtype=_DTYPES[config.accumulation_dtype],
        loss_dtype=_DTYPES[config.loss_dtype],
        fp8_state=fp8_state if delayed else None,
    )


@contextmanager
def precision_context(policy: PrecisionPolicy) -> Iterator[None]:
    """Make one policy visible at model/objective boundaries (precision.py:70-78)."""

    token = _ACTIVE_PRECISION.set(policy)
    try:
        yield
    finally:
        _ACTIVE_PRECISION.reset(token)


def active_policy() -> PrecisionPolicy | None:
    return _ACTIVE_PRECISION.get()


def _is_inexact(value: Any) -> bool:
    return isinstance(value, torch.Tensor) and (value.is_floating_point() or value.is_complex())


def cast_floating_tree(tree: Any, dtype: torch.dtype) -> Any:
    """Cast floating tensors in nested dict/list/tuple containers (precision.py:81-87).

    Integer tensors (packed weights, scale bits) are returned unchanged.
    """

    if isinstance(tree, torch.Tensor):
        return tree.to(dtype) if _is_inexact(tree) else tree
    if isinstance(tree, dict):
        return {k: cast_floating_tree(v, dtype) for k, v in tree.items()}
    if isinstance(tree, (list, tuple)):
        return type(tree)(cast_floating_tree(v, dtype) for v in tree)
    return tree


def prepare_master_model(model: torch.nn.Module, policy: PrecisionPolicy) -> torch.nn.Module:
    """Store floating parameters in the master dtype (precision.py:90-93)."""

    for p in model.parameters():
        if p.is_floating_point():
            p.data = p.data.to(policy.parameter_dtype)
    return model


def model_for_compute(model: torch.nn.Module, policy: PrecisionPolicy) -> torch.nn.Module:
    """Transient compute copy with floating parameters in the compute dtype
    (precision.py:96-99). Modules of this package also cast at each use site
    through ``compute_parameter``, which keeps the fp32 masters as the leaves
    that receive gradients."""

    import copy

    view = copy.deepcopy(model)
    for p in view.parameters():
        if p.is_floating_point():
            p.data = p.data.to(policy.compute_dtype)
    return view


def active_model_for_compute(model: torch.nn.Module) -> torch.nn.Module:
    """``model_for_compute`` under the active policy, else ``model``
    (precision.py:102-108)."""

    policy = _ACTIVE_PRECISION.get()
    if policy is None:
        return model
    return model_for_compute(model, policy)


_COMPUTE_VIEWS: ContextVar[dict[int, torch.Tensor] | None] = ContextVar(
    "representax_amd_compute_views", default=None
)


@contextmanager
def compute_views(views: dict[int, torch.Tensor] | None) -> Iterator[None]:
    """Make precomputed compute views visible to ``compute_parameter``:
    ``views`` maps ``id(master)`` to a tensor holding exactly
    ``master.to(compute_dtype)`` (for instance a slice of one buffer that a
    train step converts from all its masters at once), which then stands for
    the per-use cast; its gradient is the cast's gradient in the compute
    dtype. Entries of another dtype than the active policy's are ignored."""

    token = _COMPUTE_VIEWS.set(views)
    try:
        yield
    finally:
        _COMPUTE_VIEWS.reset(token)


def active_compute_views() -> dict[int, torch.Tensor] | None:
    return _COMPUTE_VIEWS.get()


def compute_parameter(value: torch.Tensor) -> torch.Tensor:
    """Compute view of a parameter at its use site (precision.py:111-117)."""

    policy = _ACTIVE_PRECISION.get()
    if policy is None:
        return value
    views = _COMPUTE_VIEWS.get()
    if views is not None:
        view = views.get(id(value))
        if view is not None and view.dtype == policy.compute_dtype:
            return view
    return value.to(policy.compute_dtype)


def active_compute_dtype(fallback: torch.dtype) -> torch.dtype:
    """Active policy's compute dtype, else ``fallback`` (precision.py:120-124)."""

    policy = _ACTIVE_PRECISION.get()
    return fallback if policy is None else policy.compute_dtype


def linear_matmul(left: torch.Tensor, right: torch.Tensor, *, out_sharding: Any = None,
                  fp8_owner: object = None) -> torch.Tensor:
    """Apply the active matrix policy to ``left [..., K] @ right [K, N]``
    (precision.py:224-239). Under delayed fp8 scaling ``fp8_owner`` (the
    calling module) names the product's scale slots; without it the product
    is scaled dynamically, as in the reference."""

    del out_sharding  # single-device: sharding annotations are the identity
    policy = _ACTIVE_PRECISION.get()
    if policy is None or policy.matrix_dtype != torch.float8_e4m3fn:
        return torch.matmul(left, right)
    leading = left.shape[:-1]
    flat = left.reshape(math.prod(leading), left.shape[-1])
    if policy.fp8_state is not None and fp8_owner is not None:
        slots = policy.fp8_state.slots_for(fp8_owner, LINEAR_FORMATS)
        out = ops.Fp8DelayedLinearFn.apply(flat, right, policy.activation_dtype,
                                           policy.fp8_state, slots)
    else:
        out = ops.Fp8LinearFn.apply(flat, right, policy.activation_dtype)
    return out.reshape(*leading, right.shape[-1]).to(policy.activation_dtype)


def activation_inputs(inputs: Any) -> Any:
    """Cast model inputs to the activation dtype (precision.py:242-248)."""

    policy = _ACTIVE_PRECISION.get()
    if policy is None:
        return inputs
    return cast_floating_tree(inputs, policy.activation_dtype)


def objective_output(value: torch.Tensor) -> torch.Tensor:
    policy = _ACTIVE_PRECISION.get()
    if policy is None:
        return value
    return value.to(policy.accumulation_dtype)


def loss_value(value: torch.Tensor) -> torch.Tensor:
    policy = _ACTIVE_PRECISION.get()
    if policy is None:
        return value
    return value.to(policy.loss_dtype)


def accumulated_values(tree: Any) -> Any:
    policy = _ACTIVE_PRECISION.get()
    if policy is None:
        return tree
    return cast_floating_tree(tree, policy.accumulation_dtype)


__all__ = [
    "DelayedScaling",
    "FP32_POLICY",
    "PrecisionPolicy",
    "accumulated_values",
    "active_compute_dtype",
    "active_model_for_compute",
    "active_policy",
    "activation_inputs",
    "cast_floating_tree",
    "active_compute_views",
    "compute_parameter",
    "compute_views",
    "linear_matmul",
    "loss_value",
    "model_for_compute",
    "objective_output",
    "precision_context",
    "prepare_master_model",
    "resolve_precision_policy",
]
