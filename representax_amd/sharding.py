"""Sharding hooks on the quantized-linear path (mirror of
src/representax/core/sharding.py:63-114).

The reference calls these around every projection: ``activation_out_sharding``
names the output layout of ``linear_matmul`` (adapters.py:164-168),
``replicate`` marks the packed weight and the bias as replicated
(adapters.py:141-148,178-180) and ``constrain_activation`` pins the output's
batch-leading layout (adapters.py:182). With no mesh policy active they are
the identity, which is the only state a single process with one GPU has:
this package runs one GPU per process, so there is no mesh to activate and
the hooks keep the reference's names and return values for callers written
against it.
"""

from __future__ import annotations

from typing import Any


def activation_out_sharding(rank: int) -> None:
    """The active batch-leading output layout: none without a mesh policy
    (sharding.py:63-67)."""

    del rank
    return None


def scanned_out_sharding(rank: int) -> None:
    """The scan-leading layout: none without a mesh policy (sharding.py:70-74)."""

    del rank
    return None


def replicated_out_sharding() -> None:
    """The fully replicated layout: none without a mesh policy (sharding.py:77-83)."""

    return None


def active_data_axis_size() -> int:
    """Size of the data axis: 1 in a single-GPU process (sharding.py:86-90)."""

    return 1


def constrain_activation(value: Any) -> Any:
    """Keep an activation in its batch-leading layout: the identity without
    a mesh policy (sharding.py:93-102)."""

    return value


def replicate(value: Any) -> Any:
    """Replicate a value at a global-program boundary: the identity without
    a mesh policy (sharding.py:105-114)."""

    return value


__all__ = [
    "activation_out_sharding",
    "active_data_axis_size",
    "constrain_activation",
    "replicate",
    "replicated_out_sharding",
    "scanned_out_sharding",
]
