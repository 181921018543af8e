"""Checkpoint-size policy for the time-recompute paths (checkpointing.py:1-60)."""

from __future__ import annotations

import math
from typing import Literal, Union

CheckpointPolicy = Literal["memory", "balanced", "speed"]
CheckpointSize = Union[int, CheckpointPolicy]
_POLICIES = ("memory", "balanced", "speed")


def recommended_checkpoint_size(timesteps: int, *, policy: CheckpointPolicy = "balanced") -> int:
    """Chunk length for a horizon: memory = ceil(sqrt T), balanced = ceil(T/4),
    speed = ceil(T/2), clamped to [1, T] (checkpointing.py:13-33)."""

    if timesteps <= 0:
        raise ValueError("timesteps must be positive")
    if policy == "memory":
        size = math.ceil(math.sqrt(timesteps))
    elif policy == "balanced":
        size = math.ceil(timesteps / 4)
    elif policy == "speed":
        size = math.ceil(timesteps / 2)
    else:
        raise ValueError("policy must be 'memory', 'balanced', or 'speed'")
    return max(1, min(timesteps, size))


def resolve_checkpoint_size(timesteps: int, checkpoint_size: CheckpointSize) -> int:
    """An int is capped at T; a policy name is resolved (checkpointing.py:36-43)."""

    if isinstance(checkpoint_size, int):
        if checkpoint_size <= 0:
            raise ValueError("checkpoint_size must be positive")
        return min(checkpoint_size, timesteps)
    return recommended_checkpoint_size(timesteps, policy=checkpoint_size)


def parse_checkpoint_size(value: str) -> CheckpointSize:
    """Parse a policy name or positive integer (checkpointing.py:46-60)."""

    if value in _POLICIES:
        return value  # type: ignore[return-value]
    try:
        size = int(value)
    except ValueError as exc:
        raise ValueError(
            "checkpoint_size must be a positive integer or one of: " + ", ".join(sorted(_POLICIES))
        ) from exc
    if size <= 0:
        raise ValueError("checkpoint_size must be positive")
    return size
