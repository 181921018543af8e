"""Neuron parameter and state types (same fields and properties as
``myelin.neurons``, neurons.py:14-71)."""

from __future__ import annotations

from dataclasses import dataclass

import torch


def _euler_decay(tau: float, what: str) -> float:
    if tau <= 0:
        raise ValueError(f"{what} must be positive")
    return 1.0 - (1.0 / tau)


@dataclass(frozen=True)
class LIFParams:
    """Leaky integrate-and-fire parameters (neurons.py:14-28)."""

    tau_mem: float = 20.0
    threshold: float = 1.0
    reset: float = 0.0

    @property
    def decay(self) -> float:
        """Per-step membrane decay ``1 - 1/tau_mem`` (computed in double)."""

        return _euler_decay(self.tau_mem, "tau_mem")


@dataclass(frozen=True)
class LIFState:
    """LIF state carried between steps (neurons.py:31-35)."""

    membrane: torch.Tensor


@dataclass(frozen=True)
class ALIFParams:
    """Adaptive LIF parameters (neurons.py:38-62); ``beta`` is the adaptation
    strength, ``adaptation_decay`` is ``1 - 1/tau_adaptation``."""

    tau_mem: float = 20.0
    tau_adaptation: float = 100.0
    threshold: float = 1.0
    reset: float = 0.0
    beta: float = 1.0

    @property
    def decay(self) -> float:
        return _euler_decay(self.tau_mem, "tau_mem")

    @property
    def adaptation_decay(self) -> float:
        return _euler_decay(self.tau_adaptation, "tau_adaptation")


@dataclass(frozen=True)
class ALIFState:
    """ALIF state carried between steps (neurons.py:65-70)."""

    membrane: torch.Tensor
    adaptation: torch.Tensor
