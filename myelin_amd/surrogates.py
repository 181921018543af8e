"""Surrogate registry: names, ids and the primitive callables.

The primitives are part of the public API because modules take them as
constructor arguments (``SurrogateLIFCell(surrogate=atan_surrogate)``) and
map them back to names (surrogates.py:113-152).  The HIP kernels evaluate
the closed-form derivatives themselves (``sg_deriv`` in
``csrc/recurrence.hip``); these Python functions only identify the choice.
"""

from __future__ import annotations

from collections.abc import Callable
from typing import Literal

import torch

SurrogateFn = Callable[[torch.Tensor], torch.Tensor]
SurrogateName = Literal["sigmoid", "fast_sigmoid", "atan", "triangular", "superspike", "multi_gaussian"]
SURROGATE_NAMES: tuple[SurrogateName, ...] = (
    "sigmoid",
    "fast_sigmoid",
    "atan",
    "triangular",
    "superspike",
    "multi_gaussian",
)
# kernel ids (include/myelin_hip.h, same numbering as triton/lif.py:356-370)
SURROGATE_IDS: dict[str, int] = {name: i for i, name in enumerate(SURROGATE_NAMES)}


def sigmoid_surrogate(centered: torch.Tensor) -> torch.Tensor:
    """Logistic primitive (surrogates.py:29-32)."""

    return torch.sigmoid(centered)


def fast_sigmoid_surrogate(centered: torch.Tensor) -> torch.Tensor:
    """``0.5 * (c / (1 + |c|) + 1)`` (surrogates.py:35-38)."""

    return 0.5 * (centered / (1.0 + centered.abs()) + 1.0)


def atan_surrogate(centered: torch.Tensor) -> torch.Tensor:
    """``atan(pi c / 2) / pi + 1/2`` (surrogates.py:41-44)."""

    return torch.atan(torch.pi * centered / 2.0) / torch.pi + 0.5


def triangular_surrogate(centered: torch.Tensor) -> torch.Tensor:
    """``clamp(1 - |c|, 0, 1)`` (surrogates.py:47-50)."""

    return (1.0 - centered.abs()).clamp(min=0.0, max=1.0)


def superspike_surrogate(centered: torch.Tensor) -> torch.Tensor:
    """Primitive with derivative ``1 / (1 + |c|)^2`` (surrogates.py:53-61)."""

    return centered / (1.0 + centered.abs()) + 0.5


def multi_gaussian_surrogate(centered: torch.Tensor) -> torch.Tensor:
    """CDF of the 0.6 N(0, .5) + 0.2 N(1, 1) + 0.2 N(-1, 1) mixture (surrogates.py:64-75)."""

    def cdf(mean: float, sigma: float) -> torch.Tensor:
        return 0.5 * (1.0 + torch.erf((centered - mean) / (1.4142135623730951 * sigma)))

    return 0.6 * cdf(0.0, 0.5) + 0.2 * cdf(1.0, 1.0) + 0.2 * cdf(-1.0, 1.0)


_BY_NAME: dict[str, SurrogateFn] = {
    "sigmoid": sigmoid_surrogate,
    "fast_sigmoid": fast_sigmoid_surrogate,
    "atan": atan_surrogate,
    "triangular": triangular_surrogate,
    "superspike": superspike_surrogate,
    "multi_gaussian": multi_gaussian_surrogate,
}


def surrogate_from_name(name: SurrogateName) -> SurrogateFn:
    """Primitive for a stable name (surrogates.py:113-127)."""

    try:
        return _BY_NAME[name]
    except KeyError:
        raise ValueError(f"unknown surrogate {name!r}; expected one of {SURROGATE_NAMES}") from None


def surrogate_name(surrogate: SurrogateFn) -> SurrogateName:
    """Stable name of a built-in primitive (surrogates.py:130-152)."""

    for name, fn in _BY_NAME.items():
        if fn is surrogate:
            return name  # type: ignore[return-value]
    raise ValueError(
        "the HIP surrogate backward supports only built-in surrogate functions: "
        "sigmoid_surrogate, fast_sigmoid_surrogate, atan_surrogate, "
        "triangular_surrogate, superspike_surrogate, and multi_gaussian_surrogate."
    )


def surrogate_id(name: str) -> int:
    """Kernel id of a surrogate name."""

    if name not in SURROGATE_IDS:
        raise ValueError(f"unknown surrogate {name!r}; expected one of {SURROGATE_NAMES}")
    return SURROGATE_IDS[name]
