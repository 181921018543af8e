"""Shared comparison helpers for the parity tests (test code only)."""

from __future__ import annotations

import numpy as np
import torch


def to_np(t) -> np.ndarray:
    if isinstance(t, torch.Tensor):
        return t.detach().cpu().numpy()
    return np.asarray(t)


def norm_rel_err(a, b) -> float:
    """max|a - b| / max|b| (0 when both are all zero)."""

    a = to_np(a).astype(np.float64)
    b = to_np(b).astype(np.float64)
    scale = np.abs(b).max() if b.size else 0.0
    diff = np.abs(a - b).max() if b.size else 0.0
    if scale == 0.0:
        return float(diff)
    return float(diff / scale)


def assert_norm_close(a, b, rtol: float, what: str = "") -> None:
    err = norm_rel_err(a, b)
    assert err <= rtol, f"{what}: max|a-b|/max|b| = {err:.3e} > {rtol:.1e}"


def raster_agreement(a, b) -> float:
    a = to_np(a) != 0
    b = to_np(b) != 0
    return float((a == b).mean()) if a.size else 1.0


def seeded(seed: int) -> torch.Generator:
    return torch.Generator().manual_seed(seed)
