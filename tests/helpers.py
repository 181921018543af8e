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


def elementwise_rel_err(a, b, floor: float = 1e-3) -> float:
    """max |a - b| / max(|b|, floor * max|b|): a relative bound per element,
    with elements below `floor` of the tensor's largest held to that floor."""

    a = to_np(a).astype(np.float64)
    b = to_np(b).astype(np.float64)
    if b.size == 0:
        return 0.0
    top = np.abs(b).max()
    if top == 0.0:
        return float(np.abs(a).max())
    scale = np.maximum(np.abs(b), floor * top)
    return float((np.abs(a - b) / scale).max())


def assert_elementwise_close(a, b, rtol: float, what: str = "", floor: float = 1e-3) -> None:
    err = elementwise_rel_err(a, b, floor)
    assert err <= rtol, f"{what}: max |a-b| / max(|b|, {floor:g} max|b|) = {err:.3e} > {rtol:.1e}"


def assert_same_bits(a, b, what: str = "") -> None:
    """Equal values (torch.equal: -0 == +0), with the first mismatches named."""

    a_t = torch.as_tensor(to_np(a))
    b_t = torch.as_tensor(to_np(b))
    assert a_t.shape == b_t.shape, f"{what}: shape {tuple(a_t.shape)} vs {tuple(b_t.shape)}"
    if torch.equal(a_t, b_t):
        return
    bad = (a_t != b_t).nonzero()
    idx = tuple(bad[0].tolist())
    raise AssertionError(f"{what}: {bad.shape[0]} of {a_t.numel()} elements differ; first at {idx}: "
                         f"{a_t[idx].item()!r} vs {b_t[idx].item()!r} (max rel {norm_rel_err(a_t, b_t):.2e})")


def f32_params(tau: float, *scalars: float) -> tuple[float, ...]:
    """(tau', s1', ...) for evaluating an fp32 network in float64: every
    scalar rounded to the fp32 value an fp32 evaluation multiplies or
    compares by, and tau' such that the float64 decay 1 - 1/tau' is the
    fp32-rounded decay of tau (to float64 rounding)."""

    d32 = float(np.float32(1.0 - 1.0 / tau))
    return (1.0 / (1.0 - d32), *(float(np.float32(s)) for s in scalars))


def assert_elementwise_close_or_truer(a, b, truth, rtol: float, what: str = "", floor: float = 1e-3) -> None:
    """Per element, a within `rtol` of the reference value b (relative,
    floored at `floor` of max|b|) -- or a no farther from the float64 value
    `truth` than b itself is, where two fp32 evaluations differ by more
    than that at elements far below the tensor's largest."""

    a = to_np(a).astype(np.float64)
    b = to_np(b).astype(np.float64)
    t = to_np(truth).astype(np.float64)
    if b.size == 0:
        return
    top = np.abs(b).max()
    scale = np.maximum(np.abs(b), floor * top) if top > 0 else np.ones_like(b)
    close = np.abs(a - b) <= rtol * scale
    truer = np.abs(a - t) <= np.abs(b - t)
    bad = ~(close | truer)
    assert not bad.any(), (
        f"{what}: {int(bad.sum())} elements neither within {rtol:.1e} of the reference nor as close as it to "
        f"float64; worst |a-b|/scale = {float((np.abs(a - b) / scale).max()):.3e}")
