"""Public fused-kernel entry points (the drop-in boundary of ``myelin.kernels``,
kernels.py:30-865).

Same function names, positional and keyword arguments, defaults, return
types and validation messages as the reference.  ``backend`` accepts every
name the reference does; all of them select the single HIP path, so
callers that pass ``"triton"``, ``"triton_generated"``, ``"auto"`` or
``"torch"`` run unchanged.  Triton tile knobs (``block_size``, ``block_b``,
``block_n``, ``block_f``) are accepted and ignored: the HIP kernels pick
their own launch shapes.  Inputs must be fp32 ROCm device tensors; there is
no CPU fallback.
"""

from __future__ import annotations

from typing import Literal

import torch

from myelin_amd import _lib
from myelin_amd.autograd import HipALIFFunction, HipLIFFunction
from myelin_amd.checkpointing import CheckpointSize, resolve_checkpoint_size
from myelin_amd.neurons import ALIFParams, ALIFState, LIFParams, LIFState
from myelin_amd.packing import PackedSpikes, packed_last_dim_size
from myelin_amd.surrogates import SurrogateName, surrogate_id

Backend = Literal["auto", "torch", "hip", "triton", "triton_generated", "triton_compile"]
_BACKENDS = ("auto", "torch", "hip", "triton", "triton_generated", "triton_compile")


def _check_backend(backend: str) -> None:
    if backend not in _BACKENDS:
        raise ValueError(f"unsupported backend: {backend}")


def _check_inputs(inputs: torch.Tensor, what: str = "inputs", dims: str = "[T, B, N]") -> None:
    if inputs.ndim != 3:
        raise ValueError(f"{what} must be shaped {dims}; got {tuple(inputs.shape)}")
    _lib.require_device(inputs, what)
    if inputs.dtype != torch.float32:
        raise ValueError(f"{what} must be float32 for the HIP path; got {inputs.dtype}")
    if inputs.shape[0] == 0:
        raise ValueError(f"{what} must have at least one timestep")


def _check_state(t: torch.Tensor, inputs: torch.Tensor, name: str) -> torch.Tensor:
    if t.shape != inputs.shape[1:]:
        raise ValueError(
            f"initial_state.{name} must match inputs.shape[1:]; "
            f"got {tuple(t.shape)} and {tuple(inputs.shape[1:])}"
        )
    if t.device != inputs.device:
        raise ValueError(f"initial_state.{name} must be on the same device as inputs")
    if t.dtype != inputs.dtype:
        raise ValueError(f"initial_state.{name} must have the same dtype as inputs")
    return t.contiguous()


def _f32(v: float) -> float:
    return float(v)


def lif_forward(
    inputs: torch.Tensor,
    initial_state: LIFState,
    params: LIFParams,
    *,
    backend: Backend = "auto",
    block_size: int = 256,
) -> tuple[LIFState, torch.Tensor]:
    """Fused-time hard-reset LIF (kernels.py:52-93).

    Spikes are bit-identical to ``lif_unroll`` (functional.py:21-45) and
    carry no gradient, as in that function; the final membrane is
    differentiable with respect to inputs and the initial membrane.
    """

    _check_backend(backend)
    _check_inputs(inputs)
    m0 = _check_state(initial_state.membrane, inputs, "membrane")
    with torch.cuda.device(inputs.device):
        m, spikes = HipLIFFunction.apply(
            inputs.contiguous(), m0, _f32(params.decay), _f32(params.threshold), _f32(params.reset),
            0.0, _lib.RULE_THRESHOLD, _lib.SG_NONE,
        )
    return LIFState(membrane=m), spikes


fused_lif_unroll = lif_forward
"""Compatibility alias (kernels.py:849-865)."""


def lif_forward_packed_spikes(
    inputs: torch.Tensor,
    initial_state: LIFState,
    params: LIFParams,
    *,
    backend: Backend = "auto",
    block_b: int = 8,
) -> tuple[LIFState, PackedSpikes]:
    """LIF forward writing spikes straight into int32 words (kernels.py:96-156).

    A wave ballot packs 64 neurons per step, so the dense ``[T, B, N]``
    spikes are never written.  Forward only, like the reference.
    """

    _check_backend(backend)
    _check_inputs(inputs)
    m0 = _check_state(initial_state.membrane, inputs, "membrane")
    x = inputs.contiguous()
    T, B, N = x.shape
    m = torch.empty_like(m0)
    words = torch.empty((T, B, packed_last_dim_size(N)), dtype=torch.int32, device=x.device)
    with torch.cuda.device(x.device):
        _lib.call(
            "myelin_lif_fwd_f32",
            _lib.ptr(x), _lib.ptr(m0), _lib.ptr(m), None, _lib.ptr(words), None,
            T, B, N, _f32(params.decay), _f32(params.threshold), _f32(params.reset), 0.0,
            _lib.RULE_THRESHOLD, 1, _lib.stream(x.device),
        )
    return LIFState(membrane=m), PackedSpikes(data=words, original_shape=tuple(inputs.shape))


def alif_forward(
    inputs: torch.Tensor,
    initial_state: ALIFState,
    params: ALIFParams,
    *,
    backend: Backend = "auto",
    block_size: int = 256,
) -> tuple[ALIFState, torch.Tensor]:
    """Fused-time adaptive LIF (kernels.py:159-199).

    Bit-identical to ``alif_unroll`` (functional.py:48-78); final membrane
    and adaptation are differentiable (membrane path), spikes are not.
    """

    _check_backend(backend)
    _check_inputs(inputs)
    m0 = _check_state(initial_state.membrane, inputs, "membrane")
    a0 = _check_state(initial_state.adaptation, inputs, "adaptation")
    with torch.cuda.device(inputs.device):
        m, a, spikes = HipALIFFunction.apply(
            inputs.contiguous(), m0, a0, _f32(params.decay), _f32(params.adaptation_decay),
            _f32(params.threshold), _f32(params.beta), _f32(params.reset), 0.0,
            _lib.RULE_THRESHOLD, _lib.SG_NONE,
        )
    return ALIFState(membrane=m, adaptation=a), spikes


def surrogate_lif_forward(
    inputs: torch.Tensor,
    initial_state: LIFState,
    params: LIFParams,
    *,
    surrogate: SurrogateName = "atan",
    surrogate_slope: float = 10.0,
    hard_forward: bool = True,
    backend: Backend = "auto",
    block_size: int = 256,
) -> tuple[LIFState, torch.Tensor]:
    """Hard-forward surrogate LIF with a fused reverse-time backward (kernels.py:249-337)."""

    sid = surrogate_id(surrogate)
    _check_backend(backend)
    if not hard_forward:
        raise ValueError("HIP surrogate LIF currently supports only hard_forward=True")
    _check_inputs(inputs)
    m0 = _check_state(initial_state.membrane, inputs, "membrane")
    with torch.cuda.device(inputs.device):
        m, spikes = HipLIFFunction.apply(
            inputs.contiguous(), m0, _f32(params.decay), _f32(params.threshold), _f32(params.reset),
            _f32(surrogate_slope), _lib.RULE_SURROGATE, sid,
        )
    return LIFState(membrane=m), spikes


def surrogate_alif_forward(
    inputs: torch.Tensor,
    initial_state: ALIFState,
    params: ALIFParams,
    *,
    surrogate: SurrogateName = "atan",
    surrogate_slope: float = 10.0,
    hard_forward: bool = True,
    backend: Backend = "auto",
) -> tuple[ALIFState, torch.Tensor]:
    """Hard-forward surrogate ALIF with the fused two-state adjoint (kernels.py:340-392).

    The reference has no fused path here (it falls back to torch autograd);
    the gradient matches autograd through ``surrogate_alif_unroll``.
    """

    sid = surrogate_id(surrogate)
    _check_backend(backend)
    if not hard_forward:
        raise ValueError("HIP surrogate ALIF currently supports only hard_forward=True")
    _check_inputs(inputs)
    m0 = _check_state(initial_state.membrane, inputs, "membrane")
    a0 = _check_state(initial_state.adaptation, inputs, "adaptation")
    with torch.cuda.device(inputs.device):
        m, a, spikes = HipALIFFunction.apply(
            inputs.contiguous(), m0, a0, _f32(params.decay), _f32(params.adaptation_decay),
            _f32(params.threshold), _f32(params.beta), _f32(params.reset), _f32(surrogate_slope),
            _lib.RULE_SURROGATE, sid,
        )
    return ALIFState(membrane=m, adaptation=a), spikes


def _resolve(inputs: torch.Tensor, checkpoint_size: CheckpointSize | None) -> int | None:
    if checkpoint_size is None:
        return None
    return resolve_checkpoint_size(int(inputs.shape[0]), checkpoint_size)
