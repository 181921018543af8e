"""Public fused-kernel entry points (the drop-in boundary of ``myelin.kernels``,
kernels.py:30-865).

Same function names, positional and keyword arguments, defaults, return
types and validation messages as the reference.  ``backend`` accepts every
name the reference does and every name runs the HIP kernels, so callers
that pass ``"triton"``, ``"triton_generated"``, ``"auto"`` or ``"torch"``
run unchanged.  For the surrogate LIF/ALIF forwards the name also picks the
arithmetic the reference would have run: torch autograd's (straight-through
spike values, autograd's operation order) or its fused GPU kernels' (0/1
spikes, closed-form derivative).  Triton tile knobs (``block_size``, ``block_b``,
``block_n``, ``block_f``) are accepted and ignored: the HIP kernels pick
their own launch shapes.  Inputs must be fp32 ROCm device tensors; there is
no CPU fallback.
"""

from __future__ import annotations

from typing import Literal

import torch

from myelin_amd import _lib
from myelin_amd.autograd import BWD_CHUNK, HipALIFFunction, HipLIFFunction
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


def _direct(*tensors: torch.Tensor) -> bool:
    """No autograd graph is needed and the tensors are on the current device:
    the forward can launch directly, without the autograd Function and the
    device switch (the same entry point and outputs, less host time)."""

    if torch.is_grad_enabled() and any(t.requires_grad for t in tensors):
        return False
    return tensors[0].device.index == torch.cuda.current_device()


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
    x = inputs.contiguous()
    if _direct(x, m0):
        T, B, N = x.shape
        m = torch.empty_like(m0)
        spikes = torch.empty_like(x)
        _lib.call("myelin_lif_fwd_f32", x.data_ptr(), m0.data_ptr(), m.data_ptr(), spikes.data_ptr(), None, None,
                  T, B, N, _f32(params.decay), _f32(params.threshold), _f32(params.reset), 0.0,
                  _lib.RULE_THRESHOLD, BWD_CHUNK, _lib.stream(x.device))
        return LIFState(membrane=m), spikes
    with torch.cuda.device(inputs.device):
        m, spikes = HipLIFFunction.apply(
            x, m0, _f32(params.decay), _f32(params.threshold), _f32(params.reset),
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
    x = inputs.contiguous()
    if _direct(x, m0, a0):
        T, B, N = x.shape
        m, a = torch.empty_like(m0), torch.empty_like(a0)
        spikes = torch.empty_like(x)
        _lib.call("myelin_alif_fwd_f32", x.data_ptr(), m0.data_ptr(), a0.data_ptr(), m.data_ptr(), a.data_ptr(),
                  spikes.data_ptr(), None, None, None, T, B, N, _f32(params.decay), _f32(params.adaptation_decay),
                  _f32(params.threshold), _f32(params.beta), _f32(params.reset), 0.0, _lib.RULE_THRESHOLD,
                  BWD_CHUNK, _lib.stream(x.device))
        return ALIFState(membrane=m, adaptation=a), spikes
    with torch.cuda.device(inputs.device):
        m, a, spikes = HipALIFFunction.apply(
            x, m0, a0, _f32(params.decay), _f32(params.adaptation_decay),
            _f32(params.threshold), _f32(params.beta), _f32(params.reset), 0.0,
            _lib.RULE_THRESHOLD, _lib.SG_NONE,
        )
    return ALIFState(membrane=m, adaptation=a), spikes


def _surrogate_codes(sid: int, hard_forward: bool, autograd_order: bool) -> tuple[int, int]:
    """(forward spike rule, backward surrogate code) of one arithmetic.

    ``autograd_order``: the arithmetic of myelin's torch backend
    (``surrogate_*_unroll`` differentiated by autograd, functional.py:115-189):
    straight-through spike values ``(H + sigma) - sigma`` (or ``sigma`` when
    ``hard_forward=False``), reset ``m'(1 - s) + reset s`` and the adjoint
    in autograd's operation order.  Otherwise the fused GPU kernels'
    arithmetic (triton/lif.py:195-288): exact 0/1 spikes and the closed-form
    ``sigma'(c)`` of surrogates.py:78-102.
    """

    if autograd_order:
        if hard_forward:
            return _lib.RULE_STRAIGHT_THROUGH + sid, _lib.SG_AUTOGRAD + sid
        return _lib.RULE_SMOOTH + sid, _lib.SG_AUTOGRAD_SMOOTH + sid
    return _lib.RULE_SURROGATE, sid


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
    """Surrogate LIF with a fused reverse-time backward (kernels.py:249-337).

    The backend picks the arithmetic the reference would run on a GPU
    tensor: ``"torch"`` (and any backend with ``hard_forward=False``, which
    the reference sends to torch) reproduces ``surrogate_lif_unroll`` under
    torch autograd -- straight-through spike values and autograd's operation
    order; ``"auto"``, ``"hip"``, ``"triton"`` and ``"triton_generated"``
    run the fused kernels' arithmetic (0/1 spikes, closed-form derivative),
    as the reference's Triton route does (triton/lif.py:195-288).
    """

    sid = surrogate_id(surrogate)
    _check_backend(backend)
    if not hard_forward and backend == "triton":
        raise ValueError("Triton surrogate LIF currently supports only hard_forward=True")
    if not hard_forward and backend == "triton_generated":
        raise ValueError("generated Triton surrogate LIF currently supports only hard_forward=True")
    _check_inputs(inputs)
    m0 = _check_state(initial_state.membrane, inputs, "membrane")
    rule, code = _surrogate_codes(sid, hard_forward, backend == "torch" or not hard_forward)
    with torch.cuda.device(inputs.device):
        m, spikes = HipLIFFunction.apply(
            inputs.contiguous(), m0, _f32(params.decay), _f32(params.threshold), _f32(params.reset),
            _f32(surrogate_slope), rule, code,
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
    """Surrogate ALIF with the fused two-state adjoint (kernels.py:340-392).

    The reference runs this only through torch autograd (``"auto"`` falls
    back to it, kernels.py:374-389), so ``"auto"`` and ``"torch"`` reproduce
    that arithmetic: straight-through spike values and the adjoint in
    autograd's operation order, in the fused kernels.  ``"hip"``,
    ``"triton"`` and ``"triton_generated"`` select the fused kernels' own
    arithmetic (0/1 spikes, closed-form derivative); with
    ``hard_forward=False`` every backend runs the smooth forward of
    ``surrogate_alif_unroll`` in autograd order.
    """

    sid = surrogate_id(surrogate)
    _check_backend(backend)
    _check_inputs(inputs)
    m0 = _check_state(initial_state.membrane, inputs, "membrane")
    a0 = _check_state(initial_state.adaptation, inputs, "adaptation")
    autograd_order = backend in ("auto", "torch") or not hard_forward
    rule, code = _surrogate_codes(sid, hard_forward, autograd_order)
    with torch.cuda.device(inputs.device):
        m, a, spikes = HipALIFFunction.apply(
            inputs.contiguous(), m0, a0, _f32(params.decay), _f32(params.adaptation_decay),
            _f32(params.threshold), _f32(params.beta), _f32(params.reset), _f32(surrogate_slope),
            rule, code,
        )
    return ALIFState(membrane=m, adaptation=a), spikes


def _lean(checkpoint_size) -> bool:
    """The memory policy asks for small chunk scratch (checkpointing.py:13-20):
    the HIP layers then size their chunk and span buffers to one checkpoint
    chunk instead of 2**25 floats (an int checkpoint size keeps the larger,
    faster buffers)."""

    return checkpoint_size == "memory"


def _resolve(inputs: torch.Tensor, checkpoint_size: CheckpointSize | None) -> int | None:
    if checkpoint_size is None:
        return None
    return resolve_checkpoint_size(int(inputs.shape[0]), checkpoint_size)


def linear_surrogate_lif_forward(
    inputs: torch.Tensor,
    weight: torch.Tensor,
    bias: torch.Tensor | None,
    params: LIFParams,
    *,
    surrogate: SurrogateName = "atan",
    surrogate_slope: float = 10.0,
    hard_forward: bool = True,
    backend: Backend = "auto",
    checkpoint_size: CheckpointSize | None = None,
    block_b: int = 16,
    block_n: int = 32,
    block_f: int = 32,
    synapse_precision: Literal["fp32", "bf16"] = "fp32",
) -> tuple[LIFState, torch.Tensor]:
    """Dense projection streamed through surrogate LIF (kernels.py:395-562).

    ``inputs [T, B, F] @ weight [F, N] (+ bias)`` is computed on MFMA tiles
    fused ahead of the neuron update; the membrane starts at zero.
    ``checkpoint_size=None`` saves the pre-reset trace for the backward;
    an int or policy saves chunk-start membranes and recomputes chunks.
    ``synapse_precision="bf16"`` rounds the GEMM inputs to bf16 (fp32
    accumulate); the default keeps the reference's fp32 matmul.
    """

    from myelin_amd.linear import linear_forward

    sid = surrogate_id(surrogate)
    _check_backend(backend)
    if not hard_forward:
        raise ValueError("HIP linear surrogate LIF currently supports only hard_forward=True")
    ck = _resolve(inputs, checkpoint_size)
    m, spikes = linear_forward(inputs, weight, bias, params, sid, surrogate_slope, ck, False, synapse_precision,
                               lean=_lean(checkpoint_size))
    return LIFState(membrane=m), spikes


def linear_surrogate_lif_rate_forward(
    inputs: torch.Tensor,
    weight: torch.Tensor,
    bias: torch.Tensor | None,
    params: LIFParams,
    *,
    surrogate: SurrogateName = "atan",
    surrogate_slope: float = 10.0,
    hard_forward: bool = True,
    backend: Backend = "auto",
    checkpoint_size: CheckpointSize = 25,
    block_b: int = 16,
    block_n: int = 32,
    block_f: int = 32,
    reduction: Literal["mean", "none"] = "mean",
    synapse_precision: Literal["fp32", "bf16"] = "fp32",
) -> tuple[LIFState, torch.Tensor]:
    """Dense projection + surrogate LIF returning spike rates (kernels.py:565-702).

    The forward keeps spike counts in registers and writes only ``[B, N]``
    rates and chunk-start membranes: no ``[T, B, N]`` tensor is written.
    The backward injects ``grad_rates / T`` at every step.
    """

    from myelin_amd.linear import linear_forward

    sid = surrogate_id(surrogate)
    _check_backend(backend)
    if not hard_forward:
        if backend == "triton_compile":
            raise ValueError(
                "backend='triton_compile' is experimental and currently supports only hard_forward=True"
            )
        raise ValueError("HIP spike-rate LIF currently supports only hard_forward=True")
    if reduction not in ("mean", "none"):
        raise ValueError("reduction must be 'mean' or 'none'")
    ck = resolve_checkpoint_size(int(inputs.shape[0]), checkpoint_size)
    if backend == "triton_compile":
        # the compile-visible operators (kernels.py:637-684 of the reference)
        if surrogate != "fast_sigmoid":
            raise ValueError(
                "backend='triton_compile' is experimental and currently supports only surrogate='fast_sigmoid'"
            )
        from myelin_amd import compile_ops

        if bias is None:
            m, rates, _ = compile_ops.linear_lif_checkpoint_rate_forward_no_bias_op(
                inputs, weight, params.decay, params.threshold, params.reset, surrogate_slope, ck, block_b,
                block_n, block_f)
        else:
            m, rates, _ = compile_ops.linear_lif_checkpoint_rate_forward_bias_op(
                inputs, weight, bias, params.decay, params.threshold, params.reset, surrogate_slope, ck, block_b,
                block_n, block_f)
    else:
        m, rates = linear_forward(inputs, weight, bias, params, sid, surrogate_slope, ck, True, synapse_precision,
                                  lean=_lean(checkpoint_size))
    if reduction == "mean":
        return LIFState(membrane=m), rates.mean()
    return LIFState(membrane=m), rates


def linear_surrogate_lif_packed_forward(
    inputs: torch.Tensor,
    weight: torch.Tensor,
    bias: torch.Tensor | None,
    params: LIFParams,
    *,
    surrogate: SurrogateName = "atan",
    surrogate_slope: float = 10.0,
    hard_forward: bool = True,
    backend: Backend = "auto",
    checkpoint_size: CheckpointSize = 25,
    block_b: int = 16,
    block_f: int = 32,
    synapse_precision: Literal["fp32", "bf16"] = "fp32",
) -> tuple[LIFState, PackedSpikes]:
    """Dense projection + LIF writing bitpacked spikes only (kernels.py:705-776).

    Forward-only, like the reference: a wave ballot packs 64 neurons per step
    straight from the fused kernel, so dense spikes are never written.
    """

    from myelin_amd.linear import linear_packed_forward

    surrogate_id(surrogate)
    _check_backend(backend)
    if not hard_forward:
        raise ValueError("HIP packed surrogate LIF currently supports only hard_forward=True")
    ck = resolve_checkpoint_size(int(inputs.shape[0]), checkpoint_size)
    m, packed = linear_packed_forward(inputs, weight, bias, params, ck, synapse_precision)
    return LIFState(membrane=m), packed


def two_layer_surrogate_lif_rate_recompute_forward(
    inputs: torch.Tensor,
    hidden_weight: torch.Tensor,
    hidden_bias: torch.Tensor | None,
    output_weight: torch.Tensor,
    output_bias: torch.Tensor | None,
    params: LIFParams,
    *,
    surrogate: SurrogateName = "fast_sigmoid",
    surrogate_slope: float = 5.0,
    hard_forward: bool = True,
    checkpoint_size: CheckpointSize = 25,
    synapse_precision: Literal["fp32", "bf16"] = "fp32",
) -> torch.Tensor:
    """Two-layer LIF rate network, input -> hidden -> readout rates ``[B, O]``
    (kernels.py:779-808; autograd.py:926-1126).

    Only the inputs, weights and chunk-start membranes of both layers are
    kept for the backward; the two layers run interleaved per checkpoint
    chunk, so hidden spikes and their gradient exist one chunk at a time.
    """

    from myelin_amd.two_layer import two_layer_rate_forward

    sid = surrogate_id(surrogate)
    if not hard_forward:
        raise ValueError("two-layer recompute currently supports only hard_forward=True")
    ck = resolve_checkpoint_size(int(inputs.shape[0]), checkpoint_size)
    return two_layer_rate_forward(inputs, hidden_weight, hidden_bias, output_weight, output_bias, params, sid,
                                  surrogate_slope, ck, synapse_precision, packed_hidden=False,
                                  lean=_lean(checkpoint_size))


def two_layer_surrogate_lif_rate_packed_hidden_forward(
    inputs: torch.Tensor,
    hidden_weight: torch.Tensor,
    hidden_bias: torch.Tensor | None,
    output_weight: torch.Tensor,
    output_bias: torch.Tensor | None,
    params: LIFParams,
    *,
    surrogate: SurrogateName = "fast_sigmoid",
    surrogate_slope: float = 5.0,
    hard_forward: bool = True,
    checkpoint_size: CheckpointSize = 25,
    block_b: int = 16,
    block_n: int = 32,
    block_f: int = 32,
    synapse_precision: Literal["fp32", "bf16"] = "fp32",
) -> torch.Tensor:
    """Two-layer LIF rate network that keeps the hidden spikes bitpacked
    (kernels.py:811-846; autograd.py:1129-1387).

    The forward's hidden kernel ballots the spikes straight into
    ``[T, B, ceil(H/32)]`` int32 words; the backward unpacks one checkpoint
    chunk at a time as the readout's input (the reference unpacks all T).
    Triton tile knobs are accepted and ignored.
    """

    from myelin_amd.two_layer import two_layer_rate_forward

    sid = surrogate_id(surrogate)
    if not hard_forward:
        raise ValueError("packed-hidden two-layer rate training supports only hard_forward=True")
    if not inputs.is_cuda:
        raise ValueError("packed-hidden two-layer rate training requires CUDA tensors")
    ck = resolve_checkpoint_size(int(inputs.shape[0]), checkpoint_size)
    return two_layer_rate_forward(inputs, hidden_weight, hidden_bias, output_weight, output_bias, params, sid,
                                  surrogate_slope, ck, synapse_precision, packed_hidden=True,
                                  lean=_lean(checkpoint_size))
