"""``nn.Module`` wrappers of the fused path (same constructors, defaults and
outputs as the hot-path classes of ``myelin.modules``, modules.py:112-943).

Every forward runs HIP kernels; ``backend`` arguments are accepted for
signature compatibility and select the same HIP path.  The streamed-synapse
modules take one keyword the reference does not have,
``synapse_precision`` ("fp32", the reference's arithmetic, or "bf16" MFMA
inputs with fp32 accumulation).
"""

from __future__ import annotations

from typing import Literal

import torch
from torch import nn

from myelin_amd.checkpointing import CheckpointSize
from myelin_amd.kernels import (
    Backend,
    alif_forward,
    lif_forward,
    linear_surrogate_lif_forward,
    linear_surrogate_lif_packed_forward,
    linear_surrogate_lif_rate_forward,
    surrogate_alif_forward,
    surrogate_lif_forward,
)
from myelin_amd.linear import linear
from myelin_amd.neurons import ALIFParams, ALIFState, LIFParams, LIFState
from myelin_amd.packing import PackedSpikes
from myelin_amd.surrogates import SurrogateFn, atan_surrogate, fast_sigmoid_surrogate, surrogate_name

Precision = Literal["fp32", "bf16"]


class LinearSynapse(nn.Module):
    """Trainable dense projection over time-major inputs (modules.py:112-133).

    Weight ``[in, out]`` initialised ``(rand - 0.5) * 0.02``, bias zeros; the
    projection runs on the MFMA GEMM with the bias added in its epilogue.
    """

    def __init__(self, in_features: int, out_features: int, params: LIFParams | None = None, bias: bool = True,
                 synapse_precision: Precision = "fp32") -> None:
        super().__init__()
        self.weight = nn.Parameter((torch.rand((in_features, out_features)) - 0.5) * 0.02)
        if bias:
            self.bias = nn.Parameter(torch.zeros(out_features))
        else:
            self.register_parameter("bias", None)
        self.synapse_precision = synapse_precision

    def forward(self, inputs: torch.Tensor) -> torch.Tensor:
        return linear(inputs, self.weight, self.bias, self.synapse_precision)


class LIFCell(nn.Module):
    """Single-step LIF population (one fused step, T = 1)."""

    def __init__(self, params: LIFParams | None = None) -> None:
        super().__init__()
        self.params = params or LIFParams()

    def forward(self, state: LIFState, input_current: torch.Tensor) -> tuple[LIFState, torch.Tensor]:
        st, s = lif_forward(input_current.unsqueeze(0), state, self.params)
        return st, s[0]


class ALIFCell(nn.Module):
    """Single-step ALIF population (one fused step, T = 1)."""

    def __init__(self, params: ALIFParams | None = None) -> None:
        super().__init__()
        self.params = params or ALIFParams()

    def forward(self, state: ALIFState, input_current: torch.Tensor) -> tuple[ALIFState, torch.Tensor]:
        st, s = alif_forward(input_current.unsqueeze(0), state, self.params)
        return st, s[0]


class SurrogateLIFCell(nn.Module):
    """Single-step hard-forward surrogate LIF (modules.py:211-239)."""

    def __init__(self, params: LIFParams | None = None, surrogate: SurrogateFn = atan_surrogate,
                 surrogate_slope: float = 10.0, hard_forward: bool = True) -> None:
        super().__init__()
        self.params = params or LIFParams()
        self.surrogate = surrogate
        self.surrogate_slope = surrogate_slope
        self.hard_forward = hard_forward

    def forward(self, state: LIFState, input_current: torch.Tensor) -> tuple[LIFState, torch.Tensor]:
        # the reference cell steps through torch ops: autograd arithmetic
        st, s = surrogate_lif_forward(input_current.unsqueeze(0), state, self.params,
                                      surrogate=surrogate_name(self.surrogate), surrogate_slope=self.surrogate_slope,
                                      hard_forward=self.hard_forward, backend="torch")
        return st, s[0]


class SurrogateALIFCell(nn.Module):
    """Single-step hard-forward surrogate ALIF (modules.py:242-269)."""

    def __init__(self, params: ALIFParams | None = None, surrogate: SurrogateFn = atan_surrogate,
                 surrogate_slope: float = 10.0, hard_forward: bool = True) -> None:
        super().__init__()
        self.params = params or ALIFParams()
        self.surrogate = surrogate
        self.surrogate_slope = surrogate_slope
        self.hard_forward = hard_forward

    def forward(self, state: ALIFState, input_current: torch.Tensor) -> tuple[ALIFState, torch.Tensor]:
        st, s = surrogate_alif_forward(input_current.unsqueeze(0), state, self.params,
                                       surrogate=surrogate_name(self.surrogate), surrogate_slope=self.surrogate_slope,
                                       hard_forward=self.hard_forward, backend="torch")
        return st, s[0]


class TimeUnroll(nn.Module):
    """Run a cell over time-major ``[T, B, N]`` inputs in one fused launch
    (modules.py:415-582); the initial state defaults to zeros.  The default
    backend is ``"torch"``, as in the reference: surrogate cells then keep
    the arithmetic of stepping the cell through torch ops."""

    def __init__(self, cell: nn.Module, *, backend: Backend = "torch") -> None:
        super().__init__()
        self.cell = cell
        self.backend: Backend = backend

    def forward(self, inputs: torch.Tensor, initial_state: LIFState | ALIFState | None = None):
        cell = self.cell
        alif = isinstance(cell, (ALIFCell, SurrogateALIFCell))
        if initial_state is None:
            z = torch.zeros(inputs.shape[1:], dtype=inputs.dtype, device=inputs.device)
            initial_state = ALIFState(z, torch.zeros_like(z)) if alif else LIFState(z)
        if isinstance(cell, LIFCell):
            return lif_forward(inputs, initial_state, cell.params, backend=self.backend)
        if isinstance(cell, ALIFCell):
            return alif_forward(inputs, initial_state, cell.params, backend=self.backend)
        if isinstance(cell, SurrogateLIFCell):
            return surrogate_lif_forward(inputs, initial_state, cell.params, surrogate=surrogate_name(cell.surrogate),
                                         surrogate_slope=cell.surrogate_slope, hard_forward=cell.hard_forward,
                                         backend=self.backend)
        if isinstance(cell, SurrogateALIFCell):
            return surrogate_alif_forward(inputs, initial_state, cell.params,
                                          surrogate=surrogate_name(cell.surrogate),
                                          surrogate_slope=cell.surrogate_slope, hard_forward=cell.hard_forward,
                                          backend=self.backend)
        raise TypeError(f"TimeUnroll supports LIF/ALIF cells on the HIP path; got {type(cell).__name__}")


class LinearSurrogateLIF(nn.Module):
    """Dense projection plus surrogate LIF unroll (modules.py:706-750).

    ``stream_synapse=True`` runs the fused synapse + recurrence kernel
    (``linear_surrogate_lif_forward``); otherwise the projection runs on the
    GEMM and the unroll on the fused recurrence.  Returns spikes ``[T, B, N]``.
    """

    def __init__(self, in_features: int, out_features: int, params: LIFParams | None = None,
                 surrogate: SurrogateFn = atan_surrogate, surrogate_slope: float = 10.0, hard_forward: bool = True,
                 bias: bool = True, backend: Backend = "auto", stream_synapse: bool = False,
                 checkpoint_size: CheckpointSize | None = None, synapse_precision: Precision = "fp32") -> None:
        super().__init__()
        self.synapse = LinearSynapse(in_features, out_features, bias=bias, synapse_precision=synapse_precision)
        self.stream_synapse = stream_synapse
        self.checkpoint_size: CheckpointSize | None = checkpoint_size
        self.synapse_precision = synapse_precision
        self.unroll = TimeUnroll(SurrogateLIFCell(params, surrogate, surrogate_slope, hard_forward), backend=backend)

    def forward(self, inputs: torch.Tensor) -> torch.Tensor:
        cell = self.unroll.cell
        if self.stream_synapse:
            _, spikes = linear_surrogate_lif_forward(
                inputs, self.synapse.weight, self.synapse.bias, cell.params,
                surrogate=surrogate_name(cell.surrogate), surrogate_slope=cell.surrogate_slope,
                hard_forward=cell.hard_forward, backend=self.unroll.backend, checkpoint_size=self.checkpoint_size,
                synapse_precision=self.synapse_precision,
            )
            return spikes
        _, spikes = self.unroll(self.synapse(inputs))
        return spikes


class LinearSurrogateLIFRate(nn.Module):
    """Dense projection plus surrogate LIF returning spike rates (modules.py:803-845)."""

    def __init__(self, in_features: int, out_features: int, params: LIFParams | None = None,
                 surrogate: SurrogateFn = atan_surrogate, surrogate_slope: float = 10.0, hard_forward: bool = True,
                 bias: bool = True, backend: Backend = "auto", checkpoint_size: CheckpointSize = 25,
                 reduction: Literal["mean", "none"] = "none", synapse_precision: Precision = "fp32") -> None:
        super().__init__()
        self.synapse = LinearSynapse(in_features, out_features, bias=bias, synapse_precision=synapse_precision)
        self.cell = SurrogateLIFCell(params, surrogate, surrogate_slope, hard_forward)
        self.backend: Backend = backend
        self.checkpoint_size: CheckpointSize = checkpoint_size
        self.reduction: Literal["mean", "none"] = reduction
        self.synapse_precision = synapse_precision

    def forward(self, inputs: torch.Tensor) -> torch.Tensor:
        _, rates = linear_surrogate_lif_rate_forward(
            inputs, self.synapse.weight, self.synapse.bias, self.cell.params,
            surrogate=surrogate_name(self.cell.surrogate), surrogate_slope=self.cell.surrogate_slope,
            hard_forward=self.cell.hard_forward, backend=self.backend, checkpoint_size=self.checkpoint_size,
            reduction=self.reduction, synapse_precision=self.synapse_precision,
        )
        return rates


class LinearSurrogateLIFPacked(nn.Module):
    """Dense projection plus LIF returning bitpacked spikes, forward only (modules.py:906-943)."""

    def __init__(self, in_features: int, out_features: int, params: LIFParams | None = None,
                 surrogate: SurrogateFn = atan_surrogate, surrogate_slope: float = 10.0, hard_forward: bool = True,
                 bias: bool = True, backend: Backend = "auto", checkpoint_size: CheckpointSize = 25,
                 synapse_precision: Precision = "fp32") -> None:
        super().__init__()
        self.synapse = LinearSynapse(in_features, out_features, bias=bias, synapse_precision=synapse_precision)
        self.cell = SurrogateLIFCell(params, surrogate, surrogate_slope, hard_forward)
        self.backend: Backend = backend
        self.checkpoint_size: CheckpointSize = checkpoint_size
        self.synapse_precision = synapse_precision

    def forward(self, inputs: torch.Tensor) -> PackedSpikes:
        _, packed = linear_surrogate_lif_packed_forward(
            inputs, self.synapse.weight, self.synapse.bias, self.cell.params,
            surrogate=surrogate_name(self.cell.surrogate), surrogate_slope=self.cell.surrogate_slope,
            hard_forward=self.cell.hard_forward, backend=self.backend, checkpoint_size=self.checkpoint_size,
            synapse_precision=self.synapse_precision,
        )
        return packed


class RateReadoutClassifier(nn.Module):
    """Streamed hidden LIF layer then a rate readout (modules.py:848-903)."""

    def __init__(self, in_features: int, hidden_features: int, out_features: int, params: LIFParams | None = None,
                 *, surrogate: SurrogateFn = fast_sigmoid_surrogate, surrogate_slope: float = 5.0,
                 hard_forward: bool = True, bias: bool = True, backend: Backend = "auto",
                 checkpoint_size: CheckpointSize = 25, dropout: float = 0.0,
                 synapse_precision: Precision = "fp32") -> None:
        super().__init__()
        self.hidden = LinearSurrogateLIF(in_features, hidden_features, params, surrogate=surrogate,
                                         surrogate_slope=surrogate_slope, hard_forward=hard_forward, bias=bias,
                                         backend=backend, stream_synapse=True, checkpoint_size=checkpoint_size,
                                         synapse_precision=synapse_precision)
        self.dropout = nn.Dropout(dropout)
        self.output = LinearSurrogateLIFRate(hidden_features, out_features, params, surrogate=surrogate,
                                             surrogate_slope=surrogate_slope, hard_forward=hard_forward, bias=bias,
                                             backend=backend, checkpoint_size=checkpoint_size, reduction="none",
                                             synapse_precision=synapse_precision)

    def forward(self, inputs: torch.Tensor) -> torch.Tensor:
        return self.output(self.dropout(self.hidden(inputs)))
