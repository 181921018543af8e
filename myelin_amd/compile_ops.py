"""Compile-visible operators for the checkpointed rate readout.

Registers the HIP rate path with ``torch.library.custom_op`` (fake tensor
rules via ``register_fake``, backward via ``register_autograd``) so that
``torch.compile`` traces through the allocation/launch boundary instead of
breaking the graph at an opaque ``autograd.Function``.  Mirrors the
reference's ``myelin.triton.compile_ops`` (triton/compile_ops.py:23-561):
the same four operators, argument order, outputs and fast_sigmoid backward,
in the ``myelin_amd`` namespace (so both libraries can be imported
side by side).  ``kernels.linear_surrogate_lif_rate_forward(...,
backend="triton_compile")`` dispatches here, as the reference does
(kernels.py:637-684).

Tile knobs (``block_b``, ``block_n``, ``block_f``) are accepted and ignored:
the HIP kernels choose their own tiles.
"""

from __future__ import annotations

from typing import Any

import torch
from torch.library import custom_op

from myelin_amd import _lib
from myelin_amd.surrogates import surrogate_id

_FAST_SIGMOID = surrogate_id("fast_sigmoid")


def _rate_forward(inputs, weight, bias, decay, threshold, reset, checkpoint_size):
    from myelin_amd.linear import _lif_fwd

    _lib.require_device(inputs, "inputs")
    x = inputs.contiguous()
    w = weight.contiguous()
    b = None if bias is None else bias.contiguous()
    T, B, _F = x.shape
    N = w.shape[1]
    dev = x.device
    final_membrane = torch.empty((B, N), dtype=x.dtype, device=dev)
    spike_rates = torch.empty((B, N), dtype=x.dtype, device=dev)
    chunk_starts = torch.empty(((T + checkpoint_size - 1) // checkpoint_size, B, N), dtype=x.dtype, device=dev)
    with torch.cuda.device(dev):
        _lif_fwd(x, w, b, None, 0, T, float(decay), float(threshold), float(reset), 10.0, _lib.RULE_THRESHOLD,
                 _lib.PREC["fp32"], _lib.stream(dev), m_final=final_membrane, rates=spike_rates, ckpt=chunk_starts,
                 ckpt_every=checkpoint_size, exact=True)
    return final_membrane, spike_rates, chunk_starts


def _rate_grads(inputs, weight, bias, chunk_starts, grad_final, grad_rates, decay, threshold, reset, slope,
                checkpoint_size):
    from myelin_amd.linear import linear_backward

    x = inputs.contiguous()
    return linear_backward(x, weight.contiguous(), None if bias is None else bias.contiguous(), None,
                           chunk_starts.contiguous(), None, grad_final, grad_rates, float(decay), float(threshold),
                           float(reset), _FAST_SIGMOID, float(slope), int(checkpoint_size), True,
                           _lib.PREC["fp32"], _lib.RULE_THRESHOLD, True, True, bias is not None)


# --------------------------------------------------------------------- forward


@custom_op("myelin_amd::linear_lif_checkpoint_rate_forward_no_bias", mutates_args=())
def linear_lif_checkpoint_rate_forward_no_bias_op(
    inputs: torch.Tensor,
    weight: torch.Tensor,
    decay: float,
    threshold: float,
    reset: float,
    surrogate_slope: float,
    checkpoint_size: int,
    block_b: int,
    block_n: int,
    block_f: int,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """``(final_membrane, spike_rates, chunk_start_membranes)`` of the
    checkpointed rate forward without bias (triton/compile_ops.py:23-94)."""

    return _rate_forward(inputs, weight, None, decay, threshold, reset, checkpoint_size)


@custom_op("myelin_amd::linear_lif_checkpoint_rate_forward_bias", mutates_args=())
def linear_lif_checkpoint_rate_forward_bias_op(
    inputs: torch.Tensor,
    weight: torch.Tensor,
    bias: torch.Tensor,
    decay: float,
    threshold: float,
    reset: float,
    surrogate_slope: float,
    checkpoint_size: int,
    block_b: int,
    block_n: int,
    block_f: int,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """The same with a bias (triton/compile_ops.py:97-154)."""

    return _rate_forward(inputs, weight, bias, decay, threshold, reset, checkpoint_size)


# ----------------------------------------------------------------- gradients


@custom_op("myelin_amd::linear_lif_checkpoint_rate_grads_no_bias", mutates_args=())
def linear_lif_checkpoint_rate_grads_no_bias_op(
    inputs: torch.Tensor,
    weight: torch.Tensor,
    chunk_start_membranes: torch.Tensor,
    grad_final_membrane: torch.Tensor,
    grad_spike_rates: torch.Tensor,
    decay: float,
    threshold: float,
    reset: float,
    surrogate_slope: float,
    checkpoint_size: int,
    block_b: int,
    block_n: int,
    block_f: int,
) -> tuple[torch.Tensor, torch.Tensor]:
    """``(dinput, dweight)``, fast_sigmoid surrogate (triton/compile_ops.py:157-200)."""

    gx, gw, _ = _rate_grads(inputs, weight, None, chunk_start_membranes, grad_final_membrane, grad_spike_rates,
                            decay, threshold, reset, surrogate_slope, checkpoint_size)
    return gx, gw


@custom_op("myelin_amd::linear_lif_checkpoint_rate_grads_bias", mutates_args=())
def linear_lif_checkpoint_rate_grads_bias_op(
    inputs: torch.Tensor,
    weight: torch.Tensor,
    bias: torch.Tensor,
    chunk_start_membranes: torch.Tensor,
    grad_final_membrane: torch.Tensor,
    grad_spike_rates: torch.Tensor,
    decay: float,
    threshold: float,
    reset: float,
    surrogate_slope: float,
    checkpoint_size: int,
    block_b: int,
    block_n: int,
    block_f: int,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """``(dinput, dweight, dbias)``, fast_sigmoid surrogate (triton/compile_ops.py:203-249)."""

    return _rate_grads(inputs, weight, bias, chunk_start_membranes, grad_final_membrane, grad_spike_rates,
                       decay, threshold, reset, surrogate_slope, checkpoint_size)


# ------------------------------------------------------------ fake tensors


def _forward_fake(inputs, weight, checkpoint_size):
    T, B = inputs.shape[0], inputs.shape[1]
    N = weight.shape[1]
    chunks = (T + checkpoint_size - 1) // checkpoint_size
    return (inputs.new_empty((B, N)), inputs.new_empty((B, N)), inputs.new_empty((chunks, B, N)))


@linear_lif_checkpoint_rate_forward_no_bias_op.register_fake
def _(inputs, weight, decay, threshold, reset, surrogate_slope, checkpoint_size, block_b, block_n, block_f):
    return _forward_fake(inputs, weight, checkpoint_size)


@linear_lif_checkpoint_rate_forward_bias_op.register_fake
def _(inputs, weight, bias, decay, threshold, reset, surrogate_slope, checkpoint_size, block_b, block_n, block_f):
    return _forward_fake(inputs, weight, checkpoint_size)


@linear_lif_checkpoint_rate_grads_no_bias_op.register_fake
def _(inputs, weight, chunk_start_membranes, grad_final_membrane, grad_spike_rates, decay, threshold, reset,
      surrogate_slope, checkpoint_size, block_b, block_n, block_f):
    return torch.empty_like(inputs, memory_format=torch.contiguous_format), torch.empty_like(weight)


@linear_lif_checkpoint_rate_grads_bias_op.register_fake
def _(inputs, weight, bias, chunk_start_membranes, grad_final_membrane, grad_spike_rates, decay, threshold,
      reset, surrogate_slope, checkpoint_size, block_b, block_n, block_f):
    return (torch.empty_like(inputs, memory_format=torch.contiguous_format), torch.empty_like(weight),
            torch.empty_like(bias))


# ----------------------------------------------------------------- autograd


def _setup(ctx: Any, inputs: tuple, output: tuple, has_bias: bool) -> None:
    if has_bias:
        x, w, b, decay, threshold, reset, slope, ck, bb, bn, bf = inputs
    else:
        x, w, decay, threshold, reset, slope, ck, bb, bn, bf = inputs
        b = None
    ctx.save_for_backward(x, w, output[2], *(() if b is None else (b,)))
    ctx.args = (decay, threshold, reset, slope, ck, bb, bn, bf)
    ctx.has_bias = has_bias


def _backward(ctx: Any, grad_final, grad_rates, _grad_chunks):
    n_in = 11 if ctx.has_bias else 10
    if grad_final is None and grad_rates is None:
        return (None,) * n_in
    x, w, chunks = ctx.saved_tensors[:3]
    B, N = x.shape[1], w.shape[1]
    gf = x.new_zeros((B, N)) if grad_final is None else grad_final
    gr = x.new_zeros((B, N)) if grad_rates is None else grad_rates
    if ctx.has_bias:
        b = ctx.saved_tensors[3]
        gx, gw, gb = linear_lif_checkpoint_rate_grads_bias_op(x, w, b, chunks, gf, gr, *ctx.args)
    else:
        gx, gw = linear_lif_checkpoint_rate_grads_no_bias_op(x, w, chunks, gf, gr, *ctx.args)
        gb = None
    needs = ctx.needs_input_grad
    grads = [gx if needs[0] else None, gw if needs[1] else None]
    if ctx.has_bias:
        grads.append(gb if needs[2] else None)
    return tuple(grads) + (None,) * (n_in - len(grads))


linear_lif_checkpoint_rate_forward_no_bias_op.register_autograd(
    _backward, setup_context=lambda ctx, inputs, output: _setup(ctx, inputs, output, False))
linear_lif_checkpoint_rate_forward_bias_op.register_autograd(
    _backward, setup_context=lambda ctx, inputs, output: _setup(ctx, inputs, output, True))
