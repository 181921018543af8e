"""``torch.autograd.Function`` boundaries around the HIP recurrence kernels.

Plugin convention follows the reference (autograd.py:130-201): forward takes
tensors plus Python scalars, calls ``ctx.set_materialize_grads(False)``,
saves what backward needs; backward returns one entry per input (``None``
for scalars and for inputs that need no gradient).

Memory policy: the forward saves the input currents ``x`` (by reference, no
copy) and chunk-start states every ``BWD_CHUNK`` steps -- 8/C bytes per
neuron-step for ALIF -- instead of the reference Triton path's ``[T,B,N]``
pre-reset trace plus packed spikes (autograd.py:161-163).  The backward
re-reads ``x`` once to recompute each chunk.
"""

from __future__ import annotations

import math
from typing import Any

import torch

from myelin_amd import _lib

# chunk length of the checkpointed backward (a compiled kernel parameter,
# 8 or 16).  16 halves the checkpoint traffic of 8 (0.5 instead of 1 B per
# neuron-step for ALIF, each way); the backward issues its loads a quarter
# chunk at a time so its registers stay near those of 8.  ALIF [256, 128,
# 4096] fast_sigmoid: forward 190.5 -> 183.5 us, backward 270 -> 268 us.
BWD_CHUNK = 16


def _chunks(T: int) -> int:
    return math.ceil(T / BWD_CHUNK)


def _contig_f32(t: torch.Tensor | None) -> torch.Tensor | None:
    if t is None:
        return None
    if t.dtype != torch.float32:
        t = t.float()
    return t.contiguous()


class HipLIFFunction(torch.autograd.Function):
    """Fused-time LIF with a reverse-time adjoint.

    ``sid == SG_NONE`` is the plain ``lif_unroll`` (spikes carry no gradient,
    functional.py:21-45); otherwise the hard-forward surrogate unroll with
    straight-through spikes (functional.py:115-146).
    """

    @staticmethod
    def forward(ctx: Any, x, m0, decay, threshold, reset, slope, rule, sid):
        T, B, N = x.shape
        need = ctx.needs_input_grad[0] or ctx.needs_input_grad[1]
        m_final = torch.empty_like(m0)
        spikes = torch.empty_like(x)
        ckpt = torch.empty((_chunks(T), B, N), dtype=x.dtype, device=x.device) if need else None
        _lib.call(
            "myelin_lif_fwd_f32",
            _lib.ptr(x), _lib.ptr(m0), _lib.ptr(m_final), _lib.ptr(spikes), None, _lib.ptr(ckpt),
            T, B, N, decay, threshold, reset, slope, rule, BWD_CHUNK, _lib.stream(x.device),
        )
        ctx.set_materialize_grads(False)
        if sid == _lib.SG_NONE:
            ctx.mark_non_differentiable(spikes)
        if need:
            ctx.save_for_backward(x, ckpt)
        ctx.meta = (decay, threshold, reset, slope, sid)
        return m_final, spikes

    @staticmethod
    def backward(ctx: Any, g_m, g_s):
        none = (None,) * 8
        if (g_m is None and g_s is None) or not any(ctx.needs_input_grad[:2]):
            return none
        x, ckpt = ctx.saved_tensors
        decay, threshold, reset, slope, sid = ctx.meta
        T, B, N = x.shape
        g_m, g_s = _contig_f32(g_m), _contig_f32(g_s)
        gx = torch.empty_like(x)
        gm0 = torch.empty((B, N), dtype=x.dtype, device=x.device)
        with torch.cuda.device(x.device):
            _lib.call(
                "myelin_lif_bwd_f32",
                _lib.ptr(x), _lib.ptr(ckpt), _lib.ptr(g_s), _lib.ptr(g_m), _lib.ptr(gx), _lib.ptr(gm0),
                T, B * N, decay, threshold, reset, slope, sid, BWD_CHUNK, _lib.stream(x.device),
            )
        return (
            gx if ctx.needs_input_grad[0] else None,
            gm0 if ctx.needs_input_grad[1] else None,
            None, None, None, None, None, None,
        )


class HipALIFFunction(torch.autograd.Function):
    """Fused-time ALIF with the two-state (membrane, adaptation) adjoint.

    ``sid == SG_NONE`` is the plain ``alif_unroll`` (functional.py:48-78);
    otherwise ``surrogate_alif_unroll`` (functional.py:149-189), which the
    reference runs only through torch autograd (kernels.py:368-389).
    """

    @staticmethod
    def forward(ctx: Any, x, m0, a0, decay, rho, threshold, beta, reset, slope, rule, sid):
        T, B, N = x.shape
        need = any(ctx.needs_input_grad[:3])
        m_final = torch.empty_like(m0)
        a_final = torch.empty_like(a0)
        spikes = torch.empty_like(x)
        ckpt_m = ckpt_a = None
        if need:
            ckpt_m = torch.empty((_chunks(T), B, N), dtype=x.dtype, device=x.device)
            ckpt_a = torch.empty_like(ckpt_m)
        _lib.call(
            "myelin_alif_fwd_f32",
            _lib.ptr(x), _lib.ptr(m0), _lib.ptr(a0), _lib.ptr(m_final), _lib.ptr(a_final),
            _lib.ptr(spikes), None, _lib.ptr(ckpt_m), _lib.ptr(ckpt_a),
            T, B, N, decay, rho, threshold, beta, reset, slope, rule, BWD_CHUNK,
            _lib.stream(x.device),
        )
        ctx.set_materialize_grads(False)
        if sid == _lib.SG_NONE:
            ctx.mark_non_differentiable(spikes)
        if need:
            ctx.save_for_backward(x, ckpt_m, ckpt_a)
        ctx.meta = (decay, rho, threshold, beta, reset, slope, sid)
        return m_final, a_final, spikes

    @staticmethod
    def backward(ctx: Any, g_m, g_a, g_s):
        none = (None,) * 11
        if (g_m is None and g_a is None and g_s is None) or not any(ctx.needs_input_grad[:3]):
            return none
        x, ckpt_m, ckpt_a = ctx.saved_tensors
        decay, rho, threshold, beta, reset, slope, sid = ctx.meta
        T, B, N = x.shape
        g_m, g_a, g_s = _contig_f32(g_m), _contig_f32(g_a), _contig_f32(g_s)
        gx = torch.empty_like(x)
        gm0 = torch.empty((B, N), dtype=x.dtype, device=x.device)
        ga0 = torch.empty_like(gm0)
        with torch.cuda.device(x.device):
            _lib.call(
                "myelin_alif_bwd_f32",
                _lib.ptr(x), _lib.ptr(ckpt_m), _lib.ptr(ckpt_a), _lib.ptr(g_s), _lib.ptr(g_m),
                _lib.ptr(g_a), _lib.ptr(gx), _lib.ptr(gm0), _lib.ptr(ga0),
                T, B * N, decay, rho, threshold, beta, reset, slope, sid, BWD_CHUNK,
                _lib.stream(x.device),
            )
        return (
            gx if ctx.needs_input_grad[0] else None,
            gm0 if ctx.needs_input_grad[1] else None,
            ga0 if ctx.needs_input_grad[2] else None,
            None, None, None, None, None, None, None, None,
        )
