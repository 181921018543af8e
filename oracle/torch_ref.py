"""Op-by-op CPU restatement of myelin's ``torch`` backend (the oracle).

TEST INFRASTRUCTURE ONLY -- never imported by ``myelin_amd``.

Every function below restates one reference function; the citation in its
docstring is ``file:line`` inside djsaunde/myelin (``src/myelin/...``).  The
arithmetic is written with the same ATen ops in the same evaluation order as
the reference so that, on the CPU, forward results are bit-identical to what
myelin computes, and gradients are produced by ``torch.autograd`` exactly as
the reference's surrogate unrolls produce them.

How each function is pinned (checked against something other than itself;
see ``tests/test_oracle_*.py``):

* ``lif_unroll`` / ``alif_unroll`` -- the reference's own closed-form step
  vectors (``tests/test_lif_reference.py:15-27,72-113``, restated in
  ``tests/golden/reference_vectors.json``), a brute-force Python-float loop
  with fp32 rounding after every op, and bit equality with the independent C
  restatement ``oracle/c/oracle.c``.
* surrogate primitives / derivatives -- derivatives are checked against
  float64 ``torch.autograd`` of the primitives (an independent library
  routine) and against hand values at fixed points.
* ``surrogate_lif_unroll`` / ``surrogate_alif_unroll`` gradients -- against
  the closed-form adjoint in ``oracle/c/oracle.c`` (independently derived),
  float64 finite differences through the smooth (``hard_forward=False``)
  path, and golden vectors written from the reference itself
  (``tests/golden/make_golden.py``).
* ``surrogate_adjoint_autograd_order`` -- equal, value for value, to
  ``torch.autograd`` through the unrolls for every surrogate, LIF and ALIF,
  hard and smooth forward, with a nonzero reset and final-state gradients
  (``tests/test_oracle_adjoint.py``); three other summation orders of the
  spike gradient are shown to differ.
* packing -- ``numpy.packbits(bitorder="little")`` viewed as little-endian
  int32 (independent routine), the reference's vectors
  (``tests/test_packing.py:66-74,193-201``) and golden vectors.
* linear stream / checkpoint / rate functions -- invariance of every output
  and gradient to the checkpoint size (C=1, C=T, ragged C), the stream path
  against autograd through an explicit ``matmul`` + ``surrogate_lif_unroll``
  composition, ``rate == spikes.mean(0)`` (``tests/test_modules.py:892-936``),
  and golden vectors from the reference.
* ``linear_rate_adjoint_f64`` -- equal (to float64 rounding) to the
  checkpoint and rate Functions above run on float64 tensors, where those
  derive the same rasters themselves, with and without biases, for several
  surrogates; a raster or an injected gradient changed by one entry moves
  its result.
"""

from __future__ import annotations

import math
from collections.abc import Sequence

import torch

# ---------------------------------------------------------------------------
# parameters  (neurons.py:15-62)
# ---------------------------------------------------------------------------


def decay_from_tau(tau: float) -> float:
    """``LIFParams.decay`` / ``ALIFParams.adaptation_decay`` (neurons.py:22-28,56-62).

    Computed in Python double precision; ATen rounds it to fp32 when it
    multiplies an fp32 tensor.
    """

    if tau <= 0:
        raise ValueError("tau must be positive")
    return 1.0 - (1.0 / tau)


# ---------------------------------------------------------------------------
# surrogates  (surrogates.py:19-110)
# ---------------------------------------------------------------------------

SURROGATE_NAMES = ("sigmoid", "fast_sigmoid", "atan", "triangular", "superspike", "multi_gaussian")


def _ncdf(c: torch.Tensor, mean: float, sigma: float) -> torch.Tensor:
    # surrogates.py:64-65
    return 0.5 * (1.0 + torch.erf((c - mean) / (1.4142135623730951 * sigma)))


def surrogate_primitive(name: str, c: torch.Tensor) -> torch.Tensor:
    """Smooth primitive sigma(c) (surrogates.py:29-75)."""

    if name == "sigmoid":
        return torch.sigmoid(c)
    if name == "fast_sigmoid":
        return 0.5 * (c / (1.0 + c.abs()) + 1.0)
    if name == "atan":
        return torch.atan(torch.pi * c / 2.0) / torch.pi + 0.5
    if name == "triangular":
        return (1.0 - c.abs()).clamp(min=0.0, max=1.0)
    if name == "superspike":
        return c / (1.0 + c.abs()) + 0.5
    if name == "multi_gaussian":
        return 0.6 * _ncdf(c, 0.0, 0.5) + 0.2 * _ncdf(c, 1.0, 1.0) + 0.2 * _ncdf(c, -1.0, 1.0)
    raise ValueError(f"unknown surrogate {name!r}")


def surrogate_derivative(name: str, c: torch.Tensor) -> torch.Tensor:
    """Closed-form sigma'(c) (surrogates.py:78-102)."""

    if name == "sigmoid":
        v = torch.sigmoid(c)
        return v * (1.0 - v)
    if name == "fast_sigmoid":
        return 0.5 / (1.0 + c.abs()).square()
    if name == "atan":
        s = torch.pi * c / 2.0
        return 0.5 / (1.0 + s.square())
    if name == "triangular":
        return torch.where(c.abs() < 1.0, -c.sign(), torch.zeros_like(c))
    if name == "superspike":
        return 1.0 / (1.0 + c.abs()).square()
    if name == "multi_gaussian":
        k = 0.3989422804014327
        return (
            0.6 * (k / 0.5) * torch.exp(-0.5 * (c / 0.5).square())
            + 0.2 * k * torch.exp(-0.5 * (c - 1.0).square())
            + 0.2 * k * torch.exp(-0.5 * (c + 1.0).square())
        )
    raise ValueError(f"unknown surrogate {name!r}")


def hard_spike(name: str, c: torch.Tensor) -> torch.Tensor:
    """Straight-through spike ``H(c) + sigma(c) - sigma(c).detach()`` (surrogates.py:105-110).

    Note the fp32 value is ``(H + sigma) - sigma``, which is 0.99999994 rather
    than 1.0 for a fraction of spikes; the reference carries that value into
    the reset and adaptation updates.
    """

    h = (c >= 0).to(c.dtype)
    smooth = surrogate_primitive(name, c)
    return h + smooth - smooth.detach()


# ---------------------------------------------------------------------------
# unrolls  (neurons.py:106-128, functional.py:21-78,115-189)
# ---------------------------------------------------------------------------


def _check_tbn(inputs: torch.Tensor, *states: torch.Tensor) -> None:
    if inputs.ndim != 3:
        raise ValueError(f"inputs must be shaped [T, B, N]; got {tuple(inputs.shape)}")
    for s in states:
        if s.shape != inputs.shape[1:]:
            raise ValueError("initial state must match inputs.shape[1:]")


def lif_unroll(
    inputs: torch.Tensor, m0: torch.Tensor, tau: float, threshold: float, reset: float
) -> tuple[torch.Tensor, torch.Tensor]:
    """Hard-reset LIF over ``[T,B,N]`` (functional.py:21-45 via neurons.py:106-114)."""

    _check_tbn(inputs, m0)
    d = decay_from_tau(tau)
    m = m0
    out = []
    for x in inputs.unbind(0):
        m = m * d + x
        s = m >= threshold
        m = torch.where(s, reset, m)
        out.append(s.to(x.dtype))
    return m, torch.stack(out, 0)


def alif_unroll(
    inputs: torch.Tensor,
    m0: torch.Tensor,
    a0: torch.Tensor,
    tau_mem: float,
    tau_adaptation: float,
    threshold: float,
    reset: float,
    beta: float,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Adaptive LIF (functional.py:48-78 via neurons.py:117-128)."""

    _check_tbn(inputs, m0, a0)
    d = decay_from_tau(tau_mem)
    rho = decay_from_tau(tau_adaptation)
    m, a = m0, a0
    out = []
    for x in inputs.unbind(0):
        m = m * d + x
        th = threshold + beta * a
        s = m >= th
        sf = s.to(x.dtype)
        m = torch.where(s, reset, m)
        a = a * rho + sf
        out.append(sf)
    return m, a, torch.stack(out, 0)


def surrogate_lif_unroll(
    inputs: torch.Tensor,
    m0: torch.Tensor,
    tau: float,
    threshold: float,
    reset: float,
    surrogate: str,
    slope: float = 10.0,
    hard_forward: bool = True,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Surrogate-gradient LIF, differentiable by autograd (functional.py:115-146)."""

    _check_tbn(inputs, m0)
    d = decay_from_tau(tau)
    m = m0
    out = []
    for x in inputs.unbind(0):
        m = m * d + x
        c = slope * (m - threshold)
        s = hard_spike(surrogate, c) if hard_forward else surrogate_primitive(surrogate, c)
        m = m * (1.0 - s) + reset * s
        out.append(s)
    return m, torch.stack(out, 0)


def surrogate_alif_unroll(
    inputs: torch.Tensor,
    m0: torch.Tensor,
    a0: torch.Tensor,
    tau_mem: float,
    tau_adaptation: float,
    threshold: float,
    reset: float,
    beta: float,
    surrogate: str,
    slope: float = 10.0,
    hard_forward: bool = True,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Surrogate-gradient ALIF, differentiable by autograd (functional.py:149-189)."""

    _check_tbn(inputs, m0, a0)
    d = decay_from_tau(tau_mem)
    rho = decay_from_tau(tau_adaptation)
    m, a = m0, a0
    out = []
    for x in inputs.unbind(0):
        m = m * d + x
        th = threshold + beta * a
        c = slope * (m - th)
        s = hard_spike(surrogate, c) if hard_forward else surrogate_primitive(surrogate, c)
        m = m * (1.0 - s) + reset * s
        a = a * rho + s
        out.append(s)
    return m, a, torch.stack(out, 0)


# ---------------------------------------------------------------------------
# the adjoint of the surrogate unrolls in autograd's operation order
# ---------------------------------------------------------------------------


def _primitive_grad_autograd(name: str, c: torch.Tensor, g: torch.Tensor) -> torch.Tensor:
    """dL/dc for dL/dsigma = g through the primitive of surrogates.py:29-75,
    op by op as torch autograd differentiates it (each node's derivative
    formula, from the output back; two uses of c summed)."""

    if name in ("fast_sigmoid", "superspike"):
        b = 1.0 + c.abs()
        gq = g * 0.5 if name == "fast_sigmoid" else g
        return gq / b + (-gq * ((c / b) / b)) * c.sign()  # div: numerator + (denominator via abs)
    if name == "sigmoid":
        y = torch.sigmoid(c)
        return g * (1.0 - y) * y  # sigmoid_backward(grad, result)
    if name == "atan":
        p = torch.pi * c / 2.0
        return (g / torch.pi) / (p * p + 1.0) / 2.0 * torch.pi  # (/pi) atan (/2) (pi*)
    if name == "triangular":
        r = 1.0 - c.abs()
        return -(g * ((r >= 0.0) & (r <= 1.0)).to(g.dtype)) * c.sign()  # clamp mask, rsub, abs
    if name == "multi_gaussian":
        parts = []
        for w, mean, sigma in ((0.6, 0.0, 0.5), (0.2, 1.0, 1.0), (0.2, -1.0, 1.0)):
            k = 1.4142135623730951 * sigma
            z = (c - mean) / k
            parts.append(2.0 / math.sqrt(math.pi) * torch.exp(-(z.pow(2))) * (g * w * 0.5) / k)
        return (parts[1] + parts[2]) + parts[0]  # the last-built branches reach c first
    raise ValueError(f"unknown surrogate {name!r}")


def surrogate_adjoint_autograd_order(inputs, m0, a0, grad_spikes, grad_m, grad_a, tau_mem, tau_adaptation,
                                     threshold, reset, beta, surrogate, slope=10.0, hard_forward=True, alif=True):
    """Gradients of ``surrogate_alif_unroll`` / ``surrogate_lif_unroll``
    (functional.py:115-189) computed without autograd, in the operation
    order and fp32 rounding that torch autograd uses for them.

    Per step, reverse time, with G = dL/dm_{t+1}, A = dL/da_{t+1}:
      dL/ds = ((gs_t + A) + G*reset) - G*m'   (the stack, adaptation, reset
              and m'*(1 - s) nodes deliver their gradients in that order)
      gd    = primitive_grad(c, dL/ds) * slope
      gp    = G*(1 - s) + gd  -> dL/dx_t ;  A <- A*rho + (-gd)*beta ;
      G     <- gp*decay
    This is the order the HIP kernels' autograd-order mode evaluates.
    Returns (grad_x, grad_m0, grad_a0 or None).
    """

    d = decay_from_tau(tau_mem)
    rho = decay_from_tau(tau_adaptation) if alif else 0.0
    m, a = m0, a0
    trace = []
    for x in inputs.unbind(0):
        mp = m * d + x
        th = threshold + beta * a if alif else threshold
        c = slope * (mp - th)
        sm = surrogate_primitive(surrogate, c)
        s = ((c >= 0).to(c.dtype) + sm) - sm if hard_forward else sm
        trace.append((mp, c, s))
        m = mp * (1.0 - s) + reset * s
        if alif:
            a = a * rho + s
    G = torch.zeros_like(m0) if grad_m is None else grad_m
    A = torch.zeros_like(m0) if (grad_a is None or not alif) else grad_a
    gx = torch.empty_like(inputs)
    for t in range(inputs.shape[0] - 1, -1, -1):
        mp, c, s = trace[t]
        gs = grad_spikes[t] if grad_spikes is not None else torch.zeros_like(mp)
        g_s = ((gs + A) + G * reset) - G * mp
        gd = _primitive_grad_autograd(surrogate, c, g_s) * slope
        gp = G * (1.0 - s) + gd
        gx[t] = gp
        if alif:
            A = A * rho + (-gd) * beta
        G = gp * d
    return gx, G, (A if alif else None)


# ---------------------------------------------------------------------------
# checkpoint policy  (checkpointing.py:13-60)
# ---------------------------------------------------------------------------


def recommended_checkpoint_size(timesteps: int, policy: str = "balanced") -> int:
    """checkpointing.py:13-33."""

    if timesteps <= 0:
        raise ValueError("timesteps must be positive")
    if policy == "memory":
        c = math.ceil(math.sqrt(timesteps))
    elif policy == "balanced":
        c = math.ceil(timesteps / 4)
    elif policy == "speed":
        c = math.ceil(timesteps / 2)
    else:
        raise ValueError("policy must be 'memory', 'balanced', or 'speed'")
    return max(1, min(timesteps, c))


def resolve_checkpoint_size(timesteps: int, checkpoint_size: int | str) -> int:
    """checkpointing.py:36-43."""

    if isinstance(checkpoint_size, int):
        if checkpoint_size <= 0:
            raise ValueError("checkpoint_size must be positive")
        return min(checkpoint_size, timesteps)
    return recommended_checkpoint_size(timesteps, checkpoint_size)


# ---------------------------------------------------------------------------
# packing  (packing.py:14-162,165-273)
# ---------------------------------------------------------------------------

BITS = 32


def packed_words(n: int) -> int:
    """packing.py:36-42."""

    if n < 0:
        raise ValueError("size must be non-negative")
    return (n + BITS - 1) // BITS


def pack_spikes(spikes: torch.Tensor) -> tuple[torch.Tensor, tuple[int, ...]]:
    """Nonzero -> bit, LSB-first along the last dim, int32 words (packing.py:45-71)."""

    if spikes.ndim == 0:
        raise ValueError("spikes must have at least one dimension")
    n = spikes.shape[-1]
    if n == 0:
        raise ValueError("cannot pack an empty last dimension")
    w = packed_words(n)
    bits = (spikes != 0).to(torch.int64)
    pad = w * BITS - n
    if pad:
        bits = torch.cat((bits, bits.new_zeros((*spikes.shape[:-1], pad))), dim=-1)
    bits = bits.reshape(*spikes.shape[:-1], w, BITS)
    weights = torch.ones(BITS, dtype=torch.int64) << torch.arange(BITS, dtype=torch.int64)
    return (bits * weights).sum(-1).to(torch.int32), tuple(spikes.shape)


def _check_packed(data: torch.Tensor, shape: tuple[int, ...]) -> None:
    # packing.py:236-252
    if data.dtype != torch.int32:
        raise ValueError("packed.data must have dtype torch.int32")
    if len(shape) == 0:
        raise ValueError("packed.original_shape must have at least one dimension")
    if shape[-1] <= 0:
        raise ValueError("packed.original_shape must have non-empty last dimension")
    if tuple(data.shape) != (*shape[:-1], packed_words(shape[-1])):
        raise ValueError("packed.data shape does not match packed.original_shape")


def unpack_spikes(
    data: torch.Tensor, shape: tuple[int, ...], dtype: torch.dtype = torch.float32
) -> torch.Tensor:
    """packing.py:74-81."""

    _check_packed(data, shape)
    shifts = torch.arange(BITS, dtype=torch.int64)
    bits = ((data.to(torch.int64).unsqueeze(-1) >> shifts) & 1).to(dtype)
    return bits.reshape(*shape[:-1], -1)[..., : shape[-1]]


def _norm_dims(dim: int | Sequence[int], ndim: int) -> tuple[int, ...]:
    # packing.py:223-233
    raw = (dim,) if isinstance(dim, int) else tuple(dim)
    out: list[int] = []
    for d in raw:
        a = d + ndim if d < 0 else d
        if a < 0 or a >= ndim:
            raise IndexError(f"dimension out of range: {d}")
        if a in out:
            raise ValueError(f"duplicate reduction dimension: {d}")
        out.append(a)
    return tuple(out)


def _row_counts(data: torch.Tensor, shape: tuple[int, ...]) -> torch.Tensor:
    """Per-row popcount with padding bits masked (packing.py:164-205)."""

    _check_packed(data, shape)
    words = data.to(torch.int64) & 0xFFFFFFFF
    rem = shape[-1] % BITS
    if rem:
        mask = torch.full((words.shape[-1],), 0xFFFFFFFF, dtype=torch.int64)
        mask[-1] = (1 << rem) - 1
        words = words & mask
    shifts = torch.arange(BITS, dtype=torch.int64)
    return ((words.unsqueeze(-1) >> shifts) & 1).sum(dim=(-1, -2), dtype=torch.int64)


def packed_spike_counts(
    data: torch.Tensor, shape: tuple[int, ...], dim: int | Sequence[int] | None = -1
) -> torch.Tensor:
    """Counts over dims that include the last one (packing.py:110-142)."""

    rows = _row_counts(data, shape)
    if dim is None:
        return rows.sum()
    dims = _norm_dims(dim, len(shape))
    last = len(shape) - 1
    if last not in dims:
        raise ValueError(
            "packed_spike_counts requires reducing the packed/original last dimension; "
            "use packed_spike_count for dense-like reductions that keep that dimension"
        )
    rest = tuple(d for d in dims if d != last)
    return rows if not rest else rows.sum(dim=rest)


def packed_spike_count(
    data: torch.Tensor, shape: tuple[int, ...], dim: int | Sequence[int] | None = None
) -> torch.Tensor:
    """Dense-like count reductions (packing.py:84-107,209-216)."""

    if dim is None:
        return packed_spike_counts(data, shape, None)
    dims = _norm_dims(dim, len(shape))
    last = len(shape) - 1
    if last in dims:
        return packed_spike_counts(data, shape, dims)
    if dims == tuple(range(last)):
        # every leading dim reduced: per-neuron counts from the bits
        _check_packed(data, shape)
        shifts = torch.arange(BITS, dtype=torch.int64)
        bits = ((data.to(torch.int64) & 0xFFFFFFFF).unsqueeze(-1) >> shifts) & 1
        lead = tuple(range(last))
        per = bits.sum(dim=lead, dtype=torch.int64) if lead else bits.to(torch.int64)
        return per.reshape(-1)[: shape[-1]]
    dense = unpack_spikes(data, shape, torch.float32)
    return dense.sum(dim=dims).to(torch.int64)


def packed_spike_rate(
    data: torch.Tensor,
    shape: tuple[int, ...],
    dim: int | Sequence[int] | None = None,
    dtype: torch.dtype = torch.float32,
) -> torch.Tensor:
    """``count.to(dtype) / prod(reduced sizes)`` (packing.py:145-162)."""

    counts = packed_spike_count(data, shape, dim)
    dims = tuple(range(len(shape))) if dim is None else _norm_dims(dim, len(shape))
    denom = 1
    for d in dims:
        denom *= shape[d]
    return counts.to(dtype) / denom


# ---------------------------------------------------------------------------
# streamed synapse + surrogate LIF  (autograd.py:445-923)
# ---------------------------------------------------------------------------

# How the linear Functions below round their matmuls.  "native" is the
# reference's own torch.matmul in fp32.  "exact" multiplies in float64 and
# rounds each result once to fp32: an equally valid fp32 evaluation, used by
# the tests only to measure how far a case's outputs move under a different
# (here: the most accurate) fp32 matmul rounding -- its conditioning.
_MATMUL_MODE = "native"


def set_matmul_rounding(mode: str) -> str:
    """Select "native" or "exact" matmul rounding; returns the previous mode."""

    global _MATMUL_MODE
    if mode not in ("native", "exact"):
        raise ValueError("mode must be 'native' or 'exact'")
    prev, _MATMUL_MODE = _MATMUL_MODE, mode
    return prev


def _matmul(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    if _MATMUL_MODE == "native":
        return torch.matmul(a, b)
    return torch.matmul(a.double(), b.double()).to(a.dtype)



class _StreamFn(torch.autograd.Function):
    """Restates ``LinearSurrogateLIFStreamFunction`` (autograd.py:445-558)."""

    @staticmethod
    def forward(ctx, x, w, b, tau, threshold, reset, surrogate, slope):
        ctx.set_materialize_grads(False)
        d = decay_from_tau(tau)
        m = torch.zeros((x.shape[1], w.shape[1]), dtype=x.dtype)
        pres, spikes = [], []
        for xt in x.unbind(0):
            cur = _matmul(xt, w)
            if b is not None:
                cur = cur + b
            m = m * d + cur
            smooth = surrogate_primitive(surrogate, slope * (m - threshold))
            s = (m >= threshold).to(x.dtype) + smooth - smooth.detach()
            pres.append(m)
            spikes.append(s)
            m = m * (1.0 - s) + reset * s
        ctx.meta = (tau, threshold, reset, surrogate, slope, b is not None)
        ctx.save_for_backward(x, w, torch.stack(pres), torch.stack(spikes))
        return m, torch.stack(spikes)

    @staticmethod
    def backward(ctx, g_final, g_spikes):
        if g_final is None and g_spikes is None:
            return (None,) * 8
        x, w, pres, spikes = ctx.saved_tensors
        tau, threshold, reset, surrogate, slope, has_b = ctx.meta
        d_m = decay_from_tau(tau)
        need_x, need_w, need_b = ctx.needs_input_grad[:3]
        gm = torch.zeros_like(pres[0]) if g_final is None else g_final
        gx = torch.empty_like(x) if need_x else None
        gw = torch.zeros_like(w) if need_w else None
        gb = torch.zeros((w.shape[1],), dtype=x.dtype) if (need_b and has_b) else None
        for t in range(x.shape[0] - 1, -1, -1):
            pre, s = pres[t], spikes[t]
            d = slope * surrogate_derivative(surrogate, slope * (pre - threshold))
            gp = gm * ((1.0 - s) + (reset - pre) * d)
            if g_spikes is not None:
                gp = gp + g_spikes[t] * d
            if gx is not None:
                gx[t] = _matmul(gp, w.t())
            if gw is not None:
                gw = gw + _matmul(x[t].t(), gp)
            if gb is not None:
                gb = gb + gp.sum(dim=0)
            gm = gp * d_m
        return gx, gw, gb, None, None, None, None, None


def _recompute_chunk(x, w, b, m, t0, t1, d, threshold, reset):
    pres, spikes = [], []
    for t in range(t0, t1):
        cur = _matmul(x[t], w)
        if b is not None:
            cur = cur + b
        m = m * d + cur
        s = (m >= threshold).to(x.dtype)
        pres.append(m)
        spikes.append(s)
        m = m * (1.0 - s) + reset * s
    return pres, spikes


class _CheckpointFn(torch.autograd.Function):
    """Restates ``LinearSurrogateLIFCheckpointFunction`` (autograd.py:588-717) and,
    with ``rate=True``, ``LinearSurrogateLIFCheckpointRateFunction``
    (autograd.py:753-885)."""

    @staticmethod
    def forward(ctx, x, w, b, tau, threshold, reset, surrogate, slope, chunk, rate):
        ctx.set_materialize_grads(False)
        d = decay_from_tau(tau)
        m = torch.zeros((x.shape[1], w.shape[1]), dtype=x.dtype)
        counts = torch.zeros_like(m) if rate else None
        starts, spikes = [], []
        for t, xt in enumerate(x.unbind(0)):
            if t % chunk == 0:
                starts.append(m)
            cur = _matmul(xt, w)
            if b is not None:
                cur = cur + b
            m = m * d + cur
            s = (m >= threshold).to(x.dtype)
            if rate:
                counts = counts + s
            else:
                spikes.append(s)
            m = m * (1.0 - s) + reset * s
        ctx.meta = (tau, threshold, reset, surrogate, slope, chunk, rate)
        bias = torch.empty(0, dtype=x.dtype) if b is None else b
        ctx.has_b = b is not None
        ctx.save_for_backward(x, w, bias, torch.stack(starts))
        if rate:
            return m, counts / x.shape[0]
        return m, torch.stack(spikes)

    @staticmethod
    def backward(ctx, g_final, g_out):
        if g_final is None and g_out is None:
            return (None,) * 10
        x, w, bias, starts = ctx.saved_tensors
        b = bias if ctx.has_b else None
        tau, threshold, reset, surrogate, slope, chunk, rate = ctx.meta
        d_m = decay_from_tau(tau)
        T = x.shape[0]
        need_x, need_w, need_b = ctx.needs_input_grad[:3]
        gm = torch.zeros((x.shape[1], w.shape[1]), dtype=x.dtype) if g_final is None else g_final
        gx = torch.empty_like(x) if need_x else None
        gw = torch.zeros_like(w) if need_w else None
        gb = torch.zeros((w.shape[1],), dtype=x.dtype) if (need_b and ctx.has_b) else None
        g_step = None
        if rate and g_out is not None:
            g_step = g_out / T
        for k in range(starts.shape[0] - 1, -1, -1):
            t0 = k * chunk
            t1 = min(t0 + chunk, T)
            pres, spikes = _recompute_chunk(x, w, b, starts[k], t0, t1, d_m, threshold, reset)
            for j in range(t1 - t0 - 1, -1, -1):
                t = t0 + j
                pre, s = pres[j], spikes[j]
                d = slope * surrogate_derivative(surrogate, slope * (pre - threshold))
                gp = gm * ((1.0 - s) + (reset - pre) * d)
                if rate:
                    if g_step is not None:
                        gp = gp + g_step * d
                elif g_out is not None:
                    gp = gp + g_out[t] * d
                if gx is not None:
                    gx[t] = _matmul(gp, w.t())
                if gw is not None:
                    gw = gw + _matmul(x[t].t(), gp)
                if gb is not None:
                    gb = gb + gp.sum(dim=0)
                gm = gp * d_m
        return gx, gw, gb, None, None, None, None, None, None, None


def linear_surrogate_lif_stream(x, w, b, tau, threshold, reset, surrogate="atan", slope=10.0):
    """``linear_surrogate_lif_stream_function`` (autograd.py:561-585)."""

    return _StreamFn.apply(x, w, b, tau, threshold, reset, surrogate, slope)


def linear_surrogate_lif_checkpoint(
    x, w, b, tau, threshold, reset, surrogate="atan", slope=10.0, checkpoint_size=25
):
    """``linear_surrogate_lif_checkpoint_function`` (autograd.py:720-750)."""

    if checkpoint_size <= 0:
        raise ValueError("checkpoint_size must be positive")
    return _CheckpointFn.apply(
        x, w, b, tau, threshold, reset, surrogate, slope, checkpoint_size, False
    )


def linear_surrogate_lif_rate(
    x,
    w,
    b,
    tau,
    threshold,
    reset,
    surrogate="atan",
    slope=10.0,
    checkpoint_size=25,
    reduction="mean",
):
    """``linear_surrogate_lif_checkpoint_rate_function`` (autograd.py:888-923)."""

    if checkpoint_size <= 0:
        raise ValueError("checkpoint_size must be positive")
    if reduction not in ("mean", "none"):
        raise ValueError("reduction must be 'mean' or 'none'")
    m, rates = _CheckpointFn.apply(
        x, w, b, tau, threshold, reset, surrogate, slope, checkpoint_size, True
    )
    return m, (rates.mean() if reduction == "mean" else rates)


def linear_rate_adjoint_f64(x, wh, bh, wo, bo, decay, threshold, reset, surrogate, slope, hidden_spikes,
                            readout_spikes, grad_rates):
    """Float64 gradients of a checkpointed hidden layer feeding a rate readout,
    on a float64 forward whose spikes are the given rasters.

    The backward is that of ``LinearSurrogateLIFCheckpointFunction``
    (autograd.py:629-666: ``gp = gm((1 - s) + (r - m')d) + g_out_t d``,
    ``gx_t = gp W^T``, ``dW += x_t^T gp``, ``db += sum gp``, ``gm = gp decay``)
    and of the rate Function (autograd.py:842-875: the injected gradient is
    ``g_rates / T`` every step), with the readout's input gradient fed to the
    hidden layer as its ``g_out``.  Every value is a float64 tensor and every
    product is formed in float64; ``decay`` is passed in (pass the fp32 value
    an fp32 forward multiplies by, ``float(numpy.float32(d))``, to measure an
    fp32 evaluation against it).  The spikes are not re-derived from the
    float64 membranes: they are the fp32 run's own rasters, so this is the
    exact gradient of the network on that run's spike pattern, which every
    fp32 evaluation of it approximates.

    x ``[T, B, F]``, wh ``[F, H]``, wo ``[H, O]``, biases or None, rasters
    ``[T, B, H]`` / ``[T, B, O]`` (``readout_spikes`` None: the readout's
    spikes follow from its float64 membranes), grad_rates ``[B, O]``.
    Returns a dict of float64 tensors: gx, gwh, gbh, gwo, gbo, g_hidden (the
    readout's gradient into the hidden spikes), pre_hidden (the hidden
    layer's pre-reset membranes) and readout_spikes.
    """

    f64 = torch.float64
    T, B = x.shape[:2]
    xd = x.to(f64)
    sh = hidden_spikes.to(f64)

    def membranes(inp, w, b, s):
        """Pre-reset membranes; with s None the spikes are derived from them
        (m' >= threshold) and returned too."""

        cur = (inp.reshape(T * B, -1) @ w.to(f64)).reshape(T, B, -1)
        if b is not None:
            cur = cur + b.to(f64)
        m = torch.zeros(B, w.shape[1], dtype=f64)
        pres = torch.empty(T, B, w.shape[1], dtype=f64)
        derive = s is None
        if derive:
            s = torch.empty_like(pres)
        for t in range(T):
            m = m * decay + cur[t]
            pres[t] = m
            if derive:
                s[t] = (m >= threshold).to(f64)
            m = m * (1.0 - s[t]) + reset * s[t]
        return pres, s

    def reverse(pres, s, g_in, g_step):
        gm = torch.zeros_like(pres[0])
        gps = torch.empty_like(pres)
        for t in range(T - 1, -1, -1):
            pre = pres[t]
            d = slope * surrogate_derivative(surrogate, slope * (pre - threshold))
            gp = gm * ((1.0 - s[t]) + (reset - pre) * d)
            gp = gp + (g_step if g_in is None else g_in[t]) * d
            gps[t] = gp
            gm = gp * decay
        return gps.reshape(T * B, -1)

    pres_o, so = membranes(sh, wo, bo, None if readout_spikes is None else readout_spikes.to(f64))
    gp_o = reverse(pres_o, so, None, grad_rates.to(f64) / T)
    g_hidden = (gp_o @ wo.to(f64).t()).reshape(T, B, -1)
    pres_h, _ = membranes(xd, wh, bh, sh)
    gp_h = reverse(pres_h, sh, g_hidden, None)
    return {
        "pre_hidden": pres_h,
        "readout_spikes": so,
        "gx": (gp_h @ wh.to(f64).t()).reshape(x.shape),
        "g_hidden": g_hidden,
        "gwh": xd.reshape(T * B, -1).t() @ gp_h,
        "gbh": gp_h.sum(0) if bh is not None else None,
        "gwo": sh.reshape(T * B, -1).t() @ gp_o,
        "gbo": gp_o.sum(0) if bo is not None else None,
    }


def two_layer_rate(x, wh, bh, wo, bo, tau, threshold, reset, surrogate="fast_sigmoid", slope=5.0,
                   checkpoint_size=25):
    """``two_layer_surrogate_lif_rate_recompute_function`` (autograd.py:926-1126):
    the hidden checkpoint function feeding the readout checkpoint-rate function
    with ``reduction="none"``; the reference's backward replays exactly this
    composition under autograd, so the gradient is its autograd gradient."""

    if checkpoint_size <= 0:
        raise ValueError("checkpoint_size must be positive")
    _m, hidden = _CheckpointFn.apply(x, wh, bh, tau, threshold, reset, surrogate, slope, checkpoint_size, False)
    _m, rates = _CheckpointFn.apply(hidden, wo, bo, tau, threshold, reset, surrogate, slope, checkpoint_size, True)
    return rates
