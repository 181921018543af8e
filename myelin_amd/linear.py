"""Autograd boundary of the streamed-synapse LIF path (``x_t @ W`` fused ahead
of the neuron update).

Forward: one launch of ``myelin_linear_lif_fwd`` computes every step's
current tile on MFMA and runs the recurrence in the same workgroup (layers
narrower than 64 neurons use a split-K GEMM plus the recurrence kernel, see
``_lif_fwd``).

Saved state:
* ``checkpoint_size=None`` (the reference's stream Function,
  autograd.py:445-558): the pre-reset membranes ``[T, B, N]`` -- one tensor
  where the reference keeps pre-reset membranes and spikes;
* ``checkpoint_size=C`` (autograd.py:588-717) and the rate readout
  (autograd.py:753-885): chunk-start membranes every C steps only, except
  for layers of at most 32 neurons (readouts), which keep the whole trace
  as the stream path does (a few MB; their backward then recomputes
  nothing).

Backward, per span of whole chunks in reverse time: recompute the span's
pre-reset trace from its first chunk-start membrane (skipped when the trace
is saved), reverse recurrence -> G = dL/dI plus per-(b, n) bias partials,
then ``dX[t] = G_t @ W^T`` and ``dW += X_t^T G_t`` on MFMA GEMMs,
``db = sum_b`` of the bias partials.  Every reduction has a fixed order, so
gradients are run-to-run deterministic (the reference's Triton path uses
fp32 atomics, triton/lif.py:1336-1348).
"""

from __future__ import annotations

import contextlib
import math
from typing import Any

import torch

from myelin_amd import _lib


def _workspace(M, N, K, prec, device, split, ws):
    """(split-K workspace, its size in floats): ``ws``, a float32 buffer the
    caller has free on the stream (the kernel then splits K no more ways
    than it holds), else a new one of the size the kernel would use."""

    if not split:
        return None, 0
    if ws is not None:
        return ws, ws.numel()
    n_ws = _lib.load().myelin_gemm_workspace_elems(M, N, K, prec)
    return (torch.empty(n_ws, dtype=torch.float32, device=device) if n_ws > 0 else None), n_ws


def _gemm(A, B, C, M, N, K, lda, ldb, ldc, trans_a, trans_b, accumulate, prec, stream, bias=None, a_bits=False,
          split=True, ws=None, col_sum=None):
    """C (+)= op(A) op(B) (+ bias); A and B both float32 or both bfloat16, or
    (``a_bits``) A packed spike words (int32, lda in words) with B float32.
    ``split=False`` gives no workspace, so K is never split: every element is
    then one k-ordered sum that does not depend on M (the synapse currents,
    which a checkpointed backward recomputes over fewer rows and must
    reproduce bit for bit).  ``ws``: see _workspace.  ``col_sum`` = (src
    [R, Nc], dst [Nc]): also dst = src summed over rows, in the GEMM's
    split-K reduce launch when it has one (myelin_gemm_col_sum)."""

    ws, n_ws = _workspace(M, N, K, prec, C.device, split, ws)
    a_dt = _lib.DT_BITS if a_bits else _lib.DT[A.dtype]
    args = (_lib.ptr(A), a_dt, _lib.ptr(B), _lib.DT[B.dtype], _lib.ptr(bias), _lib.ptr(C), M, N, K, lda, ldb, ldc,
            int(trans_a), int(trans_b), int(accumulate), prec, _lib.ptr(ws), n_ws)
    if col_sum is None:
        _lib.call("myelin_gemm", *args, stream)
    else:
        src, dst = col_sum
        _lib.call("myelin_gemm_col_sum", *args, _lib.ptr(src), _lib.ptr(dst), src.numel() // dst.numel(),
                  dst.numel(), stream)


def _half(prec: int, F: int, N: int) -> bool:
    """bf16 synapse with operand rows the bf16 kernels can load 16 bytes at a
    time: its GEMMs then read bf16 copies of x, W and dL/dI (half the
    bytes, bit-identical results)."""

    return prec == _lib.PREC["bf16"] and F % 8 == 0 and N % 8 == 0


def _cast_bf16(t, stream):
    out = torch.empty(t.shape, dtype=torch.bfloat16, device=t.device)
    _lib.call("myelin_cast_bf16", _lib.ptr(t), _lib.ptr(out), t.numel(), stream)
    return out


def _transpose_bf16(w, stream):
    """[F, N] fp32 -> [N, F] bf16."""

    out = torch.empty((w.shape[1], w.shape[0]), dtype=torch.bfloat16, device=w.device)
    _lib.call("myelin_transpose_bf16", _lib.ptr(w), _lib.ptr(out), w.shape[0], w.shape[1], stream)
    return out


def _cast_transpose_bf16(x, w, stream):
    """(bf16 copy of x, [N, F] bf16 transpose of w [F, N]) in one launch."""

    xb = torch.empty(x.shape, dtype=torch.bfloat16, device=x.device)
    wt = torch.empty((w.shape[1], w.shape[0]), dtype=torch.bfloat16, device=w.device)
    _lib.call("myelin_cast_transpose_bf16", _lib.ptr(x), _lib.ptr(xb), x.numel(), _lib.ptr(w), _lib.ptr(wt),
              w.shape[0], w.shape[1], stream)
    return xb, wt


def _gemm_parts(A, B, parts, b_part, C, M, N, K, lda, ldb, ldc, trans_a, trans_b, accumulate, stream, bias=None,
                split=True, ws=None, col_sum=None):
    """C (+)= sum_p op(A) op(B_p) (+ bias), bf16 operands, B_p = B + p*b_part
    (elements); ``split``, ``ws`` and ``col_sum`` as in _gemm."""

    ws, n_ws = _workspace(M, N, K, _lib.PREC["bf16"], C.device, split, ws)
    args = (_lib.ptr(A), _lib.ptr(B), parts, b_part, _lib.ptr(bias), _lib.ptr(C), M, N, K, lda, ldb, ldc,
            int(trans_a), int(trans_b), int(accumulate), _lib.ptr(ws), n_ws)
    if col_sum is None:
        _lib.call("myelin_gemm_parts", *args, stream)
    else:
        src, dst = col_sum
        _lib.call("myelin_gemm_parts_col_sum", *args, _lib.ptr(src), _lib.ptr(dst), src.numel() // dst.numel(),
                  dst.numel(), stream)


# exact bf16 split of an fp32 synapse: tried for products of at least this
# many multiply-adds (the input check costs one host synchronisation)
_SPLIT_MIN_MACS = 1 << 32


class _LazyBf16:
    """A bf16 view of an fp32 input ``[T, ...]`` that keeps no whole bf16
    copy: indexing it with a slice of steps launches the cast of those steps
    on the current stream and returns a new bf16 tensor.  Used by the
    memory-lean policy (``checkpoint_size="memory"``), whose GEMMs then read
    one checkpoint chunk or span of bf16 input at a time."""

    dtype = torch.bfloat16

    def __init__(self, x: torch.Tensor):
        self.x = x
        self.shape = x.shape
        self.device = x.device
        self._last = (None, None)

    def __getitem__(self, steps: slice) -> torch.Tensor:
        # the last slice is kept: a backward span's recompute and its weight
        # gradient read the same steps, one after the other on one stream
        key = (steps.start, steps.stop, steps.step)
        if self._last[0] != key:
            part = self.x[steps]
            self._last = (key, _cast_bf16(part, _lib.stream(part.device)))
        return self._last[1]


class _Split:
    """The fp32 synapse on the bf16 MFMA, exactly: when every input value is
    a bf16 value (spikes, small integers), ``x @ W = x @ W_hi + x @ W_mid +
    x @ W_lo`` with the three bf16 planes of W summing exactly to W, so every
    product is exact and only the fp32 summation rounds -- at the bf16
    engine's rate (about 5x the fp32 one per pass).

    Construction launches the checked bf16 copy of x (``xb``; with ``lean``
    only the check, ``xb`` then a _LazyBf16 view), the split of W into
    transposed planes ``w3 [3, N, F]`` and an asynchronous copy of the
    check's flag to pinned host memory, without waiting.  ``exact()``
    waits for the flag alone (not for later work on the stream) and caches
    the answer; when it is False the fp32 GEMMs must run instead."""

    def __init__(self, x, w, stream, lean=False):
        flag = torch.zeros(1, dtype=torch.int32, device=x.device)
        if lean:
            # no whole bf16 copy: check x slice by slice into one scratch
            # buffer (the flag is only ever set), and cast per chunk later
            self.xb = _LazyBf16(x)
            step = max(1, (1 << 22) // max(1, x[0].numel()))
            scratch = torch.empty((min(step, x.shape[0]), *x.shape[1:]), dtype=torch.bfloat16, device=x.device)
            for t0 in range(0, x.shape[0], step):
                part = x[t0:t0 + step]
                _lib.call("myelin_cast_bf16_checked", _lib.ptr(part), _lib.ptr(scratch), part.numel(), _lib.ptr(flag),
                          stream)
        else:
            self.xb = torch.empty(x.shape, dtype=torch.bfloat16, device=x.device)
            _lib.call("myelin_cast_bf16_checked", _lib.ptr(x), _lib.ptr(self.xb), x.numel(), _lib.ptr(flag), stream)
        self._host = torch.empty(1, dtype=torch.int32, pin_memory=True)
        self._host.copy_(flag, non_blocking=True)
        self._ready = torch.cuda.Event()
        self._ready.record(torch.cuda.current_stream(x.device))
        F, N = w.shape
        self.w3 = torch.empty((3, N, F), dtype=torch.bfloat16, device=w.device)
        _lib.call("myelin_split_bf16x3", _lib.ptr(w), _lib.ptr(self.w3), F, N, 1, stream)
        self._exact = None

    def exact(self) -> bool:
        if self._exact is None:
            self._ready.synchronize()
            self._exact = int(self._host[0]) == 0
        return self._exact


def _split_synapse(x, w, stream, lean=False):
    """Start the exact split of ``x @ W`` (see _Split)."""

    return _Split(x, w, stream, lean)


def _split_eligible(prec: int, T: int, B: int, F: int, N: int) -> bool:
    """fp32 synapse on the chunked route with rows the bf16 loaders take and
    enough work to amortise the input check -- and no graph being captured
    on the current stream: the split's choice needs the input check's flag
    on the host (``_Split.exact``), a wait that capture does not allow and
    whose answer a replay could not revisit, so captured layers keep the
    fp32 engine."""

    return (prec == _lib.PREC["fp32"] and not _fused(B, N) and F % 8 == 0 and N % 8 == 0
            and T * B * F * N >= _SPLIT_MIN_MACS and not torch.cuda.is_current_stream_capturing())


class HipLinearFunction(torch.autograd.Function):
    """``inputs @ weight + bias`` on the MFMA GEMM (LinearSynapse, modules.py:112-133).

    Backward: ``dX = dY W^T``, ``dW = X^T dY``, ``db = sum over rows of dY``.
    """

    @staticmethod
    def forward(ctx: Any, x, w, b, prec):
        F, N = w.shape
        x2 = x.reshape(-1, F)
        M = x2.shape[0]
        out = torch.empty((M, N), dtype=x.dtype, device=x.device)
        _gemm(x2, w, out, M, N, F, F, N, N, False, False, False, prec, _lib.stream(x.device), bias=b)
        ctx.prec = prec
        ctx.has_b = b is not None
        ctx.save_for_backward(x2, w)
        ctx.in_shape = x.shape
        return out.reshape(*x.shape[:-1], N)

    @staticmethod
    def backward(ctx: Any, gy):
        x2, w = ctx.saved_tensors
        F, N = w.shape
        M = x2.shape[0]
        gy2 = gy.float().reshape(M, N).contiguous()
        dev = x2.device
        gx = gw = gb = None
        with torch.cuda.device(dev):
            stream = _lib.stream(dev)
            if ctx.needs_input_grad[0]:
                gx = torch.empty((M, F), dtype=x2.dtype, device=dev)
                _gemm(gy2, w, gx, M, F, N, N, N, F, False, True, False, ctx.prec, stream)
                gx = gx.reshape(ctx.in_shape)
            if ctx.has_b and ctx.needs_input_grad[2]:
                gb = torch.empty((N,), dtype=x2.dtype, device=dev)
            if ctx.needs_input_grad[1]:
                # db rides with dW's launches
                gw = torch.empty_like(w)
                _gemm(x2, gy2, gw, F, N, M, F, N, N, True, False, False, ctx.prec, stream,
                      col_sum=None if gb is None else (gy2, gb))
            elif gb is not None:
                _lib.call("myelin_col_sum_f32", _lib.ptr(gy2), _lib.ptr(gb), M, N, 0, stream)
        return gx, gw, gb, None


def linear(x, w, b, precision: str = "fp32"):
    """Differentiable ``x @ w + b`` for ``x [..., F]``, ``w [F, N]`` on the HIP GEMM."""

    _lib.require_device(x, "inputs")
    if x.dtype != torch.float32 or w.dtype != torch.float32:
        raise ValueError("inputs and weight must be float32 for the HIP path")
    if x.shape[-1] != w.shape[0]:
        raise ValueError("inputs.shape[-1] must match weight.shape[0]")
    with torch.cuda.device(x.device):
        return HipLinearFunction.apply(x.contiguous(), w.contiguous(), None if b is None else b.contiguous(),
                                       _lib.PREC[precision])


# currents buffer budget of the chunked path (floats)
_CURRENT_CHUNK_ELEMS = 1 << 25


def _fused_grid(B: int, N: int) -> int:
    """Workgroups of the fused kernel (its 8- or 4-row batch tiles)."""

    nt = -(-N // 64)
    return nt * -(-B // 8) if nt * -(-B // 8) >= 512 else nt * -(-B // 4)


def _fused(B: int, N: int) -> bool:
    """The forward takes the fused kernel (else GEMM chunks + recurrence)."""

    return N >= 64 and _fused_grid(B, N) >= 1024


def _span(T: int, checkpoint: int, BN: int, budget: int = _CURRENT_CHUNK_ELEMS) -> int:
    """Steps per backward span of a checkpointed layer: whole chunks, as
    many as keep a span's trace within ``budget`` floats."""

    return checkpoint * max(1, min(math.ceil(T / checkpoint), budget // (checkpoint * BN)))


# a narrow layer (<= 32 neurons) over packed spikes takes the one-launch
# currents + recurrence kernel from this batch size on: one workgroup per
# batch row, so smaller batches leave the chip idle and the GEMM + recurrence
# launches are faster
_NARROW_FUSED_MIN_B = 128

# forward chunk budget (floats) of the memory-lean policy: the forward's
# buffers are transient and never set a checkpointed step's peak, which the
# backward's span buffers do, so the forward keeps chunks large enough for
# its GEMMs to fill the chip
_LEAN_FWD_ELEMS = 1 << 24


def _budgets(lean: bool, checkpoint, B: int, N: int) -> tuple[int, int]:
    """(forward chunk, backward span) buffer budgets in floats.  Under the
    memory-lean policy (checkpoint_size="memory", whose purpose is to keep
    the chunk scratch small, checkpointing.py:13-20) a backward span is one
    checkpoint chunk and forward chunks hold 2**24 currents; otherwise both
    hold 2**25 -- fewer, larger GEMMs."""

    if lean and checkpoint is not None:
        return _LEAN_FWD_ELEMS, checkpoint * B * N
    return _CURRENT_CHUNK_ELEMS, _CURRENT_CHUNK_ELEMS


def _lif_fwd(x, w, b, m0, t0, t1, decay, threshold, reset, slope, rule, prec, stream, *, m_final=None,
             spikes=None, pre=None, packed=None, rates=None, ckpt=None, ckpt_every=1, wt=None, exact=False,
             pre_from=None, split=None, x32=None, x_bits=None, budget=_CURRENT_CHUNK_ELEMS, cur=None):
    """Synaptic currents + LIF recurrence over steps [t0, t1).

    ``x`` is fp32 with ``w [F, N]`` fp32, or bf16 (bf16 synapse) with ``wt``,
    the bf16 transposed weight ``[N, F]``.  Fused (one launch, currents stay
    in LDS) when N >= 64 and the fused grid has >= 1024 workgroups.
    Otherwise each workgroup would walk many chunks serially, so the steps
    are processed in chunks of up to ``budget`` currents: an MFMA GEMM (split-K
    when narrow) writes ``x_t @ W + b`` for the chunk, then the recurrence
    kernel consumes it, carrying the membrane and the spike counts across
    chunks; with several chunks, each chunk's GEMM runs on a side stream
    while the previous chunk's recurrence runs.  ``pre`` receives the steps
    from ``pre_from`` (default t0; the chunked route only) on; checkpoint
    rows count from t0.
    ``exact``: the GEMM never splits K, so a checkpointed forward and the
    backward's recompute of any chunk of it produce the same currents bit
    for bit (the fused kernel always sums that way).
    ``split`` (a _Split whose ``xb`` / ``w3`` are passed as x / wt, with
    ``x32`` the same steps of the fp32 input): the first chunk's GEMM is
    launched on the split before ``split.exact()`` is asked, so the GPU
    works while the host waits for the check; if the input is not
    bf16-exact that GEMM is redone on the fp32 engine into the same buffer
    and every later chunk takes the fp32 engine.
    ``x_bits``: the input as packed spike words ``[T, B, ceil(F / 32)]``,
    which the chunked route's GEMM reads in place of ``x`` (fp32 synapse
    weights ``w``; the same sums bit for bit).
    ``cur``: an fp32 buffer of at least one chunk's currents for the chunked
    route to use instead of allocating its own (when the GEMMs run in turn
    on the one stream).
    """

    if x_bits is not None:
        T, B = x_bits.shape[:2]
        F = w.shape[0]
    else:
        T, B, F = x.shape
    half = x_bits is None and x.dtype == torch.bfloat16
    parts = half and wt.ndim == 3  # exact split: wt holds the planes [3, N, F]
    N = wt.shape[-2] if half else w.shape[1]
    if _fused(B, N):
        if pre_from not in (None, t0):
            raise ValueError("pre_from is a chunked-route option")
        if parts or split is not None:
            raise ValueError("the split synapse is a chunked-route option")
        outs = (_lib.ptr(b), _lib.ptr(m0), _lib.ptr(m_final), _lib.ptr(spikes), _lib.ptr(pre), _lib.ptr(packed),
                _lib.ptr(rates), _lib.ptr(ckpt), T, B, F, N, t0, t1, ckpt_every, decay, threshold, reset, slope, rule)
        if half:
            _lib.call("myelin_linear_lif_fwd_bf16", _lib.ptr(x), _lib.ptr(wt), *outs, stream)
        else:
            _lib.call("myelin_linear_lif_fwd", _lib.ptr(x), _lib.ptr(w), *outs, prec, stream)
        return
    dev = x.device
    p0 = t0 if pre_from is None else pre_from  # pre holds the steps from p0 on
    if (x_bits is not None and N <= 32 and B >= _NARROW_FUSED_MIN_B and not exact and packed is None
            and ckpt is None and p0 == t0 and (rates is None or (t0 == 0 and t1 == T))
            and rule in (_lib.RULE_THRESHOLD, _lib.RULE_SURROGATE) and _lib.load().myelin_narrow_bits_fits(F, N, prec)):
        # a narrow layer over spikes with a batch that fills the chip: the
        # currents and the recurrence in one launch (never for a layer whose
        # backward recomputes, which must repeat its forward's GEMM)
        _lib.call("myelin_linear_lif_fwd_narrow_bits", _lib.ptr(x_bits), _lib.ptr(w), _lib.ptr(b), _lib.ptr(m0),
                  _lib.ptr(m_final), _lib.ptr(spikes), _lib.ptr(pre), _lib.ptr(rates), T, B, F, N, t0, t1, decay,
                  threshold, reset, slope, rule, prec, stream)
        return
    step = max(1, min(t1 - t0, budget // (B * N)))
    bounds = sorted({*range(t0, t1, step), t1} | ({p0} if t0 < p0 < t1 else set()))
    n = len(bounds) - 1
    # several chunks on the fp32 engine: each chunk's GEMM runs on the side
    # stream one chunk ahead of the recurrence, into two alternating
    # currents buffers.  The bf16 engines (and the split) fill the chip with
    # one workgroup per CU, and beside them the recurrence and the GEMM
    # slow each other down (the 1024 -> 4096 -> 20 rate network's step at
    # T=2000, B=32: 7.92-8.01 ms overlapped, 7.53 serial), so they run in
    # turn on the one stream.
    overlap = False
    if n > 1 and not half:
        main = torch.cuda.current_stream(dev)
        side = _side_stream(dev)
        overlap = main.cuda_stream == stream and side.cuda_stream != stream
    if cur is not None and not overlap and cur.dtype == torch.float32 and cur.numel() >= step * B * N:
        curs = [cur.reshape(-1)[:step * B * N].view(step, B, N)]
    else:
        curs = [torch.empty((step, B, N), dtype=torch.float32, device=dev) for _ in range(2 if overlap else 1)]
    # the membrane carried across chunks lives in m_final (each lane reads
    # its m0 before writing, so m0 may be m_final); a single chunk needs no
    # carry buffer at all
    state = m_final
    if state is None and n > 1:
        state = torch.empty((B, N), dtype=torch.float32, device=dev)
    # spike counts carried across chunks (one chunk counts in registers)
    counts = torch.zeros((B, N), dtype=torch.float32, device=dev) if rates is not None and n > 1 else None
    if overlap:
        side.wait_stream(main)
        done = [torch.cuda.Event(), torch.cuda.Event()]  # GEMM wrote buffer i
        used = [torch.cuda.Event(), torch.cuda.Event()]  # the recurrence read buffer i

    def gemm(c0, c1, cur, s):
        rows = (c1 - c0) * B
        if x_bits is not None:
            _gemm(x_bits[c0:c1], w, cur, rows, N, F, x_bits.shape[2], N, N, False, False, False, prec, s, bias=b,
                  a_bits=True, split=not exact)
        elif parts:
            _gemm_parts(x[c0:c1], wt, 3, N * F, cur, rows, N, F, F, F, N, False, True, False, s, bias=b,
                        split=not exact)
        elif half:
            _gemm(x[c0:c1], wt, cur, rows, N, F, F, F, N, False, True, False, prec, s, bias=b, split=not exact)
        else:
            _gemm(x[c0:c1], w, cur, rows, N, F, F, N, N, False, False, False, prec, s, bias=b, split=not exact)

    def fallback():
        # the input was not bf16-exact: the fp32 engine from here on
        nonlocal x, wt, half, parts
        x, wt, half, parts = x32, None, False, False

    for c in range(n):
        c0, c1 = bounds[c], bounds[c + 1]
        i = c % len(curs)
        cur = curs[i]
        s_ = side.cuda_stream if overlap else stream
        with torch.cuda.stream(side) if overlap else contextlib.nullcontext():
            if overlap and c >= 2:
                side.wait_event(used[i])
            gemm(c0, c1, cur, s_)
            if c == 0 and split is not None and not split.exact():
                fallback()
                gemm(c0, c1, cur, s_)
            if overlap:
                done[i].record(side)
        if overlap:
            main.wait_event(done[i])
        last = c1 == t1
        with_pre = pre is not None and c0 >= p0
        _lib.call(
            "myelin_lif_currents_fwd",
            _lib.ptr(cur), _lib.ptr(m0 if c0 == t0 else state), _lib.ptr(state), _lib.ptr(spikes),
            _lib.ptr(pre) if with_pre else None, _lib.ptr(packed), _lib.ptr(rates) if last else None,
            _lib.ptr(counts), _lib.ptr(ckpt), T, B, N, c0, c1, p0 if with_pre else t0, t0, ckpt_every, decay,
            threshold, reset, slope, rule, stream,
        )
        if overlap:
            used[i].record(main)
    if overlap:
        # the main stream waited on every side GEMM; the inputs' and buffers'
        # last users include the side stream
        for t_ in (*curs, x, w, b, wt, x32, *(() if split is None else (split.xb, split.w3))):
            if t_ is not None:
                t_.record_stream(side)


_SIDE_STREAMS: dict[tuple[int, int], torch.cuda.Stream] = {}


def _side_stream(dev: torch.device, which: int = 0) -> torch.cuda.Stream:
    """Side stream `which` of a device (default priority) for work that
    overlaps the current stream's, created once."""

    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    s = _SIDE_STREAMS.get((idx, which))
    if s is None:
        s = torch.cuda.Stream(device=idx)
        _SIDE_STREAMS[(idx, which)] = s
    return s


def _keep_trace(F: int, N: int) -> bool:
    """A checkpointed layer keeps its whole pre-reset trace ``[T, B, N]``
    instead of checkpoints (as the uncheckpointed path does), so its
    backward recomputes nothing, when the trace is narrow: at most 32
    neurons and at most 1/8 of the saved input's bytes -- the readout
    layers, whose recompute GEMM would re-read the whole input to rebuild a
    few columns and whose serial recurrence over T runs on a few waves."""

    return N <= 32 and 8 * N <= F


def _attach_bits(out, words) -> None:
    """Records the bit-packed copy of a spike tensor the layer wrote, with
    the tensor's version: a consumer may read the bits instead (1 bit per
    spike instead of 32) while the tensor is unmodified."""

    out._myelin_bits = (words, out._version)


def _spike_bits(x):
    """The packed words of ``x [T, B, F]`` recorded by the layer that wrote
    it, or None when there are none or ``x`` changed since (its version
    moved on)."""

    rec = getattr(x, "_myelin_bits", None)
    if rec is None:
        return None
    words, version = rec
    T, B, F = x.shape
    if version != x._version or words.shape != (T, B, -(-F // 32)) or words.device != x.device:
        return None
    return words


def _bits_consumer(B: int, F: int, N: int, prec: int) -> bool:
    """A layer reads its input's packed twin: the chunked route with a
    narrow output (the GEMMs stream the input once per pass; the bits cut
    those reads 32-fold and sum the same products in the same order)."""

    return N <= 32 and not _fused(B, N) and not _half(prec, F, N)


class HipLinearLIFFunction(torch.autograd.Function):
    """Outputs ``(final_membrane, spikes)`` or, with ``rate=True``,
    ``(final_membrane, rates)`` where ``rates = spike_count / T``."""

    @staticmethod
    def forward(ctx: Any, x, w, b, decay, threshold, reset, sid, slope, checkpoint, rate, prec, rule, lean=False):
        T, B, F = x.shape
        N = w.shape[1]
        dev = x.device
        stream = _lib.stream(dev)
        need = any(ctx.needs_input_grad[:3])
        half = _half(prec, F, N)
        xs, wt = _cast_transpose_bf16(x, w, stream) if half else (x, None)
        bits = _spike_bits(x) if _bits_consumer(B, F, N, prec) else None
        fwd_budget, budget = _budgets(lean, checkpoint, B, N)
        split = None
        if not half and bits is None and _split_eligible(prec, T, B, F, N):
            split = _split_synapse(x, w, stream, lean=lean and checkpoint is not None)
            xs, wt = split.xb, split.w3
        m_final = torch.empty((B, N), dtype=x.dtype, device=dev)
        out = torch.empty((B, N) if rate else (T, B, N), dtype=x.dtype, device=dev)
        # spikes: their packed twin too (N / 8 bytes per row more), for a
        # narrow layer reading them next
        words = torch.empty((T, B, -(-N // 32)), dtype=torch.int32, device=dev) if not rate else None
        if checkpoint is not None and _keep_trace(F, N):
            checkpoint = None
        pre = ckpt = None
        tail = 0
        if need:
            if checkpoint is None:
                pre = torch.empty((T, B, N), dtype=x.dtype, device=dev)
            else:
                ckpt = torch.empty((math.ceil(T / checkpoint), B, N), dtype=x.dtype, device=dev)
                if not _fused(B, N):
                    # the backward starts with the last span, whose trace
                    # this forward computes anyway: keep it (the buffer the
                    # backward would fill) instead of recomputing it there
                    span = _span(T, checkpoint, B * N, budget)
                    tail = (math.ceil(T / span) - 1) * span
                    pre = torch.empty((T - tail, B, N), dtype=x.dtype, device=dev)
        _lif_fwd(xs, w, b, None, 0, T, decay, threshold, reset, slope, rule, prec, stream, m_final=m_final,
                 spikes=None if rate else out, pre=pre, packed=words, rates=out if rate else None, ckpt=ckpt,
                 ckpt_every=checkpoint or 1, wt=wt, exact=ckpt is not None, pre_from=tail, split=split, x32=x,
                 x_bits=bits, budget=fwd_budget)
        if split is not None and not split.exact():
            xs, wt = x, None
        if words is not None:
            _attach_bits(out, words)
        if bits is not None:
            xs = bits  # what the backward's weight GEMM reads
        lazy = isinstance(xs, _LazyBf16)
        ctx.set_materialize_grads(False)
        ctx.meta = (decay, threshold, reset, sid, slope, checkpoint, rate, prec, rule, b is not None,
                    F if bits is not None else None, budget, lazy)
        if need:
            # the bf16 synapse keeps the bf16 copies of x and W^T (what its
            # GEMMs read); the lean split keeps x and casts per span
            ctx.save_for_backward(x if lazy else xs, w, b, pre, ckpt, wt)
        return m_final, out

    @staticmethod
    def backward(ctx: Any, g_m, g_out):
        none = (None,) * 13
        if (g_m is None and g_out is None) or not any(ctx.needs_input_grad[:3]):
            return none
        decay, threshold, reset, sid, slope, checkpoint, rate, prec, rule, has_b, bits_f, budget, lazy = ctx.meta
        xs, w, b, pre, ckpt, wt = ctx.saved_tensors
        if lazy:
            xs = _LazyBf16(xs)
        need_x, need_w, need_b = ctx.needs_input_grad[:3]
        gx, gw, gb = linear_backward(xs, w, b if has_b else None, pre, ckpt, wt, g_m, g_out, decay, threshold,
                                     reset, sid, slope, checkpoint, rate, prec, rule, need_x, need_w,
                                     need_b and has_b, bits_f=bits_f, budget=budget)
        return gx, gw, gb, None, None, None, None, None, None, None, None, None, None


def linear_backward(xs, w, b, pre, ckpt, wt, g_m, g_out, decay, threshold, reset, sid, slope, checkpoint, rate,
                    prec, rule, need_x=True, need_w=True, need_b=True, bits_f=None, budget=_CURRENT_CHUNK_ELEMS):
    """Gradients (dX, dW, db) of the streamed-synapse LIF, span by span in
    reverse time: recompute the span's pre-reset trace from its first
    checkpoint (``checkpoint=None``: the saved trace ``pre`` covers all T;
    with a checkpoint, ``pre`` if given is the last span's trace, kept by
    the forward), reverse the recurrence into G = dL/dI, then ``dX = G W^T`` and
    ``dW += X^T G`` on the MFMA GEMM and ``db`` as a fixed-order column
    sum.  ``xs`` is fp32, or
    bf16 with ``wt = W^T`` bf16 for the bf16 synapse, or (``bits_f`` = F)
    the input spikes' packed words ``[T, B, ceil(F / 32)]``; ``g_out`` is
    dL/dspikes ``[T, B, N]`` or, with ``rate``, dL/drates ``[B, N]``."""

    T, B, F = xs.shape
    x_bits = xs if bits_f is not None else None
    if x_bits is not None:
        F = bits_f
    N = w.shape[1]
    BN = B * N
    dev = xs.device
    parts = wt is not None and wt.ndim == 3  # exact split: xs bf16-exact, wt the planes of W
    half = xs.dtype == torch.bfloat16 and not parts
    with torch.cuda.device(dev):
        stream = _lib.stream(dev)
        wg = _cast_bf16(w, stream) if (half and need_x) else w
        # the reverse pass walks spans of whole checkpoint chunks, as many as
        # keep a span's trace within `budget` floats: one recompute
        # (from the span's first checkpoint, which the recurrence carries
        # through the later ones exactly as the forward did), one reverse
        # launch and one dX / dW GEMM pair per span instead of per chunk
        span = T if checkpoint is None else _span(T, checkpoint, BN, budget)
        per = 1 if checkpoint is None else span // checkpoint  # checkpoint rows per span
        want_gb = need_b and b is not None
        # one span and no membrane gradient: the reverse launch is the whole
        # pass (no adjoint buffer; it writes the bias sums itself), else the
        # zero-started buffers (the membrane adjoint unless given, the bias
        # gradient's accumulator) share one allocation: one fill launch
        whole = g_m is None and span >= T
        zeros = None
        if not whole and (g_m is None or want_gb):
            zeros = torch.zeros(((g_m is None) + want_gb, B, N), device=dev)
        gm = g_m.float().contiguous().clone() if g_m is not None else (None if whole else zeros[0])
        g_out = None if g_out is None else g_out.float().contiguous()
        g_spikes = None if rate else g_out
        g_rates = g_out if rate else None
        gx = torch.empty((T, B, F), device=dev) if need_x else None
        gw = torch.empty_like(w) if need_w else None  # the first (last-in-time) span overwrites it
        gb_acc = (torch.empty((B, N), device=dev) if whole else zeros[-1]) if want_gb else None
        gb = torch.empty((N,), device=dev) if want_gb else None
        # exact split: dW reads G as three bf16 planes [3, C, B, N] (C the
        # span's steps), written by the reverse pass itself unless dX needs
        # the fp32 G as well
        G3 = torch.empty(3 * min(span, T) * BN, dtype=torch.bfloat16, device=dev) if parts and need_w else None
        if G3 is not None and not need_x:
            G = G3
        else:
            G = torch.empty((min(span, T), B, N), dtype=torch.bfloat16 if half else torch.float32, device=dev)
        n_spans = math.ceil(T / span)
        tail = pre if checkpoint is not None else None  # the last span's trace, from the forward
        if tail is not None and tail.shape[0] != T - (n_spans - 1) * span:
            raise ValueError("the saved trace does not cover the last backward span")
        recomputes = checkpoint is not None and (tail is None or n_spans > 1)
        # GEMM recomputes on the fp32 engine run one span ahead on a side
        # stream, into two alternating trace buffers: span k-1's recompute
        # overlaps span k's reverse pass and weight GEMMs (the bf16 engines
        # and the split run in turn, as in the forward).  ready[i]: buffer i
        # holds its span's trace; free[i]: the reverse pass has read buffer i.
        overlap = checkpoint is not None and n_spans > 1 and not (half or parts)
        # in turn, the trace buffer is spent once the reverse pass has read
        # it and is refilled only by the next span's recompute: it doubles
        # as the split-K workspace of the span's dX and dW GEMMs
        ws = None
        if recomputes:
            n_sc = min(span, T) * BN
            if not overlap:
                lib, r_span = _lib.load(), min(span, T) * B
                n_sc = max(n_sc, lib.myelin_gemm_workspace_elems(r_span, F, N, prec) if need_x else 0,
                           lib.myelin_gemm_workspace_elems(F, N, r_span, _lib.PREC["bf16"] if parts else prec)
                           if need_w else 0)
            ws = torch.empty(n_sc, device=dev)
            scratch = ws[:min(span, T) * BN].view(min(span, T), B, N)
            if overlap:
                ws = None
        else:
            scratch = None
        if overlap:
            main = torch.cuda.current_stream(dev)
            side = _side_stream(dev)
            bufs = [scratch, torch.empty_like(scratch)]
            ready = [torch.cuda.Event(), torch.cuda.Event()]
            free = [torch.cuda.Event(), torch.cuda.Event()]
            side.wait_stream(main)

            def recompute(j):
                i = j % 2
                with torch.cuda.stream(side):
                    if j + 2 < n_spans:
                        side.wait_event(free[i])
                    _lif_fwd(xs, w, b, ckpt[j * per], j * span, min(j * span + span, T), decay, threshold, reset,
                             slope, rule, prec, side.cuda_stream, pre=bufs[i], wt=wt, exact=True, x_bits=x_bits,
                             budget=budget)
                    ready[i].record(side)

            if tail is None:
                recompute(n_spans - 1)
        for k in range(n_spans - 1, -1, -1):
            t0 = k * span
            t1 = min(t0 + span, T)
            C = t1 - t0
            if checkpoint is None:
                pre_k = pre
            elif k == n_spans - 1 and tail is not None:
                if overlap:
                    recompute(k - 1)
                pre_k = tail
            elif overlap:
                if k > 0:
                    recompute(k - 1)
                main.wait_event(ready[k % 2])
                pre_k = bufs[k % 2]
            else:
                # the recompute's currents may use G's buffer: the reverse
                # pass writes G only after the recompute
                _lif_fwd(xs, w, b, ckpt[k * per], t0, t1, decay, threshold, reset, slope, rule, prec, stream,
                         pre=scratch, wt=wt, exact=True, x_bits=x_bits, budget=budget, cur=G)
                pre_k = scratch
            _lib.call(
                "myelin_linear_pre_bwd",
                _lib.ptr(pre_k), _lib.ptr(g_spikes[t0:t1]) if g_spikes is not None else None,
                _lib.ptr(g_rates), _lib.ptr(gm), _lib.ptr(G), _lib.DT_BF16X3 if G is G3 else _lib.DT[G.dtype],
                _lib.ptr(gb_acc),
                C, BN, T, decay, threshold, reset, slope, sid, rule, stream,
            )
            if overlap:
                free[k % 2].record(main)
            rows = C * B
            # (dW on a third stream beside dX measured slower on the readout
            # shapes: the 784 -> 2048 -> 10 bf16 training step at T=50,
            # B=256 went from 0.547 to 0.606 ms)
            if gx is not None:
                # dX[t0:t1] = G @ W^T : [rows, N] x [N, F]
                _gemm(G, wg, gx[t0:t1], rows, F, N, N, N, F, False, True, False, prec, stream, ws=ws)
            # db (the bias sums complete once the first span's reverse pass
            # has run) rides with that span's dW launches
            cs = (gb_acc, gb) if k == 0 and gb is not None else None
            if gw is not None and parts:
                if G is not G3:
                    _lib.call("myelin_split_bf16x3", _lib.ptr(G), _lib.ptr(G3), rows, N, 0, stream)
                _gemm_parts(xs[t0:t1], G3, 3, rows * N, gw, F, N, rows, F, N, N, True, False, k != n_spans - 1,
                            stream, ws=ws, col_sum=cs)
            elif gw is not None and x_bits is not None:
                _gemm(x_bits[t0:t1], G, gw, F, N, rows, x_bits.shape[2], N, N, True, False, k != n_spans - 1, prec,
                      stream, a_bits=True, ws=ws, col_sum=cs)
            elif gw is not None:
                # dW (+)= X[t0:t1]^T @ G : [F, rows] x [rows, N]
                _gemm(xs[t0:t1], G, gw, F, N, rows, F, N, N, True, False, k != n_spans - 1, prec, stream, ws=ws,
                      col_sum=cs)
        if overlap:
            # every side-stream kernel is behind a ready[] the main stream
            # waited on; the buffers' last users include the side stream
            for t in (*bufs, xs, w, ckpt, *(() if b is None else (b,)), *(() if wt is None else (wt,))):
                t.record_stream(side)
        if gb is not None and gw is None:
            _lib.call("myelin_col_sum_f32", _lib.ptr(gb_acc), _lib.ptr(gb), B, N, 0, stream)
    return gx, gw, gb


def linear_forward(x, w, b, params, surrogate_id: int, slope: float, checkpoint, rate: bool, precision: str,
                   rule: int = _lib.RULE_THRESHOLD, lean: bool = False):
    """Validate and run the fused streamed-synapse LIF (shared by the public
    entry points in myelin_amd.kernels).  ``lean``: the memory-lean policy
    (chunk and span buffers of one checkpoint chunk)."""

    if x.ndim != 3:
        raise ValueError(f"inputs must be shaped [T, B, F]; got {tuple(x.shape)}")
    if w.ndim != 2:
        raise ValueError(f"weight must be shaped [F, N]; got {tuple(w.shape)}")
    _lib.require_device(x, "inputs")
    if w.device != x.device or w.dtype != x.dtype:
        raise ValueError("weight must have the same device and dtype as inputs")
    if x.shape[2] != w.shape[0]:
        raise ValueError("inputs.shape[2] must match weight.shape[0]")
    if b is not None:
        if b.shape != (w.shape[1],):
            raise ValueError("bias must be shaped [N]")
        if b.device != x.device or b.dtype != x.dtype:
            raise ValueError("bias must have the same device and dtype as inputs")
    if x.dtype != torch.float32:
        raise ValueError(f"inputs must be float32 for the HIP path; got {x.dtype}")
    if x.shape[0] == 0:
        raise ValueError("inputs must have at least one timestep")
    if precision not in _lib.PREC:
        raise ValueError("synapse_precision must be 'fp32' or 'bf16'")
    with torch.cuda.device(x.device):
        return HipLinearLIFFunction.apply(
            x.contiguous(), w.contiguous(), None if b is None else b.contiguous(), float(params.decay),
            float(params.threshold), float(params.reset), surrogate_id, float(slope), checkpoint, rate,
            _lib.PREC[precision], rule, lean,
        )


def linear_packed_forward(x, w, b, params, checkpoint: int, precision: str):
    """Forward-only packed-spike output (no dense [T, B, N] spikes)."""

    from myelin_amd.packing import PackedSpikes, packed_last_dim_size

    if x.ndim != 3:
        raise ValueError(f"inputs must be shaped [T, B, F]; got {tuple(x.shape)}")
    _lib.require_device(x, "inputs")
    if x.shape[2] != w.shape[0]:
        raise ValueError("inputs.shape[2] must match weight.shape[0]")
    if x.dtype != torch.float32 or w.dtype != torch.float32:
        raise ValueError("inputs and weight must be float32 for the HIP path")
    x = x.contiguous()
    w = w.contiguous()
    b = None if b is None else b.contiguous()
    T, B, F = x.shape
    N = w.shape[1]
    m_final = torch.empty((B, N), device=x.device)
    words = torch.empty((T, B, packed_last_dim_size(N)), dtype=torch.int32, device=x.device)
    with torch.cuda.device(x.device):
        _lif_fwd(x, w, b, None, 0, T, float(params.decay), float(params.threshold), float(params.reset), 10.0,
                 _lib.RULE_THRESHOLD, _lib.PREC[precision], _lib.stream(x.device), m_final=m_final, packed=words,
                 ckpt_every=checkpoint)
    return m_final, PackedSpikes(data=words, original_shape=(T, B, N))
