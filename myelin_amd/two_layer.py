"""Two-layer LIF rate network (input -> hidden LIF -> readout LIF rates) with
the two layers interleaved per checkpoint chunk.

Reference: ``TwoLayerSurrogateLIFRateRecomputeFunction`` and
``TwoLayerSurrogateLIFRatePackedHiddenFunction`` (autograd.py:926-1387),
entry points ``kernels.py:779-846``.  The reference runs each layer over all
T steps in turn, so the hidden spikes ``[T, B, H]`` exist densely between
them (in the packed variant they are unpacked to dense in both passes,
autograd.py:1185,1284), and its backward produces a dense ``[T, B, H]``
hidden-spike gradient.

Here both passes walk time in chunks of C steps (the checkpoint size):

* forward, a group of chunks at a time (as many as keep the group's hidden
  currents within 2**25 elements): hidden ``x_t @ W_h`` + LIF from the
  carried hidden membrane -> hidden spikes of the group (dense, or in the
  packed variant only their words ``[T, B, ceil(H/32)]``); readout
  ``s_t @ W_o`` + LIF from the carried readout membrane and spike counts.
  Chunk-start membranes of both layers are kept ``[ceil(T/C), B, H + O]``.
* backward, spans of whole chunks in reverse (as many chunks as keep a
  span's hidden trace within 2**24 elements): recompute the hidden span
  from its first checkpoint (pre-reset trace; its spikes, or in the packed
  variant the stored words read as bits by the readout GEMMs, feed the
  readout), take the readout's trace (saved whole when the readout is
  narrow, else recomputed), reverse the readout recurrence (adjoint carried
  across spans), ``dS = G_o @ W_o^T`` for the span only, then reverse the
  hidden recurrence with ``dS`` as its spike gradient.

So no tensor with T in its shape is written except the input gradient, the
narrow readout's pre-reset trace ``[T, B, O]`` and, in the packed variant,
the packed words -- which its readout GEMMs read directly, so that variant
never forms dense hidden spikes at all.  The
arithmetic of each step is that of the one-layer checkpointed path (same
kernels), so rates and gradients equal those of composing the two
one-layer functions.
"""

from __future__ import annotations

import math
from typing import Any

import torch

from myelin_amd import _lib
from myelin_amd.linear import (_CURRENT_CHUNK_ELEMS, _LEAN_FWD_ELEMS, _cast_bf16, _cast_transpose_bf16, _gemm,
                               _gemm_parts, _half, _keep_trace, _LazyBf16, _lif_fwd, _side_stream, _split_eligible,
                               _split_synapse)

# trace budget of a backward span (floats per buffer): the backward walks
# whole checkpoint chunks, as many at a time as keep each per-span buffer
# within it.  At T=2000, B=32, 1024 -> 4096 -> 20 with 45-step chunks
# (packed variant, the hidden synapse on the exact bf16 split), budgets of
# 2^24 / 2^25 / 2^26 floats (spans of 2 / 5 / 11 chunks) measured 8.20-8.30
# / 7.52-7.59 / 7.42 ms per training step at 502 / 870 / 1527 MB peak: a
# span's recompute GEMM of 2,880 rows fills 1.5 rounds of 256 x 128 tiles,
# one of 7,200 rows takes 256 x 256 tiles.  2^25, the one-layer budget,
# keeps the route at half the modules' peak memory.
_SPAN_ELEMS = 1 << 25


def _ds_fused(prec: int, O: int, H: int, L: int) -> bool:
    """The hidden reverse pass forms its spike gradient dS = G_o W_o^T
    itself (myelin_linear_pre_bwd_readout: the fp32 small-K GEMM's sums,
    without dS in memory) for fp32 products, a readout of at most 32
    neurons, a hidden width that is a multiple of 256 and a span whose
    G_o rows fit the kernel's 64 KB of LDS."""

    kmax = next(k for k in (8, 12, 16, 20, 24, 32) if O <= k) if O <= 32 else 0
    return prec == _lib.PREC["fp32"] and 0 < O <= 32 and H % 256 == 0 and L * kmax * 4 <= 65536


def _zeros_views(dev, *shapes):
    """Zero-filled float32 tensors of the given shapes (None gives None), all
    views of one allocation at 256-byte boundaries: one fill launch where
    separate torch.zeros calls would each launch one."""

    sizes = [0 if sh is None else math.prod(sh) for sh in shapes]
    pads = [-(-n // 64) * 64 for n in sizes]
    buf = torch.zeros(max(1, sum(pads)), device=dev)
    out, at = [], 0
    for sh, n, pn in zip(shapes, sizes, pads):
        out.append(None if sh is None else buf[at:at + n].view(sh))
        at += pn
    return out


def _readout_chunk(cur, hs, wo, bo, m0, m_final, pre, counts, rates, ckpt, T, t0, t1, C, decay, threshold, reset,
                   slope, prec, stream, exact=False):
    """Readout currents ``hs @ W_o + b_o`` for steps [t0, t1) then the LIF
    recurrence over them in absolute time (counts and rates over all T).
    ``hs`` is the chunk's hidden spikes, dense fp32 ``[L, B, H]`` or packed
    words ``[L, B, ceil(H/32)]`` int32 (read as bits by the GEMM).
    ``exact``: no K split, so a recompute reproduces the currents exactly."""

    B, O = m0.shape
    H = wo.shape[0]
    L = t1 - t0
    if hs.dtype == torch.int32:
        _gemm(hs, wo, cur, L * B, O, H, hs.shape[-1], O, O, False, False, False, prec, stream, bias=bo, a_bits=True,
              split=not exact)
    else:
        _gemm(hs, wo, cur, L * B, O, H, H, O, O, False, False, False, prec, stream, bias=bo, split=not exact)
    _lib.call(
        "myelin_lif_currents_fwd",
        _lib.ptr(cur), _lib.ptr(m0), _lib.ptr(m_final), None, _lib.ptr(pre), None, _lib.ptr(rates),
        _lib.ptr(counts), _lib.ptr(ckpt), T, B, O, t0, t1, t0, 0, C, decay, threshold, reset, slope,
        _lib.RULE_THRESHOLD, stream,
    )


class HipTwoLayerRateFunction(torch.autograd.Function):
    """Returns readout rates ``[B, O]`` = readout spike count / T."""

    @staticmethod
    def forward(ctx: Any, x, wh, bh, wo, bo, decay, threshold, reset, sid, slope, C, prec, packed_hidden, lean=False):
        T, B, F = x.shape
        H = wh.shape[1]
        O = wo.shape[1]
        dev = x.device
        stream = _lib.stream(dev)
        need = any(ctx.needs_input_grad[:5])
        K = math.ceil(T / C)
        L0 = min(C, T)
        # a narrow readout keeps its whole pre-reset trace [T, B, O] for the
        # backward, which then recomputes nothing of the readout
        keep = need and _keep_trace(H, O)
        ck_h = torch.empty((K, B, H), device=dev) if need else None
        ck_o = torch.empty((K, B, O), device=dev) if need and not keep else None
        m_h, m_o, counts = _zeros_views(dev, (B, H), (B, O), (B, O))
        rates = torch.empty((B, O), device=dev)
        # the forward has no per-chunk state to keep beyond the checkpoints,
        # so it runs whole groups of chunks: a group's hidden currents fill
        # up to 2**25 elements, as in the one-layer chunked path (2**24 under
        # the memory-lean policy: the forward's buffers stay below the
        # backward's)
        G = max(1, min(K, (_LEAN_FWD_ELEMS if lean else _CURRENT_CHUNK_ELEMS) // (L0 * B * H)))
        LG = min(G * C, T)
        # the packed variant never forms dense hidden spikes: its readout
        # GEMM reads the words, and as the words of all T are kept, the
        # readout runs once after the hidden layer (one currents GEMM and
        # one recurrence over T instead of one pair per group: a narrow
        # GEMM's rows do not depend on how many rows it is given, and the
        # recurrence carries its state exactly, so the results are the same)
        hs = None if packed_hidden else torch.empty((LG, B, H), device=dev)
        cur = torch.empty((T if packed_hidden else LG, B, O), device=dev)
        pre_o = torch.empty((T, B, O), device=dev) if keep else None
        words = torch.empty((T, B, (H + 31) // 32), dtype=torch.int32, device=dev) if packed_hidden else None
        # bf16 synapse: the hidden GEMMs read bf16 copies of x and W_h^T
        half = _half(prec, F, H)
        xs, wt = _cast_transpose_bf16(x, wh, stream) if half else (x, None)
        # spike inputs: the hidden synapse on the exact bf16 split (the first
        # group's forward learns whether the input qualifies)
        split = None
        if not half and _split_eligible(prec, T, B, F, H):
            split = _split_synapse(x, wh, stream, lean=lean)
            xs, wt = split.xb, split.w3
        for k in range(0, K, G):
            t0 = k * C
            t1 = min(t0 + G * C, T)
            L = t1 - t0
            _lif_fwd(xs[t0:t1], wh, bh, m_h, 0, L, decay, threshold, reset, slope, _lib.RULE_THRESHOLD, prec, stream,
                     m_final=m_h, spikes=None if hs is None else hs[:L],
                     packed=None if words is None else words[t0:t1], ckpt=None if ck_h is None else ck_h[k:],
                     ckpt_every=C, wt=wt, exact=need, split=split if k == 0 else None,
                     x32=x[t0:t1] if k == 0 else None, budget=LG * B * H)
            if k == 0 and split is not None and not split.exact():
                xs, wt = x, None
            if hs is not None:
                _readout_chunk(cur[:L], hs[:L], wo, bo, m_o, m_o, None if pre_o is None else pre_o[t0:t1], counts,
                               rates if t1 == T else None, ck_o, T, t0, t1, C, decay, threshold, reset, slope, prec,
                               stream, exact=need and not keep)
        if hs is None:
            _readout_chunk(cur, words, wo, bo, m_o, m_o, pre_o, counts, rates, ck_o, T, 0, T, C, decay, threshold,
                           reset, slope, prec, stream, exact=need and not keep)
        lazy = isinstance(xs, _LazyBf16)
        ctx.set_materialize_grads(False)
        ctx.meta = (decay, threshold, reset, sid, slope, C, prec, bh is not None, bo is not None, lean, lazy)
        if need:
            # the lean split keeps x and casts each span's steps to bf16
            ctx.save_for_backward(x if lazy else xs, wh, bh, wo, bo, ck_h, ck_o, words, wt, pre_o)
        return rates

    @staticmethod
    def backward(ctx: Any, g_rates):
        none = (None,) * 14
        if g_rates is None or not any(ctx.needs_input_grad[:5]):
            return none
        decay, threshold, reset, sid, slope, C, prec, has_bh, has_bo, lean, lazy = ctx.meta
        xs, wh, bh, wo, bo, ck_h, ck_o, words, wt, pre_all = ctx.saved_tensors
        if lazy:
            xs = _LazyBf16(xs)
        parts = wt is not None and wt.ndim == 3  # exact split of the hidden synapse
        half = xs.dtype == torch.bfloat16 and not parts
        need_x, need_wh, need_bh, need_wo, need_bo = ctx.needs_input_grad[:5]
        need_hidden = need_x or need_wh or (need_bh and has_bh)
        T, B, F = xs.shape
        H = wh.shape[1]
        O = wo.shape[1]
        dev = xs.device
        K = math.ceil(T / C)
        # spans of `per` whole chunks (recomputed from the span's first
        # checkpoints, which the recurrences carry through the later ones
        # exactly as the forward did); one chunk under the memory-lean policy
        per = 1 if lean else max(1, min(K, _SPAN_ELEMS // (C * B * max(H, O))))
        S = per * C
        NS = math.ceil(T / S)
        L0 = min(S, T)
        with torch.cuda.device(dev):
            stream = _lib.stream(dev)
            g_rates = g_rates.float().contiguous()
            gm_o, gm_h, gbh_acc, gbo_acc = _zeros_views(
                dev, (B, O), (B, H) if need_hidden else None, (B, H) if (need_bh and has_bh) else None,
                (B, O) if (need_bo and has_bo) else None)
            gx = torch.empty((T, B, F), device=dev) if need_x else None
            whg = _cast_bf16(wh, stream) if (half and need_x) else wh
            # the first (last-in-time) span overwrites the weight gradients
            gwh = torch.empty_like(wh) if need_wh else None
            gwo = torch.empty_like(wo) if need_wo else None
            # the bias gradients (column sums of the accumulators, complete
            # once the first span's reverse passes have run) ride with that
            # span's weight-gradient launches
            gbh = torch.empty((H,), device=dev) if gbh_acc is not None else None
            gbo = torch.empty((O,), device=dev) if gbo_acc is not None else None
            cur = torch.empty((L0, B, O), device=dev) if pre_all is None else None
            pre_o = torch.empty((L0, B, O), device=dev) if pre_all is None else None
            # the packed variant with the readout's whole trace kept: the
            # readout's reverse pass runs span by span from the last on a
            # stream of its own (a few waves walking T: beside the hidden
            # spans it costs them nothing), each hidden span waiting for its
            # rows of G_o only; dW_o reads every step's words at once, after
            # the spans (the reverse pass carries its adjoint across spans
            # exactly).  The memory-lean policy (one-chunk spans) runs the
            # reverse pass as one launch and dW_o before the spans, on the
            # one stream: there the blocks the side stream holds raise the
            # peak and the many short spans gain nothing from the overlap
            main = torch.cuda.current_stream(dev)
            whole_o = words is not None and pre_all is not None
            G_o_all = None
            o_side = whole_o and not lean
            if whole_o:
                G_o_all = torch.empty((T, B, O), device=dev)
                o_stream = _side_stream(dev, 1) if o_side else main
                o_ready = [torch.cuda.Event() for _ in range(NS)] if o_side else None
                if o_side:
                    o_stream.wait_stream(main)
                with torch.cuda.stream(o_stream):
                    for k in (range(NS - 1, -1, -1) if o_side else (None,)):
                        a0, a1 = (k * S, min(k * S + S, T)) if o_side else (0, T)
                        _lib.call(
                            "myelin_linear_pre_bwd",
                            _lib.ptr(pre_all[a0:a1]), None, _lib.ptr(g_rates), _lib.ptr(gm_o),
                            _lib.ptr(G_o_all[a0:a1]), _lib.DT[torch.float32], _lib.ptr(gbo_acc), a1 - a0, B * O, T,
                            decay, threshold, reset, slope, sid, _lib.RULE_THRESHOLD, o_stream.cuda_stream,
                        )
                        if o_side:
                            o_ready[k].record(o_stream)
                if o_side:
                    for t_ in (pre_all, g_rates, gm_o, G_o_all, gbo_acc):
                        if t_ is not None:
                            t_.record_stream(o_stream)

                def readout_weight_grads():
                    if o_side:
                        main.wait_event(o_ready[0])
                    if gwo is not None:
                        _gemm(words, G_o_all, gwo, H, O, T * B, words.shape[-1], O, O, True, False, False, prec,
                              stream, a_bits=True, col_sum=None if gbo is None else (gbo_acc, gbo))
                    elif gbo is not None:
                        _lib.call("myelin_col_sum_f32", _lib.ptr(gbo_acc), _lib.ptr(gbo), B, O, 0, stream)

                if not o_side or not need_hidden:
                    readout_weight_grads()
                if not need_hidden:
                    return gx, None, None, gwo, gbo, None, None, None, None, None, None, None, None, None
            G_o = None if whole_o else torch.empty((L0, B, O), device=dev)
            # the memory-lean policy runs the recompute in turn on the one
            # stream (one buffer set, and the recompute's currents reuse the
            # dS buffer, which that span fills only after its recompute),
            # and the hidden trace and dS (both spent once the hidden
            # reverse pass has run) share one pool with the split-K
            # workspace of the dX / dW_h GEMMs that follow it
            recomputes = need_hidden or words is None
            nset = 2 if (recomputes and NS > 1 and not lean) else 1
            # dS formed inside the hidden reverse pass needs no buffer of its
            # own (the lean recompute still borrows that pool slot)
            fused_ds = need_hidden and _ds_fused(prec, O, H, L0)
            pool = None
            if lean and need_hidden:
                n_ws = max(_lib.load().myelin_gemm_workspace_elems(F, H, L0 * B, _lib.PREC["bf16"] if parts else prec)
                           if need_wh else 0,
                           _lib.load().myelin_gemm_workspace_elems(L0 * B, F, H, prec) if need_x else 0)
                pool = torch.empty(max(2 * L0 * B * H, n_ws), device=dev)
                ghs = pool[L0 * B * H:2 * L0 * B * H].view(L0, B, H)
            else:
                ghs = torch.empty((L0, B, H), device=dev) if need_hidden and not fused_ds else None
            # exact split: dW_h reads G_h as three bf16 planes [3, L, B, H],
            # written by the reverse pass itself unless dX needs the fp32 G_h
            G3 = torch.empty(3 * L0 * B * H, dtype=torch.bfloat16, device=dev) if parts and need_wh else None
            if G3 is not None and not need_x:
                G_h = G3
            else:
                G_h = (torch.empty((L0, B, H), dtype=torch.bfloat16 if half else torch.float32, device=dev)
                       if need_hidden else None)
            # The hidden recompute (its trace, and spikes in the dense
            # variant) runs one span ahead on a side stream into two
            # alternating buffer sets, overlapping the current span's
            # readout and hidden reverse passes and GEMMs.  ready[i]: set i
            # holds its span; free[i]: the span using set i is done with it.
            hs_b = [None if words is not None else torch.empty((L0, B, H), device=dev) for _ in range(nset)]
            if pool is not None:
                pre_b = [pool[:L0 * B * H].view(L0, B, H)]
            else:
                pre_b = [torch.empty((L0, B, H), device=dev) if need_hidden else None for _ in range(nset)]
            side = _side_stream(dev) if nset == 2 else main
            ready = [torch.cuda.Event() for _ in range(nset)]
            free = [torch.cuda.Event() for _ in range(nset)]
            if nset == 2:
                side.wait_stream(main)

            def hidden_recompute(j):
                i = j % nset
                a0, a1 = j * S, min(j * S + S, T)
                n = a1 - a0
                with torch.cuda.stream(side):
                    if nset == 2 and j + 2 < NS:
                        side.wait_event(free[i])
                    pre_j = None if pre_b[i] is None else pre_b[i][:n]
                    shared = ghs if (lean and nset == 1) else None
                    if words is not None:
                        _lif_fwd(xs[a0:a1], wh, bh, ck_h[j * per], 0, n, decay, threshold, reset, slope,
                                 _lib.RULE_THRESHOLD, prec, side.cuda_stream, pre=pre_j, wt=wt, exact=True,
                                 budget=L0 * B * H, cur=shared)
                    else:
                        _lif_fwd(xs[a0:a1], wh, bh, ck_h[j * per], 0, n, decay, threshold, reset, slope,
                                 _lib.RULE_THRESHOLD, prec, side.cuda_stream, spikes=hs_b[i][:n], pre=pre_j, wt=wt,
                                 exact=True, budget=L0 * B * H, cur=shared)
                    ready[i].record(side)

            if recomputes:
                hidden_recompute(NS - 1)
            for k in range(NS - 1, -1, -1):
                t0 = k * S
                t1 = min(t0 + S, T)
                L = t1 - t0
                rows = L * B
                i = k % nset
                if recomputes:
                    if nset == 2:
                        if k > 0:
                            hidden_recompute(k - 1)  # one span ahead, on the side stream
                    elif k < NS - 1:
                        hidden_recompute(k)  # one buffer set: this span's, in turn
                    main.wait_event(ready[i])
                hs, pre_h = hs_b[i], pre_b[i]
                if whole_o:
                    if o_side:
                        main.wait_event(o_ready[k])
                    G_o = G_o_all[t0:t1]
                else:
                    s_in = words[t0:t1] if words is not None else hs[:L]
                    if pre_all is not None:
                        pre_k = pre_all[t0:t1]
                    else:
                        _readout_chunk(cur[:L], s_in, wo, bo, ck_o[k * per], None, pre_o[:L], None, None, None, T,
                                       t0, t1, C, decay, threshold, reset, slope, prec, stream, exact=True)
                        pre_k = pre_o
                    _lib.call(
                        "myelin_linear_pre_bwd",
                        _lib.ptr(pre_k), None, _lib.ptr(g_rates), _lib.ptr(gm_o), _lib.ptr(G_o), _lib.DT[G_o.dtype],
                        _lib.ptr(gbo_acc),
                        L, B * O, T, decay, threshold, reset, slope, sid, _lib.RULE_THRESHOLD, stream,
                    )
                    if gwo is not None:
                        # dW_o += S[t0:t1]^T @ G_o (S read as bits in the packed variant)
                        acc = k != NS - 1
                        cs = (gbo_acc, gbo) if k == 0 and gbo is not None else None
                        if words is not None:
                            _gemm(s_in, G_o, gwo, H, O, rows, s_in.shape[-1], O, O, True, False, acc, prec, stream,
                                  a_bits=True, col_sum=cs)
                        else:
                            _gemm(hs, G_o, gwo, H, O, rows, H, O, O, True, False, acc, prec, stream, col_sum=cs)
                if not need_hidden:
                    if nset == 2:
                        free[i].record(main)  # dW_o was the last reader of the spikes
                    continue
                g_dt = _lib.DT_BF16X3 if G_h is G3 else _lib.DT[G_h.dtype]
                if fused_ds:
                    # the hidden reverse pass with dS = G_o @ W_o^T formed in place
                    _lib.call(
                        "myelin_linear_pre_bwd_readout",
                        _lib.ptr(pre_h), _lib.ptr(G_o), _lib.ptr(wo), O, _lib.ptr(gm_h), _lib.ptr(G_h), g_dt,
                        _lib.ptr(gbh_acc), L, B, H, decay, threshold, reset, slope, sid, _lib.RULE_THRESHOLD, stream,
                    )
                else:
                    # dS[t0:t1] = G_o @ W_o^T, the hidden layer's spike gradient for this span
                    _gemm(G_o, wo, ghs, rows, H, O, O, O, H, False, True, False, prec, stream)
                    _lib.call(
                        "myelin_linear_pre_bwd",
                        _lib.ptr(pre_h), _lib.ptr(ghs), None, _lib.ptr(gm_h), _lib.ptr(G_h), g_dt,
                        _lib.ptr(gbh_acc),
                        L, B * H, T, decay, threshold, reset, slope, sid, _lib.RULE_THRESHOLD, stream,
                    )
                if nset == 2:
                    free[i].record(main)  # the trace's last reader (the spikes' was dW_o)
                if gx is not None:
                    _gemm(G_h, whg, gx[t0:t1], rows, F, H, H, H, F, False, True, False, prec, stream, ws=pool)
                if gwh is not None:
                    cs = (gbh_acc, gbh) if k == 0 and gbh is not None else None
                    if parts:
                        if G_h is not G3:
                            _lib.call("myelin_split_bf16x3", _lib.ptr(G_h), _lib.ptr(G3), rows, H, 0, stream)
                        _gemm_parts(xs[t0:t1], G3, 3, rows * H, gwh, F, H, rows, F, H, H, True, False, k != NS - 1,
                                    stream, ws=pool, col_sum=cs)
                    else:
                        _gemm(xs[t0:t1], G_h, gwh, F, H, rows, F, H, H, True, False, k != NS - 1, prec, stream,
                              ws=pool, col_sum=cs)
            if nset == 2:
                # every side-stream kernel is behind a ready[] the main stream
                # waited on; these tensors' last users include the side stream
                for t_ in (*hs_b, *pre_b, xs.x if lazy else xs, wh, ck_h, bh, wt):
                    if t_ is not None:
                        t_.record_stream(side)
            if o_side:
                readout_weight_grads()
            if gbh is not None and gwh is None:
                _lib.call("myelin_col_sum_f32", _lib.ptr(gbh_acc), _lib.ptr(gbh), B, H, 0, stream)
            if gbo is not None and gwo is None and not whole_o:
                _lib.call("myelin_col_sum_f32", _lib.ptr(gbo_acc), _lib.ptr(gbo), B, O, 0, stream)
        return gx, gwh, gbh, gwo, gbo, None, None, None, None, None, None, None, None, None


def two_layer_rate_forward(x, wh, bh, wo, bo, params, surrogate_id: int, slope: float, checkpoint: int,
                           precision: str, packed_hidden: bool, lean: bool = False):
    """Validate and run the chunk-interleaved two-layer rate network.
    ``lean``: the memory-lean policy (forward groups and backward spans of
    one checkpoint chunk; the split synapse casts the input per chunk)."""

    if checkpoint <= 0:
        raise ValueError("checkpoint_size must be positive")
    if x.ndim != 3:
        raise ValueError(f"inputs must be shaped [T, B, F]; got {tuple(x.shape)}")
    if wh.ndim != 2 or wo.ndim != 2:
        raise ValueError("hidden_weight and output_weight must be 2-D")
    _lib.require_device(x, "inputs")
    for name, t in (("hidden_weight", wh), ("hidden_bias", bh), ("output_weight", wo), ("output_bias", bo)):
        if t is not None and (t.device != x.device or t.dtype != x.dtype):
            raise ValueError(f"{name} must have the same device and dtype as inputs")
    if x.dtype != torch.float32:
        raise ValueError(f"inputs must be float32 for the HIP path; got {x.dtype}")
    if x.shape[0] == 0:
        raise ValueError("inputs must have at least one timestep")
    if x.shape[2] != wh.shape[0]:
        raise ValueError("inputs.shape[2] must match hidden_weight.shape[0]")
    if wh.shape[1] != wo.shape[0]:
        raise ValueError("hidden_weight.shape[1] must match output_weight.shape[0]")
    if bh is not None and bh.shape != (wh.shape[1],):
        raise ValueError("hidden_bias must be shaped [H]")
    if bo is not None and bo.shape != (wo.shape[1],):
        raise ValueError("output_bias must be shaped [O]")
    if precision not in _lib.PREC:
        raise ValueError("synapse_precision must be 'fp32' or 'bf16'")
    c = lambda t: None if t is None else t.contiguous()  # noqa: E731
    with torch.cuda.device(x.device):
        return HipTwoLayerRateFunction.apply(
            x.contiguous(), wh.contiguous(), c(bh), wo.contiguous(), c(bo), float(params.decay),
            float(params.threshold), float(params.reset), surrogate_id, float(slope), int(checkpoint),
            _lib.PREC[precision], packed_hidden, lean,
        )
