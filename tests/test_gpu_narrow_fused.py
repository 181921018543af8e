"""The one-launch narrow layer over packed spikes
(myelin_linear_lif_fwd_narrow_bits): currents and recurrence in one kernel
per batch row.  It sums the same products in the same K splits and order as
the narrow GEMM with its split-K reduce, so every output must equal the
GEMM + recurrence launches it replaces bit for bit, on ragged widths, split
counts 1 to 8, several 64-step chunks, partial time ranges and both
precisions; and a network whose readout takes it must train bit for bit as
with the launches.
"""

from __future__ import annotations

import pytest
import torch

import myelin_amd as myelin
from myelin_amd import _lib
from myelin_amd import linear as L
from tests.helpers import assert_same_bits, seeded

pytestmark = pytest.mark.gpu
DEV = "cuda"
THR, SUR = _lib.RULE_THRESHOLD, _lib.RULE_SURROGATE


def _print_case(**kw):
    print("case:", " ".join(f"{k}={v}" for k, v in kw.items()), flush=True)


def _words(x):
    T, B, F = x.shape
    wx = -(-F // 32)
    words = torch.empty((T, B, wx), dtype=torch.int32, device=DEV)
    _lib.call("myelin_pack", _lib.ptr(x), _lib.DT[torch.float32], _lib.ptr(words), T * B, F,
              _lib.stream(x.device))
    return words


def _outputs(T, B, N, t0, t1, rates):
    return dict(m_final=torch.full((B, N), float("nan"), device=DEV),
                spikes=torch.full((T, B, N), float("nan"), device=DEV),
                pre=torch.full((t1 - t0, B, N), float("nan"), device=DEV),
                rates=torch.full((B, N), float("nan"), device=DEV) if rates else None)


# (T, B, F, N, precision, rule, bias, m0, [t0, t1)): the 2048 -> 10 bf16
# readout at T = 50, B = 256 (4 K splits); 784 wide (2 splits of 448, the
# last step past F); 100 wide (unsplit) over five 64-step chunks; 33 wide
# with one neuron over a partial range from a start state; 4096 wide (8
# splits), surrogate rule; 2048 wide at fp32 (three W planes, 4 splits)
CASES = [
    (50, 256, 2048, 10, "bf16", THR, True, False, None),
    (50, 130, 784, 7, "fp32", THR, True, False, None),
    (300, 128, 100, 32, "fp32", SUR, False, False, None),
    (150, 129, 33, 1, "bf16", THR, True, True, (20, 140)),
    (64, 200, 4096, 4, "bf16", SUR, True, True, None),
    (70, 160, 2048, 5, "fp32", THR, True, False, None),
]


@pytest.mark.parametrize("T,B,F,N,prec,rule,has_bias,has_m0,rng", CASES)
def test_one_launch_equals_gemm_and_recurrence(T, B, F, N, prec, rule, has_bias, has_m0, rng):
    _print_case(test="narrow_fused", T=T, B=B, F=F, N=N, prec=prec, rule=rule, bias=has_bias, m0=has_m0, rng=rng)
    g = seeded(T * 7 + B + F + N)
    x = (torch.rand(T, B, F, generator=g) < 0.2).float().to(DEV)
    w = ((torch.rand(F, N, generator=g) * 2 - 1) * (6.0 / F) ** 0.5).to(DEV)
    bias = (torch.randn(N, generator=g) * 0.1).to(DEV) if has_bias else None
    m0 = (torch.rand(B, N, generator=g) * 0.5).to(DEV) if has_m0 else None
    t0, t1 = rng if rng is not None else (0, T)
    whole = (t0, t1) == (0, T)
    words = _words(x)
    decay, thr, reset, slope = 0.9, 0.3, 0.0, 10.0
    p = _lib.PREC[prec]
    stream = _lib.stream(x.device)

    # the launches it replaces: the narrow GEMM over the bits (split-K and
    # its reduce), then the recurrence over the currents
    ref = _outputs(T, B, N, t0, t1, whole)
    cur = torch.empty((t1 - t0, B, N), device=DEV)
    L._gemm(words[t0:t1], w, cur, (t1 - t0) * B, N, F, words.shape[2], N, N, False, False, False, p, stream,
            bias=bias, a_bits=True, split=True)
    _lib.call("myelin_lif_currents_fwd", _lib.ptr(cur), _lib.ptr(m0), _lib.ptr(ref["m_final"]),
              _lib.ptr(ref["spikes"]), _lib.ptr(ref["pre"]), None, _lib.ptr(ref["rates"]), None, None, T, B, N, t0,
              t1, t0, t0, 1, decay, thr, reset, slope, rule, stream)

    out = _outputs(T, B, N, t0, t1, whole)
    _lib.call("myelin_linear_lif_fwd_narrow_bits", _lib.ptr(words), _lib.ptr(w), _lib.ptr(bias), _lib.ptr(m0),
              _lib.ptr(out["m_final"]), _lib.ptr(out["spikes"]), _lib.ptr(out["pre"]), _lib.ptr(out["rates"]), T, B,
              F, N, t0, t1, decay, thr, reset, slope, rule, p, stream)
    torch.cuda.synchronize()
    # steps outside [t0, t1) are not written: compare the range
    assert_same_bits(out["spikes"][t0:t1], ref["spikes"][t0:t1], "spikes")
    assert_same_bits(out["pre"], ref["pre"], "pre-reset trace")
    assert_same_bits(out["m_final"], ref["m_final"], "final membrane")
    if whole:
        assert_same_bits(out["rates"], ref["rates"], "rates")
    spiked = ref["spikes"][t0:t1].mean().item()
    assert 0.005 < spiked < 0.995, f"degenerate raster (spike fraction {spiked:.3f})"


def test_unsplit_and_split_rows_sum_alike():
    """A row's currents do not depend on which 32-row block or chunk holds
    it: the first 64 steps of a 300-step run equal a 64-step run."""

    _print_case(test="narrow_fused_rows")
    g = seeded(11)
    T, B, F, N = 300, 128, 1500, 12
    x = (torch.rand(T, B, F, generator=g) < 0.3).float().to(DEV)
    w = ((torch.rand(F, N, generator=g) * 2 - 1) * 0.05).to(DEV)
    words = _words(x)
    stream = _lib.stream(x.device)
    outs = []
    for t1 in (T, 64):
        pre = torch.empty((t1, B, N), device=DEV)
        _lib.call("myelin_linear_lif_fwd_narrow_bits", _lib.ptr(words), _lib.ptr(w), None, None, None, None,
                  _lib.ptr(pre), None, T, B, F, N, 0, t1, 0.0, 1e30, 0.0, 10.0, THR, 0, stream)
        outs.append(pre)
    torch.cuda.synchronize()
    # decay 0 and no spikes: the trace is the currents
    assert_same_bits(outs[0][:64], outs[1], "currents of the first 64 steps")


@pytest.mark.parametrize("prec,O", [("bf16", 10), ("fp32", 5)])
def test_network_trains_alike_with_and_without_the_one_launch_readout(prec, O, monkeypatch):
    """784 -> 2048 -> O at T = 50, B = 256 (the readout reads the hidden
    spikes' packed twin): outputs and every gradient equal with the
    readout's forward as one launch and as GEMM + reduce + recurrence."""

    _print_case(test="narrow_fused_network", prec=prec, O=O)
    T, B, F, H = 50, 256, 784, 2048
    g = seeded(5)
    x = (torch.rand(T, B, F, generator=g) < 0.2).float().to(DEV)
    labels = torch.randint(0, O, (B,), generator=g).to(DEV)
    torch.manual_seed(5)
    hidden = myelin.LinearSurrogateLIF(F, H, surrogate=myelin.atan_surrogate, stream_synapse=True,
                                       synapse_precision=prec).to(DEV)
    readout = myelin.LinearSurrogateLIFRate(H, O, surrogate=myelin.atan_surrogate, checkpoint_size=25,
                                            synapse_precision=prec).to(DEV)
    with torch.no_grad():
        for mod, fan in ((hidden, F), (readout, H)):
            mod.synapse.weight.uniform_(-(6.0 / fan) ** 0.5, (6.0 / fan) ** 0.5)
    params = list(hidden.parameters()) + list(readout.parameters())
    calls = []
    real_call = _lib.call

    def counting_call(name, *args):
        calls.append(name)
        return real_call(name, *args)

    monkeypatch.setattr(_lib, "call", counting_call)

    def run(min_b):
        monkeypatch.setattr(L, "_NARROW_FUSED_MIN_B", min_b)
        calls.clear()
        for q in params:
            q.grad = None
        rates = readout(hidden(x))
        torch.nn.functional.cross_entropy(rates * T, labels).backward()
        torch.cuda.synchronize()
        return rates.detach().clone(), [q.grad.clone() for q in params], list(calls)

    fused, fused_grads, fused_calls = run(128)
    plain, plain_grads, plain_calls = run(1 << 40)
    assert "myelin_linear_lif_fwd_narrow_bits" in fused_calls
    assert "myelin_linear_lif_fwd_narrow_bits" not in plain_calls
    assert_same_bits(fused, plain, "rates")
    for i, (a, b) in enumerate(zip(fused_grads, plain_grads)):
        assert_same_bits(a, b, f"gradient {i}")
