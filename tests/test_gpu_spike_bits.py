"""The packed twin of a layer's spike output: a layer that writes spikes
[T, B, N] also writes their packed bits, and a narrow (<= 32 neuron) layer
reading that tensor next streams the bits in its synapse GEMMs instead of
the fp32 spikes.  The bits hold the same 0/1 values and the GEMMs sum the
same products in the same order, so every output and gradient must equal
the fp32 path bit for bit; a tensor changed after it was written (its
version moved on) must not be read through stale bits.
"""

from __future__ import annotations

import pytest
import torch

import myelin_amd as myelin
from myelin_amd import linear as L
from tests.helpers import assert_same_bits, seeded

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _print_case(**kw):
    print("case:", " ".join(f"{k}={v}" for k, v in kw.items()), flush=True)


def _layers(F, H, O, prec, checkpoint, seed):
    torch.manual_seed(seed)
    hidden = myelin.LinearSurrogateLIF(F, H, surrogate=myelin.atan_surrogate, stream_synapse=True,
                                       synapse_precision=prec).to(DEV)
    readout = myelin.LinearSurrogateLIFRate(H, O, surrogate=myelin.atan_surrogate, checkpoint_size=checkpoint,
                                            synapse_precision=prec).to(DEV)
    # Kaiming-uniform weights (bound sqrt(6 / fan_in)), so both layers spike
    with torch.no_grad():
        for mod, fan in ((hidden, F), (readout, H)):
            mod.synapse.weight.uniform_(-(6.0 / fan) ** 0.5, (6.0 / fan) ** 0.5)
    return hidden, readout


# the 784 -> 2048 -> 10 bf16 network at T = 50, B = 256; a ragged hidden
# width (1000: the last packed word partial) at fp32; a checkpointed readout
# whose backward recomputes its currents from the bits
@pytest.mark.parametrize("T,B,F,H,O,prec,checkpoint", [
    (50, 256, 784, 2048, 10, "bf16", 25), (23, 64, 96, 1000, 7, "fp32", 23), (40, 32, 64, 128, 20, "fp32", 8)])
def test_readout_reads_the_packed_twin_bit_for_bit(T, B, F, H, O, prec, checkpoint):
    _print_case(test="spike_bits", T=T, B=B, F=F, H=H, O=O, prec=prec, checkpoint=checkpoint)
    g = seeded(T + B + F + H + O)
    x = (torch.rand(T, B, F, generator=g) < 0.2).float().to(DEV)
    labels = torch.randint(0, O, (B,), generator=g).to(DEV)
    hidden, readout = _layers(F, H, O, prec, checkpoint, seed=T * 3 + H)
    xin = x.clone().requires_grad_()

    def run(strip):
        for p in list(hidden.parameters()) + list(readout.parameters()):
            p.grad = None
        xin.grad = None
        h = hidden(xin)
        assert L._spike_bits(h) is not None
        if strip:
            # the same values in a tensor without a packed twin
            h = h * 1.0
            assert L._spike_bits(h) is None
        rates = readout(h)
        torch.nn.functional.cross_entropy(rates * T, labels).backward()
        torch.cuda.synchronize()
        return [rates.detach().clone(), xin.grad.clone()] + [p.grad.clone() for p in
                                                             list(hidden.parameters()) + list(readout.parameters())]

    with_bits, without = run(False), run(True)
    assert bool((with_bits[0] > 0).any())
    for i, (a, b) in enumerate(zip(with_bits, without)):
        assert_same_bits(a, b, f"output {i}")


def test_stale_twin_is_not_read():
    """An in-place change after the layer wrote the spikes bumps the tensor's
    version: the consumer must read the changed fp32 values."""

    _print_case(test="spike_bits_stale")
    T, B, F, H, O = 12, 64, 32, 256, 5
    g = seeded(7)
    x = (torch.rand(T, B, F, generator=g) < 0.3).float().to(DEV)
    hidden, readout = _layers(F, H, O, "fp32", T, seed=11)
    with torch.no_grad():
        h = hidden(x)
        assert L._spike_bits(h) is not None
        h[:, :, : H // 2] = 1.0 - h[:, :, : H // 2]
        assert L._spike_bits(h) is None
        got = readout(h)
        want = readout(h.clone())
    torch.cuda.synchronize()
    assert_same_bits(got, want, "rates after an in-place change")
