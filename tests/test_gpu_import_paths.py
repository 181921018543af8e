"""Every drop-in entry point, imported through the reference's own paths
(`myelin.kernels`, `myelin.packing`, `myelin.modules`, reference
kernels.py:52-776, packing.py:45-162, modules.py:706-845), runs the HIP
kernels and agrees with the oracle on small seeded inputs.  Bars as in the
per-kernel tests: bit-exact spikes / states / words / counts / rates;
membranes and gradients 1e-5 (max-norm relative); the closed-form LIF
arithmetic (the default backend, as the reference's Triton route) against
autograd at 1e-4, the measured distance between the two evaluations."""

from __future__ import annotations

import pytest
import torch

from oracle import torch_ref as R
from tests.helpers import assert_norm_close, raster_agreement, seeded

pytestmark = pytest.mark.gpu
DEV = "cuda"


def test_kernels_through_reference_paths():
    from myelin.kernels import (alif_forward, lif_forward, linear_surrogate_lif_forward,
                                linear_surrogate_lif_packed_forward, linear_surrogate_lif_rate_forward,
                                surrogate_alif_forward, surrogate_lif_forward)
    from myelin.neurons import ALIFParams, ALIFState, LIFParams, LIFState
    from myelin.packing import pack_spikes

    print("case: import paths, kernels", flush=True)
    g = seeded(21)
    T, B, N, F = 19, 3, 70, 33
    x = 0.25 + 0.6 * torch.randn(T, B, N, generator=g)
    z = torch.zeros(B, N)
    xd, zd = x.to(DEV), z.to(DEV)

    st, s = lif_forward(xd, LIFState(zd), LIFParams(10.0, 1.0, 0.0))
    em, es = R.lif_unroll(x, z, 10.0, 1.0, 0.0)
    assert torch.equal(s.cpu(), es) and torch.equal(st.membrane.cpu(), em)

    st, s = alif_forward(xd, ALIFState(zd, zd), ALIFParams(20.0, 50.0, 1.0, 0.0, 1.8))
    em, ea, es = R.alif_unroll(x, z, z, 20.0, 50.0, 1.0, 0.0, 1.8)
    assert torch.equal(s.cpu(), es) and torch.equal(st.membrane.cpu(), em) and torch.equal(st.adaptation.cpu(), ea)

    gs = torch.randn(T, B, N, generator=g)
    xg = xd.clone().requires_grad_()
    _, s = surrogate_lif_forward(xg, LIFState(zd), LIFParams(20.0, 1.0, 0.0), surrogate="atan")
    s.backward(gs.to(DEV))
    xr = x.clone().requires_grad_()
    _, sr = R.surrogate_lif_unroll(xr, z, 20.0, 1.0, 0.0, "atan", 10.0)
    sr.backward(gs)
    assert raster_agreement(s, sr) >= 0.9999
    assert_norm_close(xg.grad.cpu(), xr.grad, 1e-4, "surrogate lif grad_x (closed form)")
    xg = xd.clone().requires_grad_()
    _, s = surrogate_lif_forward(xg, LIFState(zd), LIFParams(20.0, 1.0, 0.0), surrogate="atan", backend="torch")
    s.backward(gs.to(DEV))
    assert_norm_close(s.detach().cpu(), sr.detach(), 1e-5, "surrogate lif spikes (autograd order)")
    assert_norm_close(xg.grad.cpu(), xr.grad, 1e-5, "surrogate lif grad_x (autograd order)")

    xg = xd.clone().requires_grad_()
    _, s = surrogate_alif_forward(xg, ALIFState(zd, zd), ALIFParams(20.0, 50.0, 1.0, 0.0, 1.8),
                                  surrogate="fast_sigmoid", surrogate_slope=10.0)
    s.backward(gs.to(DEV))
    xr = x.clone().requires_grad_()
    _, _, sr = R.surrogate_alif_unroll(xr, z, z, 20.0, 50.0, 1.0, 0.0, 1.8, "fast_sigmoid", 10.0)
    sr.backward(gs)
    # the default ALIF arithmetic is autograd's: same spikes and gradient
    assert torch.equal(s.detach().cpu(), sr.detach())
    assert torch.equal(xg.grad.cpu(), xr.grad)

    xs = (torch.rand(T, B, F, generator=g) < 0.3).float()
    w = (torch.rand(F, N, generator=g) - 0.5) * 0.6
    p = LIFParams(9.0, 0.7, -0.2)
    xsd, wd = xs.to(DEV).requires_grad_(), w.to(DEV).requires_grad_()
    st, s = linear_surrogate_lif_forward(xsd, wd, None, p, surrogate="fast_sigmoid", surrogate_slope=5.0)
    s.backward(gs.to(DEV))
    xsr, wr = xs.clone().requires_grad_(), w.clone().requires_grad_()
    mr, sr = R.linear_surrogate_lif_stream(xsr, wr, None, 9.0, 0.7, -0.2, "fast_sigmoid", 5.0)
    sr.backward(gs)
    assert raster_agreement(s, sr) >= 0.9999
    assert_norm_close(st.membrane.detach().cpu(), mr.detach(), 1e-5, "linear membrane")
    assert_norm_close(xsd.grad.cpu(), xsr.grad, 1e-5, "linear grad_x")
    assert_norm_close(wd.grad.cpu(), wr.grad, 1e-5, "linear grad_w")

    _, r = linear_surrogate_lif_rate_forward(xs.to(DEV), w.to(DEV), None, p, surrogate="superspike",
                                             surrogate_slope=5.0, checkpoint_size=4, reduction="none")
    _, rr = R.linear_surrogate_lif_rate(xs, w, None, 9.0, 0.7, -0.2, "superspike", 5.0, 4, reduction="none")
    assert torch.equal(r.cpu(), rr)

    _, pk = linear_surrogate_lif_packed_forward(xs.to(DEV), w.to(DEV), None, p, surrogate="fast_sigmoid",
                                                surrogate_slope=5.0, checkpoint_size=4)
    _, dense = linear_surrogate_lif_forward(xs.to(DEV), w.to(DEV), None, p, surrogate="fast_sigmoid",
                                            surrogate_slope=5.0, checkpoint_size=4)
    assert torch.equal(pk.data, pack_spikes(dense).data)


def test_packing_through_reference_paths():
    from myelin.packing import (pack_spikes, packed_spike_count, packed_spike_counts, packed_spike_rate,
                                unpack_spikes)

    print("case: import paths, packing", flush=True)
    g = seeded(22)
    s = (torch.rand(13, 4, 75, generator=g) < 0.2).float()
    pk = pack_spikes(s.to(DEV))
    words, shape = R.pack_spikes(s)
    assert torch.equal(pk.data.cpu(), words)
    assert torch.equal(unpack_spikes(pk).cpu(), s)
    assert torch.equal(packed_spike_counts(pk).cpu(), R.packed_spike_counts(words, shape))
    for dim in (0, -1, (0, -1), None):
        assert torch.equal(packed_spike_count(pk, dim=dim).cpu(), R.packed_spike_count(words, shape, dim)), dim
        assert torch.equal(packed_spike_rate(pk, dim=dim).cpu(), R.packed_spike_rate(words, shape, dim)), dim


def test_modules_through_reference_paths():
    from myelin.modules import LinearSurrogateLIF, LinearSurrogateLIFRate

    print("case: import paths, modules", flush=True)
    g = seeded(23)
    T, B, F, H, O = 12, 4, 40, 64, 10
    x = (torch.rand(T, B, F, generator=g) < 0.3).float()
    torch.manual_seed(23)
    hidden = LinearSurrogateLIF(F, H, stream_synapse=True, checkpoint_size=5)
    readout = LinearSurrogateLIFRate(H, O, checkpoint_size=5)
    with torch.no_grad():
        hidden.synapse.weight.mul_(20.0)
        readout.synapse.weight.mul_(20.0)
    wh, wo = hidden.synapse.weight.detach().clone(), readout.synapse.weight.detach().clone()
    hidden.to(DEV)
    readout.to(DEV)
    rates = readout(hidden(x.to(DEV)))
    rates.sum().backward()
    xr = x.clone()
    whr, wor = wh.clone().requires_grad_(), wo.clone().requires_grad_()
    _, hs = R.linear_surrogate_lif_checkpoint(xr, whr, torch.zeros(H), 20.0, 1.0, 0.0, "atan", 10.0, 5)
    _, rr = R.linear_surrogate_lif_rate(hs, wor, torch.zeros(O), 20.0, 1.0, 0.0, "atan", 10.0, 5, reduction="none")
    rr.sum().backward()
    assert torch.equal(rates.detach().cpu(), rr.detach())
    assert_norm_close(hidden.synapse.weight.grad.cpu(), whr.grad, 1e-5, "hidden grad_w")
    assert_norm_close(readout.synapse.weight.grad.cpu(), wor.grad, 1e-5, "readout grad_w")
