"""GPU tests of the module wrappers: cells, ``TimeUnroll``, ``LinearSynapse``
and training behaviour (the reference's tests/test_modules.py cases for the
hot-path modules: 21-120, 246-396, 936-1003).

Bars: plain LIF/ALIF rasters and membranes bit-exact against the oracle
(the recurrence is elementwise fp32).  Surrogate cells and TimeUnroll of
them run torch autograd's arithmetic (the reference steps the cell through
torch ops): spikes (including the straight-through value (H + sigma) -
sigma), states and gradients equal autograd's through the oracle for
fast_sigmoid; for atan (whose atan the kernels round from double) within
1e-5 max-norm relative and 3e-4 per element.  GEMM outputs within 1e-5 of
the fp32 CPU matmul (the MFMA sums in another order).
"""

from __future__ import annotations

import pytest
import torch

import myelin_amd as myelin
from oracle import torch_ref as R
from tests.helpers import assert_elementwise_close, assert_norm_close, assert_same_bits, raster_agreement, seeded, to_np

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _print_case(**kw):
    print("case:", " ".join(f"{k}={v}" for k, v in kw.items()), flush=True)


def _same_as_autograd(got, ref, sg, what):
    if sg == "fast_sigmoid":
        assert_same_bits(got, ref, what)
    else:
        assert_norm_close(to_np(got), ref, 1e-5, what)
        assert_elementwise_close(got, ref, 3e-4, what)


def test_linear_synapse_and_lif_unroll_match_functional_reference():
    """LinearSynapse then TimeUnroll(LIFCell) equals x @ W + b followed by
    the hard-reset LIF recurrence (test_modules.py:21-45)."""

    _print_case(test="synapse_lif_unroll")
    torch.manual_seed(3)
    syn = myelin.LinearSynapse(5, 7)
    with torch.no_grad():
        syn.weight.mul_(50.0)
        syn.bias.fill_(0.1)
    x = torch.rand(9, 4, 5, generator=seeded(4))
    syn = syn.to(DEV)
    cur = syn(x.to(DEV))
    ref_cur = x @ syn.weight.detach().cpu() + syn.bias.detach().cpu()
    assert_norm_close(to_np(cur), ref_cur, 1e-5, "synaptic current")
    p = myelin.LIFParams(tau_mem=6.0, threshold=0.4, reset=0.0)
    state, spikes = myelin.TimeUnroll(myelin.LIFCell(p))(cur)
    em, es = R.lif_unroll(cur.detach().cpu(), torch.zeros(4, 7), 6.0, 0.4, 0.0)
    assert torch.equal(spikes.cpu(), es)
    assert torch.equal(state.membrane.cpu(), em)
    assert 0 < float(es.sum()) < es.numel()


def test_linear_synapse_bias_can_be_disabled():
    _print_case(test="synapse_no_bias")
    syn = myelin.LinearSynapse(3, 4, bias=False).to(DEV)
    assert syn.bias is None
    x = torch.rand(2, 3, 3, generator=seeded(5))
    assert_norm_close(to_np(syn(x.to(DEV))), x @ syn.weight.detach().cpu(), 1e-5, "projection without bias")


@pytest.mark.parametrize("sg", ["atan", "fast_sigmoid"])
def test_surrogate_lif_cell_matches_functional_reference_with_reset(sg):
    """One surrogate LIF step from a nonzero state with a nonzero reset,
    forward and gradients (test_modules.py:246-276)."""

    _print_case(test="surrogate_lif_cell", sg=sg)
    g = seeded(6)
    x = torch.randn(5, 8, generator=g)
    m0 = torch.rand(5, 8, generator=g)
    p = myelin.LIFParams(tau_mem=4.0, threshold=0.5, reset=-0.3)
    fn = {"atan": myelin.atan_surrogate, "fast_sigmoid": myelin.fast_sigmoid_surrogate}[sg]
    cell = myelin.SurrogateLIFCell(p, surrogate=fn, surrogate_slope=4.0)
    xd, md = x.to(DEV).requires_grad_(), m0.to(DEV).requires_grad_()
    state, s = cell(myelin.LIFState(md), xd)
    (s.sum() * 2.0 + (state.membrane * torch.arange(8.0, device=DEV)).sum()).backward()
    xr, mr = x.clone().requires_grad_(), m0.clone().requires_grad_()
    em, es = R.surrogate_lif_unroll(xr.unsqueeze(0), mr, 4.0, 0.5, -0.3, sg, 4.0)
    (es[0].sum() * 2.0 + (em * torch.arange(8.0)).sum()).backward()
    assert raster_agreement(s, es[0]) >= 0.9999
    _same_as_autograd(s.detach(), es[0].detach(), sg, "spikes")
    _same_as_autograd(state.membrane.detach(), em.detach(), sg, "membrane")
    _same_as_autograd(xd.grad, xr.grad, sg, "grad_input")
    _same_as_autograd(md.grad, mr.grad, sg, "grad_initial_membrane")


def test_surrogate_alif_cell_matches_functional_reference_and_backpropagates():
    _print_case(test="surrogate_alif_cell")
    g = seeded(7)
    x = torch.randn(4, 6, generator=g) + 0.5
    m0, a0 = torch.rand(4, 6, generator=g), torch.rand(4, 6, generator=g)
    p = myelin.ALIFParams(tau_mem=10.0, tau_adaptation=30.0, threshold=0.8, reset=0.0, beta=1.5)
    cell = myelin.SurrogateALIFCell(p, surrogate=myelin.fast_sigmoid_surrogate, surrogate_slope=10.0)
    xd, md, ad = (t.to(DEV).requires_grad_() for t in (x, m0, a0))
    state, s = cell(myelin.ALIFState(md, ad), xd)
    (s.sum() + state.membrane.sum() + 0.5 * state.adaptation.sum()).backward()
    xr, mr, ar = (t.clone().requires_grad_() for t in (x, m0, a0))
    em, ea, es = R.surrogate_alif_unroll(xr.unsqueeze(0), mr, ar, 10.0, 30.0, 0.8, 0.0, 1.5, "fast_sigmoid", 10.0)
    (es[0].sum() + em.sum() + 0.5 * ea.sum()).backward()
    _same_as_autograd(s.detach(), es[0].detach(), "fast_sigmoid", "spikes")
    _same_as_autograd(state.membrane.detach(), em.detach(), "fast_sigmoid", "membrane")
    _same_as_autograd(state.adaptation.detach(), ea.detach(), "fast_sigmoid", "adaptation")
    for name, a, b in (("x", xd, xr), ("m0", md, mr), ("a0", ad, ar)):
        _same_as_autograd(a.grad, b.grad, "fast_sigmoid", f"grad_{name}")


@pytest.mark.parametrize("alif", [False, True])
def test_time_unroll_of_surrogate_cells_matches_reference(alif):
    """TimeUnroll runs the whole sequence in one fused launch; its zero
    initial state, spikes and input gradients match the oracle unroll."""

    _print_case(test="time_unroll_surrogate", alif=alif)
    T, B, N = 23, 3, 70
    g = seeded(8 + alif)
    x = torch.randn(T, B, N, generator=g) * 0.6 + 0.2
    gs = torch.randn(T, B, N, generator=g)
    xd = x.to(DEV).requires_grad_()
    xr = x.clone().requires_grad_()
    z = torch.zeros(B, N)
    if alif:
        p = myelin.ALIFParams(tau_mem=8.0, tau_adaptation=20.0, threshold=1.0, reset=0.0, beta=1.2)
        unroll = myelin.TimeUnroll(myelin.SurrogateALIFCell(p, surrogate=myelin.atan_surrogate))
        _, _, es = R.surrogate_alif_unroll(xr, z, z, 8.0, 20.0, 1.0, 0.0, 1.2, "atan", 10.0)
    else:
        p = myelin.LIFParams(tau_mem=8.0, threshold=1.0, reset=0.0)
        unroll = myelin.TimeUnroll(myelin.SurrogateLIFCell(p, surrogate=myelin.atan_surrogate))
        _, es = R.surrogate_lif_unroll(xr, z, 8.0, 1.0, 0.0, "atan", 10.0)
    _, s = unroll(xd)
    (s * gs.to(DEV)).sum().backward()
    (es * gs).sum().backward()
    assert raster_agreement(s, es) >= 0.9999
    _same_as_autograd(s.detach(), es.detach(), "atan", "spikes")
    _same_as_autograd(xd.grad, xr.grad, "atan", "grad_input")


def test_time_unroll_alif_cell_matches_reference():
    _print_case(test="time_unroll_alif")
    T, B, N = 31, 4, 33
    g = seeded(10)
    x = torch.randn(T, B, N, generator=g) * 0.5 + 0.3
    p = myelin.ALIFParams(tau_mem=12.0, tau_adaptation=40.0, threshold=1.0, reset=0.1, beta=0.8)
    state, s = myelin.TimeUnroll(myelin.ALIFCell(p))(x.to(DEV))
    z = torch.zeros(B, N)
    em, ea, es = R.alif_unroll(x, z, z, 12.0, 40.0, 1.0, 0.1, 0.8)
    assert torch.equal(s.cpu(), es)
    assert torch.equal(state.membrane.cpu(), em)
    assert torch.equal(state.adaptation.cpu(), ea)


def test_smooth_forward_cell_matches_functional_reference():
    """hard_forward=False: the spike is the smooth primitive itself
    (test_modules.py:348-366); fast_sigmoid's is IEEE-exact."""

    _print_case(test="smooth_forward_cell")
    g = seeded(12)
    x = torch.randn(3, 7, generator=g)
    m0 = torch.rand(3, 7, generator=g)
    cell = myelin.SurrogateLIFCell(myelin.LIFParams(5.0, 0.6, -0.1), surrogate=myelin.fast_sigmoid_surrogate,
                                   surrogate_slope=3.0, hard_forward=False)
    xd, md = x.to(DEV).requires_grad_(), m0.to(DEV).requires_grad_()
    state, s = cell(myelin.LIFState(md), xd)
    (s.square().sum() + state.membrane.sum()).backward()
    xr, mr = x.clone().requires_grad_(), m0.clone().requires_grad_()
    em, es = R.surrogate_lif_unroll(xr.unsqueeze(0), mr, 5.0, 0.6, -0.1, "fast_sigmoid", 3.0, hard_forward=False)
    (es[0].square().sum() + em.sum()).backward()
    assert bool(((s > 0) & (s < 1)).all()), "smooth spikes lie strictly inside (0, 1)"
    _same_as_autograd(s.detach(), es[0].detach(), "fast_sigmoid", "spikes")
    _same_as_autograd(state.membrane.detach(), em.detach(), "fast_sigmoid", "membrane")
    _same_as_autograd(xd.grad, xr.grad, "fast_sigmoid", "grad_input")
    _same_as_autograd(md.grad, mr.grad, "fast_sigmoid", "grad_initial_membrane")


def _spike_rate_loss(spikes, target):
    return (spikes.mean() - target).square()


def test_linear_surrogate_lif_training_step_updates_weight_and_reduces_loss():
    """SGD on a spike-rate loss moves the weight and lowers the loss
    (test_modules.py:936-963)."""

    _print_case(test="training_spike_rate")
    torch.manual_seed(0)
    layer = myelin.LinearSurrogateLIF(3, 6, surrogate=myelin.fast_sigmoid_surrogate).to(DEV)
    x = torch.rand(8, 4, 3, generator=seeded(11)).to(DEV)
    opt = torch.optim.SGD(layer.parameters(), lr=1.0)
    w0 = layer.synapse.weight.detach().clone()
    first = _spike_rate_loss(layer(x), 0.2).item()
    for _ in range(25):
        opt.zero_grad()
        _spike_rate_loss(layer(x), 0.2).backward()
        opt.step()
    assert not torch.equal(layer.synapse.weight.detach(), w0)
    assert _spike_rate_loss(layer(x), 0.2).item() < first


def test_rate_readout_classifier_returns_logits_and_trains():
    """Streamed hidden layer plus rate readout: [B, classes] logits, and a
    few Adam steps lower a tiny cross-entropy (test_modules.py:968-1003)."""

    _print_case(test="rate_readout_classifier")
    torch.manual_seed(24)
    x = torch.rand(8, 4, 3, generator=seeded(12)).to(DEV)
    targets = torch.tensor([0, 1, 0, 1], device=DEV)
    model = myelin.RateReadoutClassifier(3, 8, 2, surrogate=myelin.fast_sigmoid_surrogate, surrogate_slope=5.0,
                                         checkpoint_size=4).to(DEV)
    assert model(x).shape == (4, 2)
    ce = torch.nn.CrossEntropyLoss()
    opt = torch.optim.Adam(model.parameters(), lr=0.1)
    first = ce(model(x), targets).item()
    for _ in range(20):
        opt.zero_grad()
        ce(model(x), targets).backward()
        opt.step()
    assert ce(model(x), targets).item() < first
