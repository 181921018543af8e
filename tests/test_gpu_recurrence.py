"""GPU parity of the fused-time LIF / ALIF kernels against the oracle.

Bars (written per assertion):
* plain lif_forward / alif_forward: spikes and states bit-identical to the
  reference torch path (oracle.torch_ref), any shape.
* surrogate paths in the fused kernels' own arithmetic (backend "hip" for
  ALIF, the default for LIF; the autograd-order arithmetic is tested in
  test_gpu_autograd_order): forward spikes and states bit-identical to the C oracle
  (exact 0/1 spikes); against the torch oracle (whose straight-through
  spike is (H + sigma) - sigma, 1 ulp below 1 for some spikes) rasters agree
  on >= 99.99 % of entries and states within 1e-5 (max-norm relative).
* gradients: within 1e-5 (max-norm relative) of the exact adjoint of the
  fp32 forward (oracle orc_adjoint_exact), and within TOL_VS_AUTOGRAD of
  torch.autograd through the reference unroll (see test_oracle_adjoint).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import myelin_amd as myelin
from oracle import c_ref
from oracle import torch_ref as R
from tests.helpers import assert_norm_close, raster_agreement, seeded, to_np
from tests.test_oracle_adjoint import TOL_VS_AUTOGRAD

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _print_case(**kw):
    print("case:", " ".join(f"{k}={v}" for k, v in kw.items()), flush=True)


# ---------------------------------------------------------------- plain LIF
def test_lif_forward_T100_B64_N1024_bit_exact():
    """LIF, hard reset, x ~ N(0.3, 0.5) [100, 64, 1024], beta=0.9 (tau 10), theta=1, v0=0."""

    _print_case(test="lif_T100_B64_N1024")
    g = seeded(1)
    x = 0.3 + 0.5 * torch.randn(100, 64, 1024, generator=g)
    m0 = torch.zeros(64, 1024)
    em, es = R.lif_unroll(x, m0, 10.0, 1.0, 0.0)
    st, s = myelin.lif_forward(x.to(DEV), myelin.LIFState(m0.to(DEV)), myelin.LIFParams(10.0, 1.0, 0.0))
    assert torch.equal(s.cpu(), es)
    assert torch.equal(st.membrane.cpu(), em)


@pytest.mark.parametrize("T,B,N", [(1, 1, 1), (7, 3, 5), (17, 2, 31), (9, 3, 32), (16, 1, 33), (33, 2, 65),
                                   (5, 4, 1023)])
def test_lif_forward_shapes_bit_exact(T, B, N):
    _print_case(test="lif_shapes", T=T, B=B, N=N)
    g = seeded(T * 1000 + B * 10 + N)
    x = torch.rand(T, B, N, generator=g)
    m0 = torch.rand(B, N, generator=g) * 0.2
    em, es = R.lif_unroll(x, m0, 8.0, 0.7, -0.25)
    st, s = myelin.lif_forward(x.to(DEV), myelin.LIFState(m0.to(DEV)), myelin.LIFParams(8.0, 0.7, -0.25))
    assert torch.equal(s.cpu(), es)
    assert torch.equal(st.membrane.cpu(), em)


def test_lif_forward_unaligned_view_takes_scalar_path():
    _print_case(test="lif_unaligned")
    g = seeded(3)
    base = torch.rand(6 * 2 * 17 + 1, generator=g)
    x = base[1:].view(6, 2, 17)  # storage offset 1: not 8-byte aligned
    m0 = torch.zeros(2, 17)
    em, es = R.lif_unroll(x, m0, 5.0, 0.5, 0.0)
    xd = base.to(DEV)[1:].view(6, 2, 17)
    st, s = myelin.lif_forward(xd, myelin.LIFState(m0.to(DEV)), myelin.LIFParams(5.0, 0.5, 0.0))
    assert torch.equal(s.cpu(), es) and torch.equal(st.membrane.cpu(), em)


def test_lif_forward_membrane_gradient_matches_autograd():
    _print_case(test="lif_grad_final")
    g = seeded(4)
    x = torch.rand(21, 3, 40, generator=g)
    m0 = torch.rand(3, 40, generator=g) * 0.2
    xr, mr = x.clone().requires_grad_(), m0.clone().requires_grad_()
    em, es = R.lif_unroll(xr, mr, 8.0, 0.7, -0.2)
    em.square().sum().backward()
    xd = x.to(DEV).requires_grad_()
    md = m0.to(DEV).requires_grad_()
    st, s = myelin.lif_forward(xd, myelin.LIFState(md), myelin.LIFParams(8.0, 0.7, -0.2))
    assert not s.requires_grad
    st.membrane.square().sum().backward()
    assert_norm_close(xd.grad.cpu(), xr.grad, 1e-6, "grad_x")
    assert_norm_close(md.grad.cpu(), mr.grad, 1e-6, "grad_m0")


def test_lif_forward_packed_matches_dense():
    for N in (1, 31, 32, 33, 65):
        _print_case(test="lif_packed", N=N)
        g = seeded(N)
        x = torch.rand(5, 2, N, generator=g)
        m0 = torch.rand(2, N, generator=g) * 0.2
        em, es = R.lif_unroll(x, m0, 10.0, 1.0, -0.25)
        st, pk = myelin.lif_forward_packed_spikes(x.to(DEV), myelin.LIFState(m0.to(DEV)),
                                                  myelin.LIFParams(10.0, 1.0, -0.25))
        words, _ = R.pack_spikes(es)
        assert torch.equal(pk.data.cpu(), words)
        assert pk.original_shape == (5, 2, N)
        assert torch.equal(st.membrane.cpu(), em)


# ---------------------------------------------------------------- plain ALIF
@pytest.mark.parametrize("T,B,N", [(1, 1, 1), (40, 3, 33), (100, 2, 257)])
def test_alif_forward_bit_exact(T, B, N):
    _print_case(test="alif_fwd", T=T, B=B, N=N)
    g = seeded(T + N)
    x = 0.25 + 0.6 * torch.randn(T, B, N, generator=g)
    m0 = 0.1 * torch.randn(B, N, generator=g)
    a0 = 0.2 * torch.rand(B, N, generator=g)
    p = myelin.ALIFParams(20.0, 50.0, 1.0, 0.0, 1.8)
    em, ea, es = R.alif_unroll(x, m0, a0, 20.0, 50.0, 1.0, 0.0, 1.8)
    st, s = myelin.alif_forward(x.to(DEV), myelin.ALIFState(m0.to(DEV), a0.to(DEV)), p)
    assert torch.equal(s.cpu(), es)
    assert torch.equal(st.membrane.cpu(), em)
    assert torch.equal(st.adaptation.cpu(), ea)


# ---------------------------------------------------------------- surrogate paths
def _check_grads_vs_oracles(surrogate, x, m0, a0, gs, gm, ga, hip_grads, alif, tau=20.0, tau_a=50.0,
                            thr=1.0, reset=0.0, beta=1.8, slope=10.0, autograd=True):
    d = np.float32(R.decay_from_tau(tau))
    rho = np.float32(R.decay_from_tau(tau_a))
    exact = c_ref.adjoint_exact(x.numpy(), m0.numpy(), None if a0 is None else a0.numpy(), gs.numpy(),
                                gm.numpy(), None if ga is None else ga.numpy(), d, rho, thr, beta, reset,
                                slope, surrogate, alif=alif)
    names = ["grad_x", "grad_m0", "grad_a0"][: len(hip_grads)]
    for name, h, e in zip(names, hip_grads, exact):
        assert_norm_close(to_np(h), e, 1e-5, f"{surrogate} {name} vs exact adjoint")
    if not autograd:
        return
    xr, mr = x.clone().requires_grad_(), m0.clone().requires_grad_()
    if alif:
        ar = a0.clone().requires_grad_()
        m, a, s = R.surrogate_alif_unroll(xr, mr, ar, tau, tau_a, thr, reset, beta, surrogate, slope)
        torch.autograd.backward([s, m, a], [gs, gm, ga])
        refs = [xr.grad, mr.grad, ar.grad]
    else:
        m, s = R.surrogate_lif_unroll(xr, mr, tau, thr, reset, surrogate, slope)
        torch.autograd.backward([s, m], [gs, gm])
        refs = [xr.grad, mr.grad]
    for name, h, r in zip(names, hip_grads, refs):
        assert_norm_close(to_np(h), r, TOL_VS_AUTOGRAD[surrogate], f"{surrogate} {name} vs autograd")


@pytest.mark.parametrize("surrogate", R.SURROGATE_NAMES)
@pytest.mark.parametrize("T,B,N", [(4, 2, 5), (37, 3, 67)])
def test_surrogate_lif_matches_oracles(surrogate, T, B, N):
    _print_case(test="surrogate_lif", surrogate=surrogate, T=T, B=B, N=N)
    g = seeded(42 + T)
    x = torch.rand(T, B, N, generator=g)
    m0 = torch.rand(B, N, generator=g) * 0.2
    gs = torch.randn(T, B, N, generator=g)
    gm = torch.randn(B, N, generator=g)
    xd, md = x.to(DEV).requires_grad_(), m0.to(DEV).requires_grad_()
    st, s = myelin.surrogate_lif_forward(xd, myelin.LIFState(md), myelin.LIFParams(8.0, 0.7, -0.2),
                                         surrogate=surrogate, surrogate_slope=4.0)
    torch.autograd.backward([s, st.membrane], [gs.to(DEV), gm.to(DEV)])
    cm, cs = c_ref.lif_fwd(x.numpy(), m0.numpy(), np.float32(R.decay_from_tau(8.0)), 0.7, -0.2, True, 4.0)
    assert np.array_equal(to_np(s), cs)
    assert np.array_equal(to_np(st.membrane), cm)
    em, es = R.surrogate_lif_unroll(x, m0, 8.0, 0.7, -0.2, surrogate, 4.0)
    assert raster_agreement(s, es) >= 0.9999
    assert_norm_close(st.membrane.detach(), em.detach(), 1e-5, "membrane")
    _check_grads_vs_oracles(surrogate, x, m0, None, gs, gm, None, [xd.grad, md.grad], alif=False, tau=8.0,
                            thr=0.7, reset=-0.2, beta=0.0, slope=4.0)


@pytest.mark.parametrize("surrogate", ["fast_sigmoid", "superspike", "atan"])
def test_closed_form_backward_of_huge_membrane(surrogate):
    """A membrane of 1e20 makes (1 + |c|)^2 overflow: sigma'(c) is 0 there,
    as in torch and the C oracle, not NaN; the other neuron is unaffected."""

    _print_case(test="closed_form_huge_membrane", surrogate=surrogate)
    x = torch.tensor([[[1e20, 0.5, 0.9]], [[0.0, 0.7, 0.2]], [[0.3, 0.1, 0.8]]])
    m0 = torch.zeros(1, 3)
    gs = torch.ones_like(x)
    xd = x.to(DEV).requires_grad_()
    _, s = myelin.surrogate_lif_forward(xd, myelin.LIFState(m0.to(DEV)), myelin.LIFParams(20.0, 1.0, 0.0),
                                        surrogate=surrogate, surrogate_slope=10.0)
    s.backward(gs.to(DEV))
    gx, _ = c_ref.lif_bwd(x.numpy(), m0.numpy(), gs.numpy(), np.zeros((1, 3), np.float32),
                          np.float32(R.decay_from_tau(20.0)), 1.0, 0.0, 10.0, surrogate)
    got = to_np(xd.grad)
    assert np.isfinite(got).all()
    assert got[0, 0, 0] == 0.0 and gx[0, 0, 0] == 0.0
    assert_norm_close(got, gx, 1e-6, "grad_x")


@pytest.mark.parametrize("surrogate", R.SURROGATE_NAMES)
@pytest.mark.parametrize("T,B,N", [(4, 2, 5), (50, 3, 129)])
def test_surrogate_alif_matches_oracles(surrogate, T, B, N):
    _print_case(test="surrogate_alif", surrogate=surrogate, T=T, B=B, N=N)
    g = seeded(7 + T)
    x = 0.25 + 0.6 * torch.randn(T, B, N, generator=g)
    m0 = 0.1 * torch.randn(B, N, generator=g)
    a0 = 0.2 * torch.rand(B, N, generator=g)
    gs = torch.randn(T, B, N, generator=g)
    gm = torch.randn(B, N, generator=g)
    ga = torch.randn(B, N, generator=g)
    xd, md, ad = (t.to(DEV).requires_grad_() for t in (x, m0, a0))
    p = myelin.ALIFParams(20.0, 50.0, 1.0, 0.0, 1.8)
    st, s = myelin.surrogate_alif_forward(xd, myelin.ALIFState(md, ad), p, surrogate=surrogate,
                                          surrogate_slope=10.0, backend="hip")
    torch.autograd.backward([s, st.membrane, st.adaptation], [gs.to(DEV), gm.to(DEV), ga.to(DEV)])
    cm, ca, cs = c_ref.alif_fwd(x.numpy(), m0.numpy(), a0.numpy(), np.float32(R.decay_from_tau(20.0)),
                                np.float32(R.decay_from_tau(50.0)), 1.0, 1.8, 0.0, True, 10.0)
    assert np.array_equal(to_np(s), cs)
    assert np.array_equal(to_np(st.membrane), cm) and np.array_equal(to_np(st.adaptation), ca)
    em, ea, es = R.surrogate_alif_unroll(x, m0, a0, 20.0, 50.0, 1.0, 0.0, 1.8, surrogate, 10.0)
    assert raster_agreement(s, es) >= 0.9999
    assert_norm_close(st.membrane.detach(), em.detach(), 1e-5, "membrane")
    assert_norm_close(st.adaptation.detach(), ea.detach(), 1e-5, "adaptation")
    _check_grads_vs_oracles(surrogate, x, m0, a0, gs, gm, ga, [xd.grad, md.grad, ad.grad], alif=True)


@pytest.mark.parametrize("T", [1, 15, 16, 17, 33, 48])
def test_surrogate_alif_chunk_edges(T):
    """Horizons around the 16-step recompute chunk."""

    _print_case(test="alif_chunk_edges", T=T)
    g = seeded(100 + T)
    x = 0.25 + 0.6 * torch.randn(T, 2, 70, generator=g)
    z = torch.zeros(2, 70)
    gs = torch.randn(T, 2, 70, generator=g)
    xd = x.to(DEV).requires_grad_()
    st, s = myelin.surrogate_alif_forward(xd, myelin.ALIFState(z.to(DEV), z.to(DEV)),
                                          myelin.ALIFParams(20.0, 50.0, 1.0, 0.0, 1.8), surrogate="fast_sigmoid",
                                          backend="hip")
    s.backward(gs.to(DEV))
    exact, _, _ = c_ref.adjoint_exact(x.numpy(), z.numpy(), z.numpy(), gs.numpy(), None, None,
                                      np.float32(0.95), np.float32(R.decay_from_tau(50.0)), 1.0, 1.8, 0.0, 10.0,
                                      "fast_sigmoid")
    assert_norm_close(to_np(xd.grad), exact, 1e-5, "grad_x")


def test_headline_alif_fast_sigmoid_full_size():
    """Closed-form arithmetic (backend="hip"):
    ALIF fwd + fast_sigmoid bwd at T=256, B=128, N=4096 (x ~ N(0.25, 0.6),
    gs ~ N(0, 1)).  Neurons are independent, so rows b in {0, 63, 127} are
    checked against the oracles; the whole output is checked for
    determinism and for 0/1 spikes."""

    _print_case(test="headline_full")
    T, B, N = 256, 128, 4096
    g = seeded(2)
    x = 0.25 + 0.6 * torch.randn(T, B, N, generator=g)
    gs = torch.randn(T, B, N, generator=g)
    z = torch.zeros(B, N)
    p = myelin.ALIFParams(20.0, 50.0, 1.0, 0.0, 1.8)
    xd = x.to(DEV).requires_grad_()
    gsd = gs.to(DEV)
    st, s = myelin.surrogate_alif_forward(xd, myelin.ALIFState(z.to(DEV), z.to(DEV)), p, surrogate="fast_sigmoid",
                                          backend="hip")
    s.backward(gsd)
    gx1 = xd.grad.clone()
    xd.grad = None
    st2, s2 = myelin.surrogate_alif_forward(xd, myelin.ALIFState(z.to(DEV), z.to(DEV)), p,
                                            surrogate="fast_sigmoid", backend="hip")
    s2.backward(gsd)
    assert torch.equal(s, s2) and torch.equal(gx1, xd.grad)
    assert bool(((s == 0) | (s == 1)).all())
    rows = [0, 63, 127]
    xs, gss = x[:, rows].contiguous(), gs[:, rows].contiguous()
    zs = torch.zeros(len(rows), N)
    cm, ca, cs = c_ref.alif_fwd(xs.numpy(), zs.numpy(), zs.numpy(), np.float32(0.95),
                                np.float32(R.decay_from_tau(50.0)), 1.0, 1.8, 0.0, True, 10.0)
    assert np.array_equal(to_np(s[:, rows]), cs)
    assert np.array_equal(to_np(st.membrane[rows]), cm) and np.array_equal(to_np(st.adaptation[rows]), ca)
    em, ea, es = R.surrogate_alif_unroll(xs, zs, zs, 20.0, 50.0, 1.0, 0.0, 1.8, "fast_sigmoid", 10.0)
    assert raster_agreement(s[:, rows], es) >= 0.9999
    exact, _, _ = c_ref.adjoint_exact(xs.numpy(), zs.numpy(), zs.numpy(), gss.numpy(), None, None,
                                      np.float32(0.95), np.float32(R.decay_from_tau(50.0)), 1.0, 1.8, 0.0, 10.0,
                                      "fast_sigmoid")
    assert_norm_close(to_np(gx1[:, rows]), exact, 1e-5, "grad_x vs exact adjoint")
    xr = xs.clone().requires_grad_()
    _, _, sr = R.surrogate_alif_unroll(xr, zs, zs, 20.0, 50.0, 1.0, 0.0, 1.8, "fast_sigmoid", 10.0)
    sr.backward(gss)
    assert_norm_close(to_np(gx1[:, rows]), xr.grad, TOL_VS_AUTOGRAD["fast_sigmoid"], "grad_x vs autograd")
