"""The oracle against golden vectors recorded from the reference itself
(tests/golden/make_golden.py).  The oracle restates the same ATen ops in
the same order, so forward values and gradients must be bit-identical."""

from __future__ import annotations

import itertools
import pathlib

import numpy as np
import pytest
import torch

from oracle import torch_ref as R

G = pathlib.Path(__file__).parent / "golden"


def _load(name):
    return dict(np.load(G / name))


PACK = _load("packing_counts.npz")
UNR = _load("surrogate_unrolls.npz")
LIN = _load("linear_paths.npz")
TWO = _load("two_layer_rate.npz")


@pytest.mark.parametrize("i", [0, 1, 2])
def test_packing_counts_every_dim_bitwise(i):
    s = torch.from_numpy(PACK[f"s{i}"])
    words, shape = R.pack_spikes(s)
    assert np.array_equal(words.numpy(), PACK[f"words{i}"])
    assert np.array_equal(R.unpack_spikes(words, shape).numpy(), PACK[f"unpack{i}"])
    nd = len(shape)
    dims_list = [None] + [d for r in range(1, nd + 1) for d in itertools.combinations(range(nd), r)]
    for dims in dims_list:
        tag = "none" if dims is None else "_".join(map(str, dims))
        c = R.packed_spike_count(words, shape, dims)
        assert c.dtype == torch.int64
        assert np.array_equal(c.numpy(), PACK[f"count{i}_{tag}"]), dims
        assert np.array_equal(R.packed_spike_rate(words, shape, dims).numpy(), PACK[f"rate{i}_{tag}"]), dims
        assert np.array_equal(R.packed_spike_rate(words, shape, dims, torch.float64).numpy(),
                              PACK[f"rate64{i}_{tag}"]), dims
        if f"counts{i}_{tag}" in PACK:
            assert np.array_equal(R.packed_spike_counts(words, shape, dims).numpy(), PACK[f"counts{i}_{tag}"])


@pytest.mark.parametrize("name", R.SURROGATE_NAMES)
def test_surrogate_unrolls_bitwise(name):
    x, m0, a0, gs, gm, ga = (torch.from_numpy(UNR[k]) for k in ("x", "m0", "a0", "gs", "gm", "ga"))
    xr, mr, ar = (t.clone().requires_grad_() for t in (x, m0, a0))
    m, a, s = R.surrogate_alif_unroll(xr, mr, ar, 20.0, 50.0, 1.0, 0.0, 1.8, name, 10.0)
    torch.autograd.backward([s, m, a], [gs, gm, ga])
    for k, v in dict(s=s, mT=m, aT=a, gx=xr.grad, gm0=mr.grad, ga0=ar.grad).items():
        assert np.array_equal(v.detach().numpy(), UNR[f"alif_{name}_{k}"]), k
    xr, mr = x.clone().requires_grad_(), m0.clone().requires_grad_()
    m, s = R.surrogate_lif_unroll(xr, mr, 8.0, 0.7, -0.2, name, 4.0)
    torch.autograd.backward([s, m], [gs, gm])
    for k, v in dict(s=s, mT=m, gx=xr.grad, gm0=mr.grad).items():
        assert np.array_equal(v.detach().numpy(), UNR[f"lif_{name}_{k}"]), k


@pytest.mark.parametrize("bias", [False, True])
@pytest.mark.parametrize("ck", [None, 1, 4, 9])
@pytest.mark.parametrize("with_final", [False, True])
def test_linear_spike_paths_bitwise(bias, ck, with_final):
    x, w, b, gs, gfin = (torch.from_numpy(LIN[k]) for k in ("x", "w", "b", "gs", "gfin"))
    xr, wr = x.clone().requires_grad_(), w.clone().requires_grad_()
    br = b.clone().requires_grad_() if bias else None
    if ck is None:
        m, s = R.linear_surrogate_lif_stream(xr, wr, br, 9.0, 0.7, -0.2, "atan", 5.0)
    else:
        m, s = R.linear_surrogate_lif_checkpoint(xr, wr, br, 9.0, 0.7, -0.2, "atan", 5.0, ck)
    outs, grads = [s], [gs]
    if with_final:
        outs.append(m)
        grads.append(gfin)
    torch.autograd.backward(outs, grads)
    tag = f"spk_{'b' if bias else 'nob'}_c{ck}_f{int(with_final)}"
    assert np.array_equal(s.detach().numpy(), LIN[f"{tag}_s"])
    assert np.array_equal(m.detach().numpy(), LIN[f"{tag}_mT"])
    assert np.array_equal(xr.grad.numpy(), LIN[f"{tag}_gx"])
    assert np.array_equal(wr.grad.numpy(), LIN[f"{tag}_gw"])
    if bias:
        assert np.array_equal(br.grad.numpy(), LIN[f"{tag}_gb"])


@pytest.mark.parametrize("bias", [False, True])
@pytest.mark.parametrize("ck", [1, 4, 9])
@pytest.mark.parametrize("red", ["none", "mean"])
def test_linear_rate_paths_bitwise(bias, ck, red):
    x, w, b, grate = (torch.from_numpy(LIN[k]) for k in ("x", "w", "b", "grate"))
    xr, wr = x.clone().requires_grad_(), w.clone().requires_grad_()
    br = b.clone().requires_grad_() if bias else None
    m, r = R.linear_surrogate_lif_rate(xr, wr, br, 9.0, 0.7, -0.2, "superspike", 5.0, ck, reduction=red)
    if red == "none":
        r.backward(grate)
    else:
        r.backward()
    tag = f"rate_{'b' if bias else 'nob'}_c{ck}_{red}"
    assert np.array_equal(r.detach().numpy(), LIN[f"{tag}_r"])
    assert np.array_equal(m.detach().numpy(), LIN[f"{tag}_mT"])
    assert np.array_equal(xr.grad.numpy(), LIN[f"{tag}_gx"])
    assert np.array_equal(wr.grad.numpy(), LIN[f"{tag}_gw"])
    if bias:
        assert np.array_equal(br.grad.numpy(), LIN[f"{tag}_gb"])


@pytest.mark.parametrize("bias", [False, True])
@pytest.mark.parametrize("ck", [1, 4, 11])
@pytest.mark.parametrize("sg", ["fast_sigmoid", "superspike"])
def test_two_layer_rate_bitwise(bias, ck, sg):
    x, wh, bh, wo, bo, grate = (torch.from_numpy(TWO[k]) for k in ("x", "wh", "bh", "wo", "bo", "grate"))
    xr, whr, wor = (t.clone().requires_grad_() for t in (x, wh, wo))
    bhr = bh.clone().requires_grad_() if bias else None
    bor = bo.clone().requires_grad_() if bias else None
    r = R.two_layer_rate(xr, whr, bhr, wor, bor, 6.0, 0.6, -0.1, sg, 5.0, ck)
    r.backward(grate)
    tag = f"{'b' if bias else 'nob'}_c{ck}_{sg}"
    assert np.array_equal(r.detach().numpy(), TWO[f"{tag}_r"])
    for k, v in dict(gx=xr.grad, gwh=whr.grad, gwo=wor.grad).items():
        assert np.array_equal(v.numpy(), TWO[f"{tag}_{k}"]), k
    if bias:
        assert np.array_equal(bhr.grad.numpy(), TWO[f"{tag}_gbh"])
        assert np.array_equal(bor.grad.numpy(), TWO[f"{tag}_gbo"])
