"""GPU parity of the two-layer LIF rate network (whole-model recompute and
packed-hidden variants, kernels.py:779-846).

Bars (as for the one-layer linear paths): readout rates equal to the
reference's when the rasters agree (rates are counts / T), gradients within
1e-5 max-norm relative of the reference's and of the oracle's (measured <=
1.4e-6) and, against the reference's golden vectors, per element within
2e-4, |a - b| <= 2e-4 * max(|b|, 1e-3 max|b|), or no farther from the
float64 evaluation of the same network than the golden value is (the MFMA
GEMMs sum in another order than the CPU matmul, and the reference's spikes
(H + sigma) - sigma can sit an ulp below 1).  The packed
variant's readout GEMMs read the hidden spikes as packed bits; for readouts
narrower than 128 neurons both variants run the same GEMM kernel and K
split, so they must agree bit for bit (wider: within 1e-5).
"""

from __future__ import annotations

import pathlib

import numpy as np
import pytest
import torch

import myelin_amd as myelin
from oracle import torch_ref as R
from tests.helpers import (assert_elementwise_close_or_truer, assert_norm_close, f32_params, raster_agreement, seeded,
                           to_np)

pytestmark = pytest.mark.gpu
DEV = "cuda"
TWO = dict(np.load(pathlib.Path(__file__).parent / "golden" / "two_layer_rate.npz"))
VARIANTS = {
    "recompute": myelin.two_layer_surrogate_lif_rate_recompute_forward,
    "packed": myelin.two_layer_surrogate_lif_rate_packed_hidden_forward,
}


def _print_case(**kw):
    print("case:", " ".join(f"{k}={v}" for k, v in kw.items()), flush=True)


def _run(fn, tensors, bias, params, **kw):
    x, wh, bh, wo, bo = (t.to(DEV).requires_grad_() if t is not None else None for t in tensors)
    if not bias:
        bh = bo = None
    r = fn(x, wh, bh, wo, bo, params, **kw)
    return r, (x, wh, bh, wo, bo)


def _grads(leaves):
    return [None if t is None else to_np(t.grad) for t in leaves]


@pytest.mark.parametrize("variant", sorted(VARIANTS))
@pytest.mark.parametrize("bias", [False, True])
@pytest.mark.parametrize("ck", [1, 4, 11])
@pytest.mark.parametrize("sg", ["fast_sigmoid", "superspike"])
def test_two_layer_matches_reference(variant, bias, ck, sg):
    _print_case(test="two_layer_golden", variant=variant, bias=bias, ck=ck, sg=sg)
    tensors = [torch.from_numpy(TWO[k]) for k in ("x", "wh", "bh", "wo", "bo")]
    grate = torch.from_numpy(TWO["grate"]).to(DEV)
    p = myelin.LIFParams(tau_mem=6.0, threshold=0.6, reset=-0.1)
    r, leaves = _run(VARIANTS[variant], tensors, bias, p, surrogate=sg, surrogate_slope=5.0, checkpoint_size=ck)
    r.backward(grate)
    tag = f"{'b' if bias else 'nob'}_c{ck}_{sg}"
    assert np.array_equal(to_np(r), TWO[f"{tag}_r"])
    gx, gwh, gbh, gwo, gbo = _grads(leaves)
    truth = _truth64(tensors, bias, p, sg, ck, TWO["grate"], TWO[f"{tag}_r"])
    pairs = [(gx, "gx"), (gwh, "gwh"), (gwo, "gwo")] + ([(gbh, "gbh"), (gbo, "gbo")] if bias else [])
    for got, name in pairs:
        assert_norm_close(got, TWO[f"{tag}_{name}"], 1e-5, name)
        assert_elementwise_close_or_truer(got, TWO[f"{tag}_{name}"], truth[name], 2e-4, name)


def _truth64(tensors, bias, p, sg, ck, grate, rates):
    """The oracle network in float64 on the golden inputs (every scalar at
    its fp32 value); its rates must equal the golden ones."""

    x, wh, bh, wo, bo = (t.double().requires_grad_() for t in tensors)
    if not bias:
        bh = bo = None
    tau, thr, rst = f32_params(p.tau_mem, p.threshold, p.reset)
    r = R.two_layer_rate(x, wh, bh, wo, bo, tau, thr, rst, sg, 5.0, ck)
    assert np.array_equal(to_np(r.float()), rates), "float64 rates differ from the golden ones"
    r.backward(torch.from_numpy(grate).double())
    return {"gx": x.grad, "gwh": wh.grad, "gwo": wo.grad, "gbh": None if bh is None else bh.grad,
            "gbo": None if bo is None else bo.grad}


def _random_net(seed, T, B, F, H, O):
    g = seeded(seed)
    x = (torch.rand(T, B, F, generator=g) < 0.3).float()
    wh = (torch.rand(F, H, generator=g) - 0.4) * (2.0 / F ** 0.5)
    bh = torch.rand(H, generator=g) * 0.05
    wo = (torch.rand(H, O, generator=g) - 0.45) * (3.0 / H ** 0.5)
    bo = torch.rand(O, generator=g) * 0.05
    grate = torch.randn(B, O, generator=g)
    return [x, wh, bh, wo, bo], grate


# (T, B, F, H, O): ragged word edges, a hidden layer on the fused kernel
# (B x H fills >= 1024 workgroups), one on the GEMM + recurrence route, and
# a readout of 128+ neurons (the dense variant's readout GEMMs then take the
# 128 x 128 kernel, whose K split differs from the packed variant's)
SHAPES = [(13, 3, 20, 37, 5), (29, 6, 70, 100, 20), (5, 256, 32, 2048, 10), (9, 32, 40, 300, 130)]


@pytest.mark.parametrize("shape", SHAPES)
def test_two_layer_matches_oracle_and_variants_agree(shape):
    T, B, F, H, O = shape
    _print_case(test="two_layer_oracle", shape=shape)
    tensors, grate = _random_net(sum(shape), *shape)
    p = myelin.LIFParams(tau_mem=8.0, threshold=0.7, reset=-0.2)
    out = {}
    for name, fn in VARIANTS.items():
        r, leaves = _run(fn, tensors, True, p, surrogate="fast_sigmoid", surrogate_slope=5.0, checkpoint_size=4)
        r.backward(grate.to(DEV))
        out[name] = [to_np(r)] + _grads(leaves)
    if O < 128:
        # same GEMM kernel and K split for words and dense spikes
        for a, b in zip(out["recompute"], out["packed"]):
            assert np.array_equal(a, b)
    else:
        assert np.abs(out["recompute"][0] - out["packed"][0]).max() <= 1.0 / T + 1e-7
        if np.array_equal(out["recompute"][0], out["packed"][0]):
            for name, a, b in zip(("x", "wh", "bh", "wo", "bo"), out["recompute"][1:], out["packed"][1:]):
                assert_norm_close(a, b, 1e-5, f"packed vs recompute grad_{name}")
    leaves = [t.clone().requires_grad_() for t in tensors]
    rr = R.two_layer_rate(*leaves, 8.0, 0.7, -0.2, "fast_sigmoid", 5.0, 4)
    rr.backward(grate)
    got = out["recompute"]
    if np.array_equal(got[0], rr.detach().numpy()):
        for name, g, t in zip(("x", "wh", "bh", "wo", "bo"), got[1:], leaves):
            assert_norm_close(g, t.grad, 1e-5, f"grad_{name}")
    else:
        # a threshold tie flipped one readout spike: rates differ by 1/T there
        assert np.abs(got[0] - rr.detach().numpy()).max() <= 1.0 / T + 1e-7


def test_two_layer_equals_composed_one_layer_paths():
    """The interleaved network equals the hidden checkpoint layer followed by
    the rate readout, both run on their own (tests/test_modules.py:680-735
    pattern)."""

    _print_case(test="two_layer_composed")
    tensors, grate = _random_net(7, 17, 4, 30, 45, 6)
    p = myelin.LIFParams(tau_mem=8.0, threshold=0.7, reset=-0.2)
    r, leaves = _run(myelin.two_layer_surrogate_lif_rate_recompute_forward, tensors, True, p, checkpoint_size=3)
    r.backward(grate.to(DEV))
    x, wh, bh, wo, bo = (t.to(DEV).requires_grad_() for t in tensors)
    _, hs = myelin.linear_surrogate_lif_forward(x, wh, bh, p, surrogate="fast_sigmoid", surrogate_slope=5.0,
                                                checkpoint_size=3)
    _, rates = myelin.linear_surrogate_lif_rate_forward(hs, wo, bo, p, surrogate="fast_sigmoid", surrogate_slope=5.0,
                                                        checkpoint_size=3, reduction="none")
    rates.backward(grate.to(DEV))
    assert torch.equal(r.detach(), rates.detach())
    for name, a, b in zip(("x", "wh", "bh", "wo", "bo"), leaves, (x, wh, bh, wo, bo)):
        assert_norm_close(to_np(a.grad), to_np(b.grad), 1e-5, f"grad_{name}")


def test_two_layer_checkpoint_sizes_and_partial_grads():
    _print_case(test="two_layer_ck_partial")
    T = 23
    tensors, grate = _random_net(11, T, 5, 24, 40, 7)
    p = myelin.LIFParams(tau_mem=8.0, threshold=0.7, reset=-0.2)
    ref = None
    for ck in (1, 6, T, 100):
        r, leaves = _run(myelin.two_layer_surrogate_lif_rate_packed_hidden_forward, tensors, True, p,
                         checkpoint_size=ck)
        r.backward(grate.to(DEV))
        res = [to_np(r)] + _grads(leaves)
        if ref is None:
            ref = res
            continue
        assert np.array_equal(res[0], ref[0]) and np.array_equal(res[1], ref[1])
        for a, b in zip(res[2:], ref[2:]):
            assert_norm_close(a, b, 1e-6, "weight/bias grads across checkpoint sizes")
    # only the readout weight trainable: the hidden backward is skipped
    x, wh, bh, wo, bo = (t.to(DEV) for t in tensors)
    wo = wo.clone().requires_grad_()
    r = myelin.two_layer_surrogate_lif_rate_recompute_forward(x, wh, bh, wo, bo, p, checkpoint_size=6)
    r.backward(grate.to(DEV))
    assert_norm_close(to_np(wo.grad), ref[4], 1e-6, "readout weight grad alone")
    # no grad needed at all: forward only
    with torch.no_grad():
        r2 = myelin.two_layer_surrogate_lif_rate_recompute_forward(x, wh, bh, wo, bo, p, checkpoint_size=6)
    assert np.array_equal(to_np(r2), ref[0])


def test_two_layer_bf16_synapse_within_tolerance():
    _print_case(test="two_layer_bf16")
    tensors, grate = _random_net(5, 20, 16, 128, 256, 10)
    p = myelin.LIFParams()
    r, leaves = _run(myelin.two_layer_surrogate_lif_rate_recompute_forward, tensors, True, p, checkpoint_size=5,
                     synapse_precision="bf16")
    loss = (r * grate.to(DEV)).sum()
    loss.backward()
    rt = [t.clone() for t in tensors]
    rt[1] = rt[1].to(torch.bfloat16).float()
    rt[3] = rt[3].to(torch.bfloat16).float()
    leaves_r = [t.requires_grad_() for t in rt]
    rr = R.two_layer_rate(*leaves_r, 20.0, 1.0, 0.0, "fast_sigmoid", 5.0, 5)
    (rr * grate).sum().backward()
    assert raster_agreement(to_np(r) * 20, rr.detach() * 20) >= 0.99
    assert abs(loss.item() - (rr * grate).sum().item()) <= 2e-2 * max(1.0, abs(loss.item()))
    for name, a, b in zip(("wh", "bh", "wo", "bo"), leaves[1:], leaves_r[1:]):
        assert_norm_close(to_np(a.grad), b.grad, 2e-2, f"grad_{name}")
