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


@pytest.mark.parametrize("variant", sorted(VARIANTS))
def test_memory_policy_spans_equal_one_span(variant):
    """checkpoint_size="memory" walks the backward one checkpoint chunk at a
    time (T=40: 7-step chunks, 6 spans, one buffer set); an explicit
    checkpoint_size=7 walks one span.  Same rates, gradients within 1e-5."""

    T, B, F, H, O = 40, 3, 24, 37, 5
    _print_case(test="two_layer_memory_policy", variant=variant)
    tensors, grate = _random_net(77, T, B, F, H, O)
    p = myelin.LIFParams(tau_mem=8.0, threshold=0.7, reset=-0.2)
    out = {}
    for ck in ("memory", 7):
        r, leaves = _run(VARIANTS[variant], tensors, True, p, surrogate="fast_sigmoid", surrogate_slope=5.0,
                         checkpoint_size=ck)
        r.backward(grate.to(DEV))
        out[ck] = (to_np(r), _grads(leaves))
    assert np.array_equal(out["memory"][0], out[7][0])
    for a, b, name in zip(out["memory"][1], out[7][1], ("gx", "gwh", "gbh", "gwo", "gbo")):
        assert_norm_close(a, b, 1e-5, name)


def test_linear_memory_policy_spans_equal_one_span():
    """The one-layer streamed-synapse path: "memory" (one-chunk spans) and
    the explicit chunk size give the same spikes and input gradient, and
    weight gradients within 1e-6."""

    _print_case(test="linear_memory_policy")
    (x, wh, bh, _, _), _ = _random_net(78, 40, 3, 24, 37, 5)
    gs = torch.randn(40, 3, 37, generator=seeded(79))
    p = myelin.LIFParams(tau_mem=8.0, threshold=0.7, reset=-0.2)
    out = {}
    for ck in ("memory", 7):
        xd, wd, bd = (t.to(DEV).requires_grad_() for t in (x, wh, bh))
        _, s = myelin.linear_surrogate_lif_forward(xd, wd, bd, p, surrogate="atan", surrogate_slope=5.0,
                                                   checkpoint_size=ck)
        s.backward(gs.to(DEV))
        out[ck] = (to_np(s), to_np(xd.grad), to_np(wd.grad), to_np(bd.grad))
    assert np.array_equal(out["memory"][0], out[7][0]) and np.array_equal(out["memory"][1], out[7][1])
    assert_norm_close(out["memory"][2], out[7][2], 1e-6, "grad_w")
    assert_norm_close(out["memory"][3], out[7][3], 1e-6, "grad_b")


# (T, B, F, H, O, checkpoint, split, x_grad): small and wide grids, G
# written as fp32 (dX needs it) and as the three bf16 planes of the exact
# split, readouts of 5, 12, 20 and 32 neurons (the 8-, 12-, 20- and 32-term
# sums), a ragged last span under "memory"
DS_CASES = [(23, 4, 40, 256, 5, 5, False, True), (23, 4, 40, 512, 20, "memory", True, False),
            (19, 128, 32, 512, 32, 5, False, True), (19, 128, 32, 1024, 12, 4, True, False)]


@pytest.mark.parametrize("case", DS_CASES)
def test_fused_spike_gradient_equals_the_ds_gemm(case, monkeypatch):
    """The hidden reverse pass that forms dS = G_o W_o^T itself
    (myelin_linear_pre_bwd_readout) takes the small-K GEMM's sums, so the
    packed network's rates and every gradient equal those of the route that
    writes dS with that GEMM and reads it back, bit for bit."""

    from myelin_amd import _lib, linear, two_layer

    T, B, F, H, O, ck, split, x_grad = case
    _print_case(test="fused_ds", case=case)
    tensors, grate = _random_net(91 + H + O, T, B, F, H, O)
    tensors[0] = (torch.rand(T, B, F, generator=seeded(92)) < 0.2).float()  # spikes: bf16-exact
    if split:
        monkeypatch.setattr(linear, "_SPLIT_MIN_MACS", 0)
    p = myelin.LIFParams(tau_mem=8.0, threshold=0.7, reset=-0.2)
    real, names = _lib.call, []
    monkeypatch.setattr(_lib, "call", lambda name, *a: names.append(name) or real(name, *a))

    def run():
        names.clear()
        x, wh, bh, wo, bo = (t.to(DEV) for t in tensors)
        leaves = [x.requires_grad_(x_grad), *(t.requires_grad_() for t in (wh, bh, wo, bo))]
        r = myelin.two_layer_surrogate_lif_rate_packed_hidden_forward(*leaves, p, surrogate="superspike",
                                                                     surrogate_slope=5.0, checkpoint_size=ck)
        r.backward(grate.to(DEV))
        torch.cuda.synchronize()
        return [to_np(r)] + [to_np(t.grad) for t in leaves if t.requires_grad], list(names)

    fused, called = run()
    assert "myelin_linear_pre_bwd_readout" in called
    assert ("myelin_split_bf16x3" in called) == split
    monkeypatch.setattr(two_layer, "_ds_fused", lambda *a: False)
    gemm, called = run()
    assert "myelin_linear_pre_bwd_readout" not in called
    for a, b in zip(fused, gemm):
        assert np.array_equal(a, b)
