"""GPU parity of the streamed-synapse path: MFMA GEMM, fused synapse + LIF
forward, chunked backward, rate readout, packed forward and modules.

Bars:
* GEMM: fp32 within 1e-5 (max-norm relative) of a float64 CPU product;
  bf16 within 1e-5 of the float64 product of the bf16-rounded inputs.
* fp32 linear paths vs the reference (golden vectors recorded from myelin's
  torch backend) and the oracle: spike rasters >= 99.99 % equal, membranes
  and gradients within 1e-5 max-norm relative (measured <= 4e-7); against
  the golden vectors also per element: within 1e-4, |a - b| <= 1e-4 *
  max(|b|, 1e-3 max|b|), or no farther from the float64 evaluation of the
  same network (the oracle run in float64 on the golden inputs, every
  scalar at its fp32 value) than the golden value itself is.  Two fp32
  evaluations differ by more than 1e-4 at elements near the floor: the
  GEMMs sum in another order than the CPU matmul, and the reference's spikes
  (H + sigma) - sigma can sit an ulp below 1 in its reset and backward.
* bf16 synapse: against the fp32 oracle run on bf16-rounded weights, rasters
  >= 99.99 %, losses and gradients within 2e-2 relative.
"""

from __future__ import annotations

import pathlib

import numpy as np
import pytest
import torch

import myelin_amd as myelin
from myelin_amd import _lib
from myelin_amd.linear import _gemm, linear
from oracle import torch_ref as R
from tests.helpers import (assert_elementwise_close_or_truer, assert_norm_close, assert_same_bits, f32_params,
                           raster_agreement, seeded, to_np)

pytestmark = pytest.mark.gpu
DEV = "cuda"
LIN = dict(np.load(pathlib.Path(__file__).parent / "golden" / "linear_paths.npz"))
P = myelin.LIFParams(tau_mem=9.0, threshold=0.7, reset=-0.2)


def _print_case(**kw):
    print("case:", " ".join(f"{k}={v}" for k, v in kw.items()), flush=True)


def _bf16(t):
    return t.to(torch.bfloat16).to(torch.float32)


# includes the narrow-output route (N <= 32: readout currents and dW_o, with
# K splits) and the small-K route (K <= 32: dS = G_o W_o^T)
@pytest.mark.parametrize("M,N,K", [(1, 1, 1), (64, 64, 64), (70, 33, 100), (300, 17, 784), (5, 200, 10),
                                   (129, 65, 31), (128, 128, 64), (300, 260, 1000), (256, 384, 3000),
                                   (520, 132, 200), (129, 130, 64), (8200, 1032, 72), (6400, 10, 2048),
                                   (4096, 20, 1500), (257, 32, 1025), (33, 7, 5), (1440, 2050, 20), (70, 40, 32)])
@pytest.mark.parametrize("ta,tb", [(False, False), (False, True), (True, False), (True, True)])
@pytest.mark.parametrize("prec", ["fp32", "bf16"])
def test_gemm(M, N, K, ta, tb, prec):
    _print_case(test="gemm", M=M, N=N, K=K, ta=ta, tb=tb, prec=prec)
    g = seeded(M * 7 + N * 3 + K)
    A = torch.randn((K, M) if ta else (M, K), generator=g)
    B = torch.randn((N, K) if tb else (K, N), generator=g)
    bias = torch.randn(N, generator=g)
    C0 = torch.randn(M, N, generator=g)
    a64 = (A.t() if ta else A).double()
    b64 = (B.t() if tb else B).double()
    if prec == "bf16":
        a64 = _bf16(A.t() if ta else A).double()
        b64 = _bf16(B.t() if tb else B).double()
    ref = a64 @ b64
    Ad, Bd = A.to(DEV), B.to(DEV)
    C = torch.empty(M, N, device=DEV)
    stream = _lib.stream(torch.device(DEV))
    _gemm(Ad, Bd, C, M, N, K, A.shape[1], B.shape[1], N, ta, tb, False, _lib.PREC[prec], stream)
    assert_norm_close(C.cpu().double(), ref, 1e-5, "C")
    Cacc = C0.to(DEV)
    _gemm(Ad, Bd, Cacc, M, N, K, A.shape[1], B.shape[1], N, ta, tb, True, _lib.PREC[prec], stream, bias=bias.to(DEV))
    assert_norm_close(Cacc.cpu().double(), C0.double() + ref + bias.double(), 1e-5, "C accumulate + bias")


@pytest.mark.parametrize("ta,tb", [(False, False), (False, True), (True, False), (True, True)])
@pytest.mark.parametrize("prec", ["fp32", "bf16"])
@pytest.mark.parametrize("M,N,K", [(260, 200, 300), (8200, 1032, 72)])
def test_gemm_tile_sizes_sum_identically(ta, tb, prec, M, N, K):
    """The 128 x 128 / 256 x 128 kernels (16-byte-aligned operands) and the
    64 x 64 kernel (same operands one float off alignment) run the same k
    order per output element, so with no K split all give bit-identical
    products."""

    _print_case(test="gemm_tiles", ta=ta, tb=tb, prec=prec, M=M, N=N, K=K)
    g = seeded(99)
    A = torch.randn((K, M) if ta else (M, K), generator=g)
    B = torch.randn((N, K) if tb else (K, N), generator=g)
    stream = _lib.stream(torch.device(DEV))
    out = []
    for shift in (0, 1):
        Ab = torch.zeros(A.numel() + 4, device=DEV)
        Ab[shift:shift + A.numel()] = A.reshape(-1).to(DEV)
        Ad = Ab[shift:shift + A.numel()].view(A.shape)
        C = torch.empty(M, N, device=DEV)
        _gemm(Ad, B.to(DEV), C, M, N, K, A.shape[1], B.shape[1], N, ta, tb, False, _lib.PREC[prec], stream)
        out.append(C.cpu())
    assert torch.equal(out[0], out[1])


def test_linear_synapse_function_grads():
    _print_case(test="linear_fn")
    g = seeded(3)
    x = torch.randn(6, 5, 33, generator=g)
    w = torch.randn(33, 20, generator=g) * 0.1
    b = torch.randn(20, generator=g)
    gy = torch.randn(6, 5, 20, generator=g)
    xd, wd, bd = (t.to(DEV).requires_grad_() for t in (x, w, b))
    y = linear(xd, wd, bd)
    y.backward(gy.to(DEV))
    xr, wr, br = (t.double().requires_grad_() for t in (x, w, b))
    yr = xr @ wr + br
    yr.backward(gy.double())
    assert_norm_close(y.detach().cpu(), yr.detach(), 1e-5, "y")
    assert_norm_close(xd.grad.cpu(), xr.grad, 1e-5, "gx")
    assert_norm_close(wd.grad.cpu(), wr.grad, 1e-5, "gw")
    assert_norm_close(bd.grad.cpu(), br.grad, 1e-5, "gb")


def _golden_grads_close(xd, wd, bd, tag, truth):
    """Max-norm 1e-5 against the reference's golden gradients; per element
    within 1e-4 of them, or no farther than they are from the float64
    evaluation `truth` (x, w, b grads of the oracle run in float64)."""

    for (name, t), tr in zip((("gx", xd), ("gw", wd), ("gb", bd)), truth):
        if t is None:
            continue
        assert_norm_close(to_np(t.grad), LIN[f"{tag}_{name}"], 1e-5, name)
        assert_elementwise_close_or_truer(t.grad, LIN[f"{tag}_{name}"], tr, 1e-4, name)


def _golden_truth(run, x, w, b, bias, golden_spikes=None):
    """The oracle's gradients in float64 on the golden inputs (`run(x, w, b)`
    builds the reference's graph, backpropagates and returns its spikes or
    rates); the rasters must be the golden ones."""

    xr, wr = x.double().requires_grad_(), w.double().requires_grad_()
    br = b.double().requires_grad_() if bias else None
    out = run(xr, wr, br)
    if golden_spikes is not None:
        assert np.array_equal(to_np(out) > 0.5, golden_spikes > 0.5), "float64 raster differs from the golden one"
    return xr.grad, wr.grad, None if br is None else br.grad


def _golden_inputs():
    return (torch.from_numpy(LIN[k]) for k in ("x", "w", "b", "gs", "gfin", "grate"))


@pytest.mark.parametrize("bias", [False, True])
@pytest.mark.parametrize("ck", [None, 1, 4, 9])
@pytest.mark.parametrize("with_final", [False, True])
def test_linear_spike_paths_match_reference(bias, ck, with_final):
    _print_case(test="linear_spikes", bias=bias, ck=ck, with_final=with_final)
    x, w, b, gs, gfin, _ = _golden_inputs()
    xd, wd = x.to(DEV).requires_grad_(), w.to(DEV).requires_grad_()
    bd = b.to(DEV).requires_grad_() if bias else None
    st, s = myelin.linear_surrogate_lif_forward(xd, wd, bd, P, surrogate="atan", surrogate_slope=5.0,
                                                checkpoint_size=ck)
    outs, grads = [s], [gs.to(DEV)]
    if with_final:
        outs.append(st.membrane)
        grads.append(gfin.to(DEV))
    torch.autograd.backward(outs, grads)
    tag = f"spk_{'b' if bias else 'nob'}_c{ck}_f{int(with_final)}"
    assert raster_agreement(s, LIN[f"{tag}_s"]) >= 0.9999
    assert bool(((s == 0) | (s == 1)).all())
    assert_norm_close(to_np(st.membrane), LIN[f"{tag}_mT"], 1e-5, "membrane")
    tau, thr, rst = f32_params(P.tau_mem, P.threshold, P.reset)

    def run(xr, wr, br):
        if ck is None:
            m, sp = R.linear_surrogate_lif_stream(xr, wr, br, tau, thr, rst, "atan", 5.0)
        else:
            m, sp = R.linear_surrogate_lif_checkpoint(xr, wr, br, tau, thr, rst, "atan", 5.0, ck)
        torch.autograd.backward([sp, m] if with_final else [sp], [gs.double(), gfin.double()][:1 + with_final])
        return sp.detach()

    _golden_grads_close(xd, wd, bd, tag, _golden_truth(run, x, w, b, bias, LIN[f"{tag}_s"]))


@pytest.mark.parametrize("bias", [False, True])
@pytest.mark.parametrize("ck", [1, 4, 9])
@pytest.mark.parametrize("red", ["none", "mean"])
def test_linear_rate_paths_match_reference(bias, ck, red):
    _print_case(test="linear_rate", bias=bias, ck=ck, red=red)
    x, w, b, _, _, grate = _golden_inputs()
    xd, wd = x.to(DEV).requires_grad_(), w.to(DEV).requires_grad_()
    bd = b.to(DEV).requires_grad_() if bias else None
    st, r = myelin.linear_surrogate_lif_rate_forward(xd, wd, bd, P, surrogate="superspike", surrogate_slope=5.0,
                                                     checkpoint_size=ck, reduction=red)
    if red == "none":
        r.backward(grate.to(DEV))
    else:
        r.backward()
    tag = f"rate_{'b' if bias else 'nob'}_c{ck}_{red}"
    if red == "none":
        assert np.array_equal(to_np(r), LIN[f"{tag}_r"])  # counts / T: exact when rasters agree
    else:
        # torch's mean over [B, N] sums in a device-dependent order
        assert_norm_close(to_np(r), LIN[f"{tag}_r"], 1e-6, "mean rate")
    assert_norm_close(to_np(st.membrane), LIN[f"{tag}_mT"], 1e-5, "membrane")
    tau, thr, rst = f32_params(P.tau_mem, P.threshold, P.reset)

    def run(xr, wr, br):
        _, rr = R.linear_surrogate_lif_rate(xr, wr, br, tau, thr, rst, "superspike", 5.0, ck, reduction=red)
        rr.backward(grate.double() if red == "none" else None)
        return None

    _golden_grads_close(xd, wd, bd, tag, _golden_truth(run, x, w, b, bias))


@pytest.mark.parametrize("T,B,F,N", [(20, 9, 40, 70), (33, 16, 64, 128), (5, 1, 3, 1)])
def test_linear_checkpoint_sizes_agree_and_match_oracle(T, B, F, N):
    _print_case(test="linear_oracle", T=T, B=B, F=F, N=N)
    g = seeded(T + B + F + N)
    x = (torch.rand(T, B, F, generator=g) < 0.3).float()
    w = (torch.rand(F, N, generator=g) - 0.5) * 0.6
    b = torch.rand(N, generator=g) * 0.1
    gs = torch.randn(T, B, N, generator=g)
    res = []
    for ck in (None, 1, 7, T):
        xd, wd, bd = (t.to(DEV).requires_grad_() for t in (x, w, b))
        st, s = myelin.linear_surrogate_lif_forward(xd, wd, bd, P, surrogate="fast_sigmoid", surrogate_slope=5.0,
                                                    checkpoint_size=ck)
        s.backward(gs.to(DEV))
        res.append((to_np(s), to_np(xd.grad), to_np(wd.grad), to_np(bd.grad)))
    for r in res[1:]:
        # recompute reproduces the forward exactly; dW / db sum the rows in
        # chunk order, so only their rounding depends on the checkpoint size
        assert np.array_equal(r[0], res[0][0]) and np.array_equal(r[1], res[0][1])
        assert_norm_close(r[2], res[0][2], 1e-6, "grad_w across checkpoint sizes")
        assert_norm_close(r[3], res[0][3], 1e-6, "grad_b across checkpoint sizes")
    xr, wr, br = (t.clone().requires_grad_() for t in (x, w, b))
    _, es = R.linear_surrogate_lif_checkpoint(xr, wr, br, 9.0, 0.7, -0.2, "fast_sigmoid", 5.0, 4)
    es.backward(gs)
    # the shapes here give the oracle's raster exactly (every spike on the
    # same side of the threshold), so the gradients are compared always
    assert raster_agreement(res[0][0], es) == 1.0
    assert_norm_close(res[0][1], xr.grad, 1e-5, "grad_x")
    assert_norm_close(res[0][2], wr.grad, 1e-5, "grad_w")
    assert_norm_close(res[0][3], br.grad, 1e-5, "grad_b")


@pytest.mark.parametrize("N", [17, 31, 32, 33, 64, 100])
def test_linear_packed_forward_matches_dense(N):
    _print_case(test="linear_packed", N=N)
    g = seeded(N)
    x = (torch.rand(9, 5, 23, generator=g) < 0.4).float()
    w = (torch.rand(23, N, generator=g) - 0.3) * 0.8
    b = torch.rand(N, generator=g) * 0.1
    st, pk = myelin.linear_surrogate_lif_packed_forward(x.to(DEV), w.to(DEV), b.to(DEV), P, checkpoint_size=4)
    st2, s = myelin.linear_surrogate_lif_forward(x.to(DEV), w.to(DEV), b.to(DEV), P, checkpoint_size=4)
    assert torch.equal(pk.data, myelin.pack_spikes(s).data)
    assert torch.equal(st.membrane, st2.membrane)
    assert pk.original_shape == (9, 5, N)


def test_modules_match_functional_paths():
    _print_case(test="modules")
    torch.manual_seed(0)
    layer = myelin.LinearSurrogateLIF(13, 21, P, surrogate=myelin.fast_sigmoid_surrogate, surrogate_slope=5.0,
                                      stream_synapse=True, checkpoint_size=4).to(DEV)
    unfused = myelin.LinearSurrogateLIF(13, 21, P, surrogate=myelin.fast_sigmoid_surrogate, surrogate_slope=5.0,
                                        stream_synapse=False).to(DEV)
    unfused.load_state_dict(layer.state_dict())
    g = seeded(1)
    x = (torch.rand(8, 4, 13, generator=g) < 0.5).float().to(DEV)
    s1, s2 = layer(x), unfused(x)
    assert raster_agreement(s1, s2) >= 0.9999
    rate = myelin.LinearSurrogateLIFRate(21, 3, P, checkpoint_size=3).to(DEV)
    r = rate(s1)
    assert r.shape == (4, 3)
    r.sum().backward()
    assert layer.synapse.weight.grad is not None and rate.synapse.weight.grad is not None
    clf = myelin.RateReadoutClassifier(13, 21, 3, P, checkpoint_size=4).to(DEV)
    assert clf(x).shape == (4, 3)
    packed = myelin.LinearSurrogateLIFPacked(13, 21, P).to(DEV)
    packed.load_state_dict({"synapse.weight": layer.synapse.weight, "synapse.bias": layer.synapse.bias})
    assert packed(x).data.shape == (8, 4, 1)


def test_streamed_synapse_bf16_T50_B256():
    """LinearSurrogateLIF(784 -> 2048, stream_synapse=True, atan, bf16 GEMM)
    then LinearSurrogateLIFRate(2048 -> 10, atan), CE on spike counts, at the
    full [50, 256, 784] (the hidden dW is the 784 x 2048 x 12800 product with
    its K split); oracle = fp32 torch path on bf16-rounded weights (inputs
    are exactly 0/1)."""

    _print_case(test="streamed_synapse_bf16_T50_B256")
    T, B, F, H, O = 50, 256, 784, 2048, 10
    g = seeded(3)
    rate_f = torch.rand(F, generator=g) * 0.2
    x = (torch.rand(T, B, F, generator=g) < rate_f).float()
    w1 = torch.empty(H, F).uniform_(-(6 / F) ** 0.5, (6 / F) ** 0.5, generator=g).t().contiguous()
    w2 = torch.empty(O, H).uniform_(-(6 / H) ** 0.5, (6 / H) ** 0.5, generator=g).t().contiguous()
    b1, b2 = torch.zeros(H), torch.zeros(O)
    labels = torch.randint(0, O, (B,), generator=g)
    p = myelin.LIFParams()

    w1d, b1d, w2d, b2d = (t.to(DEV).requires_grad_() for t in (w1, b1, w2, b2))
    _, hs = myelin.linear_surrogate_lif_forward(x.to(DEV), w1d, b1d, p, surrogate="atan", synapse_precision="bf16")
    _, rates = myelin.linear_surrogate_lif_rate_forward(hs, w2d, b2d, p, surrogate="atan", checkpoint_size=25,
                                                        reduction="none", synapse_precision="bf16")
    loss = torch.nn.functional.cross_entropy(rates * T, labels.to(DEV))
    loss.backward()

    w1r, b1r, w2r, b2r = (t.clone().requires_grad_() for t in (_bf16(w1), b1, _bf16(w2), b2))
    _, hr = R.linear_surrogate_lif_stream(x, w1r, b1r, 20.0, 1.0, 0.0, "atan", 10.0)
    _, rr = R.linear_surrogate_lif_rate(hr, w2r, b2r, 20.0, 1.0, 0.0, "atan", 10.0, 25, reduction="none")
    loss_r = torch.nn.functional.cross_entropy(rr * T, labels)
    loss_r.backward()
    assert raster_agreement(hs, hr) >= 0.9999
    assert abs(loss.item() - loss_r.item()) <= 2e-2 * abs(loss_r.item())
    assert_norm_close(to_np(w1d.grad), w1r.grad, 2e-2, "grad_w1")
    assert_norm_close(to_np(w2d.grad), w2r.grad, 2e-2, "grad_w2")
    assert_norm_close(to_np(b1d.grad), b1r.grad, 2e-2, "grad_b1")
    assert_norm_close(to_np(b2d.grad), b2r.grad, 2e-2, "grad_b2")


@pytest.mark.parametrize("T,B,F,N", [(13, 20, 200, 300), (9, 48, 96, 256), (5, 7, 64, 128), (20, 3, 44, 64)])
@pytest.mark.parametrize("prec", ["fp32", "bf16"])
def test_fused_forward_equals_gemm_then_recurrence(T, B, F, N, prec):
    """myelin_linear_lif_fwd (128 x 128 fused tiles when N >= 128, 64 x 64
    otherwise) against the unfused route (MFMA GEMM with the bias epilogue,
    then myelin_lif_currents_fwd): same k order, same per-step arithmetic, so
    every output is bit-identical.  K stays short enough that the GEMM does
    not split."""

    _print_case(test="fused_vs_unfused", T=T, B=B, F=F, N=N, prec=prec)
    g = seeded(T * 1000 + N)
    x = (torch.rand(T, B, F, generator=g) < 0.4).float().to(DEV)
    w = ((torch.rand(F, N, generator=g) - 0.4) * 0.5).to(DEV)
    bias = (torch.rand(N, generator=g) * 0.1).to(DEV)
    m0 = (torch.rand(B, N, generator=g) * 0.5).to(DEV)
    pr = _lib.PREC[prec]
    stream = _lib.stream(torch.device(DEV))
    W = (N + 31) // 32
    ck_every = 3
    nck = -(-T // ck_every)

    def outputs():
        return dict(m=torch.empty(B, N, device=DEV), s=torch.empty(T, B, N, device=DEV),
                    pre=torch.empty(T, B, N, device=DEV), pk=torch.empty(T, B, W, dtype=torch.int32, device=DEV),
                    r=torch.empty(B, N, device=DEV), ck=torch.empty(nck, B, N, device=DEV))

    a = outputs()
    _lib.call("myelin_linear_lif_fwd", _lib.ptr(x), _lib.ptr(w), _lib.ptr(bias), _lib.ptr(m0), _lib.ptr(a["m"]),
              _lib.ptr(a["s"]), _lib.ptr(a["pre"]), _lib.ptr(a["pk"]), _lib.ptr(a["r"]), _lib.ptr(a["ck"]), T, B, F, N,
              0, T, ck_every, 0.9, 0.6, -0.1, 5.0, _lib.RULE_THRESHOLD, pr, stream)
    b = outputs()
    cur = torch.empty(T, B, N, device=DEV)
    _gemm(x, w, cur, T * B, N, F, F, N, N, False, False, False, pr, stream, bias=bias)
    _lib.call("myelin_lif_currents_fwd", _lib.ptr(cur), _lib.ptr(m0), _lib.ptr(b["m"]), _lib.ptr(b["s"]),
              _lib.ptr(b["pre"]), _lib.ptr(b["pk"]), _lib.ptr(b["r"]), None, _lib.ptr(b["ck"]), T, B, N, 0, T, 0, 0,
              ck_every, 0.9, 0.6, -0.1, 5.0, _lib.RULE_THRESHOLD, stream)
    torch.cuda.synchronize()
    for k in a:
        assert torch.equal(a[k], b[k]), k
    assert torch.equal(a["pk"], myelin.pack_spikes(a["s"]).data)


# 16 batch rows x 128 neurons per workgroup, grid >= 192: the accumulator-
# resident recurrence kernel.  F = 136: two 64-k stages and a partial one
# of one 16-k step; 64: one stage; 40: the partial stage only; 120 and 88:
# partial stages of four and two 16-k steps; ragged B and N; T not a
# multiple of the 16-step chunk; a grid that is not a multiple of 8 (195
# tiles: no XCD remapping); and the 784 -> 2048 layer at T = 50, B = 256.
@pytest.mark.parametrize("T,B,F,N,t_begin,rule", [
    (21, 250, 136, 1500, 0, 0), (17, 256, 64, 1536, 0, 1), (33, 400, 40, 1024, 0, 0),
    (21, 250, 136, 1500, 6, 1), (19, 200, 120, 1920, 0, 1), (23, 256, 88, 1536, 3, 0),
    (50, 256, 784, 2048, 0, 0)])
def test_fused_bf16_accumulator_kernel_equals_gemm_then_recurrence(T, B, F, N, t_begin, rule):
    """myelin_linear_lif_fwd_bf16 on its accumulator-recurrence kernel
    against the bf16 GEMM (bias epilogue) then myelin_lif_currents_fwd: the
    same k order and per-step arithmetic, so every output (membrane,
    spikes, pre-reset trace, packed words, rates, checkpoints) is equal bit
    for bit, from any start step."""

    _print_case(test="fused_acc_vs_unfused", T=T, B=B, F=F, N=N, t_begin=t_begin, rule=rule)
    assert -(-N // 128) * -(-B // 16) >= 192
    g = seeded(T * 7 + B + F + N)
    x = (torch.rand(T, B, F, generator=g) < 0.3).float().to(DEV)
    w = ((torch.rand(F, N, generator=g) - 0.45) * 0.4).to(DEV)
    bias = (torch.rand(N, generator=g) * 0.1).to(DEV)
    m0 = (torch.rand(B, N, generator=g) * 0.5).to(DEV)
    stream = _lib.stream(torch.device(DEV))
    xb = x.to(torch.bfloat16)
    wt = w.t().contiguous().to(torch.bfloat16)
    W = (N + 31) // 32
    ck_every = 5
    Tr = T - t_begin
    nck = -(-Tr // ck_every)

    def outputs():
        return dict(m=torch.empty(B, N, device=DEV), s=torch.zeros(T, B, N, device=DEV),
                    pre=torch.empty(Tr, B, N, device=DEV), pk=torch.zeros(T, B, W, dtype=torch.int32, device=DEV),
                    r=torch.empty(B, N, device=DEV), ck=torch.empty(nck, B, N, device=DEV))

    a = outputs()
    _lib.call("myelin_linear_lif_fwd_bf16", _lib.ptr(xb), _lib.ptr(wt), _lib.ptr(bias), _lib.ptr(m0),
              _lib.ptr(a["m"]), _lib.ptr(a["s"]), _lib.ptr(a["pre"]), _lib.ptr(a["pk"]), _lib.ptr(a["r"]),
              _lib.ptr(a["ck"]), T, B, F, N, t_begin, T, ck_every, 0.9, 0.6, -0.1, 5.0, rule, stream)
    b = outputs()
    cur = torch.empty(T, B, N, device=DEV)
    _gemm(xb, wt, cur, T * B, N, F, F, F, N, False, True, False, _lib.PREC["bf16"], stream, bias=bias, split=False)
    _lib.call("myelin_lif_currents_fwd", _lib.ptr(cur[t_begin:]), _lib.ptr(m0), _lib.ptr(b["m"]), _lib.ptr(b["s"]),
              _lib.ptr(b["pre"]), _lib.ptr(b["pk"]), _lib.ptr(b["r"]), None, _lib.ptr(b["ck"]), T, B, N, t_begin, T,
              t_begin, t_begin, ck_every, 0.9, 0.6, -0.1, 5.0, rule, stream)
    torch.cuda.synchronize()
    for k in a:
        assert torch.equal(a[k], b[k]), k
    assert bool((a["s"][t_begin:] != 0).any()) and bool((a["s"][t_begin:] == 0).any())


# The kernel is compiled apart for the training output sets (trace + spikes,
# with or without their packed twin) and the inference one (spikes),
# without the per-output branches.
@pytest.mark.parametrize("outs", ["train", "train_packed", "infer"])
@pytest.mark.parametrize("T,B,F,N,t_begin,rule", [
    (21, 250, 136, 1500, 0, 0), (19, 200, 120, 1920, 2, 1), (50, 256, 784, 2048, 0, 0)])
def test_fused_bf16_accumulator_kernel_output_sets(T, B, F, N, t_begin, rule, outs):
    """The specialised output sets of the accumulator-recurrence kernel
    against the bf16 GEMM then myelin_lif_currents_fwd, bit for bit."""

    _print_case(test="fused_acc_output_sets", T=T, B=B, F=F, N=N, t_begin=t_begin, rule=rule, outs=outs)
    g = seeded(T * 5 + B + F + N)
    x = (torch.rand(T, B, F, generator=g) < 0.3).float().to(DEV)
    w = ((torch.rand(F, N, generator=g) - 0.45) * 0.4).to(DEV)
    bias = (torch.rand(N, generator=g) * 0.1).to(DEV)
    m0 = (torch.rand(B, N, generator=g) * 0.5).to(DEV)
    stream = _lib.stream(torch.device(DEV))
    xb = x.to(torch.bfloat16)
    wt = w.t().contiguous().to(torch.bfloat16)
    Tr = T - t_begin

    W = (N + 31) // 32

    def outputs():
        o = dict(m=torch.empty(B, N, device=DEV), s=torch.zeros(T, B, N, device=DEV))
        if outs != "infer":
            o["pre"] = torch.empty(Tr, B, N, device=DEV)
        if outs == "train_packed":
            o["pk"] = torch.zeros(T, B, W, dtype=torch.int32, device=DEV)
        return o

    def ptrs(o):
        return (_lib.ptr(o["m"]), _lib.ptr(o["s"]), _lib.ptr(o.get("pre")), _lib.ptr(o.get("pk")), None, None)

    a = outputs()
    _lib.call("myelin_linear_lif_fwd_bf16", _lib.ptr(xb), _lib.ptr(wt), _lib.ptr(bias), _lib.ptr(m0), *ptrs(a),
              T, B, F, N, t_begin, T, 1, 0.9, 0.6, -0.1, 5.0, rule, stream)
    b = outputs()
    cur = torch.empty(T, B, N, device=DEV)
    _gemm(xb, wt, cur, T * B, N, F, F, F, N, False, True, False, _lib.PREC["bf16"], stream, bias=bias, split=False)
    _lib.call("myelin_lif_currents_fwd", _lib.ptr(cur[t_begin:]), _lib.ptr(m0), _lib.ptr(b["m"]), _lib.ptr(b["s"]),
              _lib.ptr(b.get("pre")), _lib.ptr(b.get("pk")), None, None, None, T, B, N, t_begin, T, t_begin, t_begin, 1,
              0.9, 0.6, -0.1, 5.0, rule, stream)
    torch.cuda.synchronize()
    for k in a:
        assert torch.equal(a[k], b[k]), k
    assert bool((a["s"][t_begin:] != 0).any()) and bool((a["s"][t_begin:] == 0).any())


@pytest.mark.parametrize("rows,cols", [(1, 1), (7, 13), (64, 64), (130, 257), (1000, 24)])
def test_bf16_copies_round_like_torch(rows, cols):
    _print_case(test="bf16_copies", rows=rows, cols=cols)
    g = seeded(rows + cols)
    x = (torch.randn(rows, cols, generator=g) * 3).to(DEV)
    stream = _lib.stream(torch.device(DEV))
    from myelin_amd.linear import _cast_bf16, _transpose_bf16
    assert torch.equal(_cast_bf16(x, stream), x.to(torch.bfloat16))
    assert torch.equal(_transpose_bf16(x, stream), x.t().contiguous().to(torch.bfloat16))


@pytest.mark.parametrize("n,rows,cols", [(8, 1, 1), (13, 7, 13), (50 * 256 * 784, 784, 2048), (4096, 130, 257),
                                         (0, 33, 5), (24, 0, 0)])
def test_cast_transpose_in_one_launch_equals_the_two(n, rows, cols):
    """myelin_cast_transpose_bf16 gives the bits of myelin_cast_bf16 and
    myelin_transpose_bf16 (the bf16 synapse's operand copies), either part
    empty too."""

    _print_case(test="cast_transpose", n=n, rows=rows, cols=cols)
    from myelin_amd.linear import _cast_bf16, _cast_transpose_bf16, _transpose_bf16

    g = seeded(n + rows + cols)
    x = (torch.randn(n, generator=g) * 3).to(DEV)
    w = (torch.randn(rows, cols, generator=g) * 3).to(DEV)
    stream = _lib.stream(torch.device(DEV))
    xb, wt = _cast_transpose_bf16(x, w, stream)
    if n:
        assert torch.equal(xb, _cast_bf16(x, stream))
    if rows and cols:
        assert torch.equal(wt, _transpose_bf16(w, stream))


# (M, N, K, prec, bits): dW-shaped products whose K is split (the column sum
# joins the split-K reduce launch, four-wide and scalar) and ones that are
# not split (the column sum runs after the GEMM), narrow and wide, fp32,
# bf16 and packed-bit operands
COLSUM_CASES = [(784, 2048, 12800, "bf16", False), (2048, 10, 12800, "bf16", True), (2048, 10, 12800, "fp32", True),
                (300, 17, 784, "fp32", False), (64, 64, 64, "fp32", False), (1024, 4096, 1440, "fp32", False),
                (37, 5, 9, "fp32", False)]


@pytest.mark.parametrize("M,N,K,prec,bits", COLSUM_CASES)
def test_gemm_with_attached_col_sum_equals_the_two_launches(M, N, K, prec, bits):
    """myelin_gemm_col_sum: C and the column sum are bit-identical to
    myelin_gemm followed by myelin_col_sum_f32, whether the column sum ran in
    the split-K reduce launch or on its own."""

    _print_case(test="gemm_col_sum", M=M, N=N, K=K, prec=prec, bits=bits)
    g = seeded(M + N + K)
    stream = _lib.stream(torch.device(DEV))
    P = _lib.PREC[prec]
    A = (torch.rand(K, M, generator=g) < 0.3).float().to(DEV)  # x^T layout: [K rows, M] read transposed
    B = torch.randn(K, N, generator=g).to(DEV)
    src = torch.randn(97, N + 3, generator=g).to(DEV)
    if bits:
        words = myelin.pack_spikes(A).data
        Aop, lda = words, words.shape[-1]
    else:
        Aop, lda = (A.to(torch.bfloat16), M) if prec == "bf16" else (A, M)
        if prec == "bf16":
            B = B.to(torch.bfloat16)
    outs = []
    for attach in (False, True):
        C = torch.full((M, N), 7.0, device=DEV)
        cs = torch.full((N + 3,), -1.0, device=DEV)
        _gemm(Aop, B, C, M, N, K, lda, N, N, True, False, False, P, stream, a_bits=bits,
              col_sum=(src, cs) if attach else None)
        if not attach:
            _lib.call("myelin_col_sum_f32", _lib.ptr(src), _lib.ptr(cs), 97, N + 3, 0, stream)
        outs.append((C, cs))
    assert torch.equal(outs[0][0], outs[1][0])
    assert torch.equal(outs[0][1], outs[1][1])
    assert torch.allclose(outs[1][1], src.sum(0), rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("M,N,K", [(1024, 4096, 1440), (784, 2048, 12800), (40, 24, 96)])
def test_gemm_parts_with_attached_col_sum_equals_the_two_launches(M, N, K):
    _print_case(test="gemm_parts_col_sum", M=M, N=N, K=K)
    from myelin_amd.linear import _gemm_parts

    g = seeded(M + N + K + 1)
    stream = _lib.stream(torch.device(DEV))
    A = (torch.rand(K, M, generator=g) < 0.3).to(torch.bfloat16).to(DEV)
    Bf = torch.randn(K, N, generator=g).to(DEV)
    B3 = torch.empty(3 * K * N, dtype=torch.bfloat16, device=DEV)
    _lib.call("myelin_split_bf16x3", _lib.ptr(Bf), _lib.ptr(B3), K, N, 0, stream)
    src = torch.randn(33, N, generator=g).to(DEV)
    outs = []
    for attach in (False, True):
        C = torch.zeros((M, N), device=DEV)
        cs = torch.zeros((N,), device=DEV)
        _gemm_parts(A, B3, 3, K * N, C, M, N, K, M, N, N, True, False, False, stream,
                    col_sum=(src, cs) if attach else None)
        if not attach:
            _lib.call("myelin_col_sum_f32", _lib.ptr(src), _lib.ptr(cs), 33, N, 0, stream)
        outs.append((C, cs))
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])


@pytest.mark.parametrize("M,N,K", [(8, 8, 8), (72, 40, 104), (128, 128, 64), (304, 264, 1000), (256, 384, 3000),
                                   (520, 136, 200), (8200, 1032, 72)])
@pytest.mark.parametrize("ta,tb", [(False, False), (False, True), (True, False), (True, True)])
def test_gemm_bf16_operands(M, N, K, ta, tb):
    """bf16 operands in memory: within 1e-5 of the float64 product of the
    bf16 values, and bit-identical to the same values passed as fp32 when
    neither call splits K (both run one k order)."""

    _print_case(test="gemm_bf16_operands", M=M, N=N, K=K, ta=ta, tb=tb)
    g = seeded(M * 5 + N * 11 + K)
    A = _bf16(torch.randn((K, M) if ta else (M, K), generator=g))
    B = _bf16(torch.randn((N, K) if tb else (K, N), generator=g))
    ref = (A.t() if ta else A).double() @ (B.t() if tb else B).double()
    stream = _lib.stream(torch.device(DEV))
    C = torch.empty(M, N, device=DEV)
    Ah, Bh = A.to(DEV).to(torch.bfloat16), B.to(DEV).to(torch.bfloat16)
    _gemm(Ah, Bh, C, M, N, K, A.shape[1], B.shape[1], N, ta, tb, False, _lib.PREC["bf16"], stream)
    assert_norm_close(C.cpu().double(), ref, 1e-5, "C")
    if K < 512:
        C32 = torch.empty(M, N, device=DEV)
        _gemm(A.to(DEV), B.to(DEV), C32, M, N, K, A.shape[1], B.shape[1], N, ta, tb, False, _lib.PREC["bf16"], stream)
        assert torch.equal(C, C32)


def test_gemm_bf16_operands_misaligned_rows_are_rejected():
    stream = _lib.stream(torch.device(DEV))
    A = torch.zeros(16, 20, dtype=torch.bfloat16, device=DEV)  # k-contiguous rows of 40 bytes
    B = torch.zeros(20, 16, dtype=torch.bfloat16, device=DEV)
    C = torch.empty(16, 16, device=DEV)
    with pytest.raises(ValueError, match="aligned"):
        _gemm(A, B, C, 16, 16, 20, 20, 16, 16, False, False, False, _lib.PREC["bf16"], stream)
    with pytest.raises(ValueError, match="bf16 precision"):
        _gemm(A[:, :16], B[:16], C, 16, 16, 16, 20, 16, 16, False, False, False, _lib.PREC["fp32"], stream)


@pytest.mark.parametrize("T,B,F,N", [(13, 20, 200, 304), (9, 48, 96, 256), (5, 7, 64, 128), (20, 3, 48, 64)])
def test_fused_forward_bf16_operands_match_fp32_operands(T, B, F, N):
    _print_case(test="fused_bf16_operands", T=T, B=B, F=F, N=N)
    g = seeded(T * 77 + N)
    x = (torch.rand(T, B, F, generator=g) < 0.4).float().to(DEV)
    w = _bf16((torch.rand(F, N, generator=g) - 0.4) * 0.5).to(DEV)
    bias = (torch.rand(N, generator=g) * 0.1).to(DEV)
    stream = _lib.stream(torch.device(DEV))
    from myelin_amd.linear import _cast_bf16, _transpose_bf16
    res = []
    for half in (False, True):
        m = torch.empty(B, N, device=DEV)
        s = torch.empty(T, B, N, device=DEV)
        pre = torch.empty(T, B, N, device=DEV)
        tail = (_lib.ptr(bias), None, _lib.ptr(m), _lib.ptr(s), _lib.ptr(pre), None, None, None, T, B, F, N, 0, T, 1,
                0.9, 0.6, -0.1, 5.0, _lib.RULE_THRESHOLD)
        if half:
            xh, wt = _cast_bf16(x, stream), _transpose_bf16(w, stream)
            _lib.call("myelin_linear_lif_fwd_bf16", _lib.ptr(xh), _lib.ptr(wt), *tail, stream)
        else:
            _lib.call("myelin_linear_lif_fwd", _lib.ptr(x), _lib.ptr(w), *tail, _lib.PREC["bf16"], stream)
        res.append((m.cpu(), s.cpu(), pre.cpu()))
    for a, b in zip(*res):
        assert torch.equal(a, b)


@pytest.mark.parametrize("M,N,K", [(1, 1, 1), (70, 33, 100), (300, 17, 784), (64, 100, 33), (100, 300, 500),
                                   (1000, 100, 2048), (4096, 20, 6400), (200, 300, 20), (130, 32, 64)])
@pytest.mark.parametrize("ta,tb", [(False, False), (False, True), (True, False), (True, True)])
@pytest.mark.parametrize("prec", ["fp32", "bf16"])
def test_gemm_packed_bit_operand_equals_dense(M, N, K, ta, tb, prec):
    """A given as packed spike words (the readout input of the packed-hidden
    network) gives the same bits as the same 0/1 matrix given densely: both
    run the same kernel (narrow-output, small-K or 64 x 64, by shape) with
    the same k order and K split, and 0/1 is exact in either MFMA input
    type."""

    _print_case(test="gemm_bits", M=M, N=N, K=K, ta=ta, tb=tb, prec=prec)
    g = seeded(M + 3 * N + 5 * K)
    A = (torch.rand((K, M) if ta else (M, K), generator=g) < 0.2).float()
    B = torch.randn((N, K) if tb else (K, N), generator=g)
    bias = torch.randn(N, generator=g).to(DEV)
    Ad, Bd = A.to(DEV), B.to(DEV)
    words = myelin.pack_spikes(Ad).data
    # a word array with slack columns: lda is the row pitch in words
    wide = torch.full((words.shape[0], words.shape[1] + 3), -1, dtype=torch.int32, device=DEV)
    wide[:, :words.shape[1]] = words
    stream = _lib.stream(torch.device(DEV))
    C0 = torch.randn(M, N, generator=g).to(DEV)
    for acc in (False, True):
        dense, bits, bits_wide = C0.clone(), C0.clone(), C0.clone()
        args = (M, N, K)
        _gemm(Ad, Bd, dense, *args, A.shape[1], B.shape[1], N, ta, tb, acc, _lib.PREC[prec], stream, bias=bias)
        _gemm(words, Bd, bits, *args, words.shape[1], B.shape[1], N, ta, tb, acc, _lib.PREC[prec], stream,
              bias=bias, a_bits=True)
        _gemm(wide, Bd, bits_wide, *args, wide.shape[1], B.shape[1], N, ta, tb, acc, _lib.PREC[prec], stream,
              bias=bias, a_bits=True)
        assert torch.equal(bits, dense)
        assert torch.equal(bits_wide, dense)


@pytest.mark.parametrize("K", [4096, 40000])
@pytest.mark.parametrize("bits", [False, True])
@pytest.mark.parametrize("prec", ["fp32", "bf16"])
def test_narrow_gemm_rows_independent_of_m(bits, prec, K):
    """The narrow-output kernel (N <= 32) splits K by K alone, so rows
    computed in a call of their own equal the same rows of one call over all
    of them, bit for bit: a readout's currents do not depend on how its
    caller divides the time steps (all at once, or a group of checkpoint
    chunks at a time).  At fp32 precision it also checks the exact
    three-plane split against float64.  K = 40000 takes the cap of 64
    splits, so each split spans 640 k and ends in a partial sub-chunk."""

    _print_case(test="narrow_rows", bits=bits, prec=prec, K=K)
    M, N = (6400 if K == 4096 else 3000), 20
    g = seeded(K + int(bits) + 2 * (prec == "fp32"))
    A = (torch.rand(M, K, generator=g) < 0.1).float()
    W = (torch.rand(K, N, generator=g) - 0.5) / 32
    Ad, Wd = A.to(DEV), W.to(DEV)
    op = myelin.pack_spikes(Ad).data if bits else Ad
    lda = op.shape[1]
    stream = _lib.stream(torch.device(DEV))

    def run(r0, r1):
        C = torch.empty(r1 - r0, N, device=DEV)
        _gemm(op[r0:r1], Wd, C, r1 - r0, N, K, lda, N, N, False, False, False, _lib.PREC[prec], stream,
              a_bits=bits)
        return C

    full = run(0, M)
    for r0, r1 in ((0, M * 9 // 20), (M * 9 // 20, M * 9 // 10), (M * 9 // 10, M), (17, 18)):
        assert torch.equal(run(r0, r1), full[r0:r1]), (r0, r1)
    if prec == "fp32":
        ref = A.double() @ W.double()
        assert_norm_close(full.cpu().double(), ref, 1e-6, "narrow fp32 (exact split) vs float64")


@pytest.mark.parametrize("prec", ["fp32", "bf16"])
@pytest.mark.parametrize("M,K", [(4096, 64000), (4056, 63993)])
def test_transposed_bit_operand_at_readout_scale(prec, M, K):
    """dW_o = S^T G_o of the 4096 -> 20 readout at T = 2000, B = 32 (K =
    64000 batch-step rows in 63 K splits; the transposed packed-bit operand
    runs its own kernel, which turns 32 x 32 bit blocks around across lanes)
    and a ragged variant (a partial word column and workgroup, a partial
    last group), each also with rows of an odd word pitch: the same bits as
    the same 0/1 matrix given densely, and at fp32 precision within 1e-6 of
    float64.  (Shapes under one round of the chip's workgroups run the
    four-wave kernels; the small-shape bits test covers those.)"""

    N = 20
    _print_case(test="bits_transposed", M=M, K=K, prec=prec)
    g = torch.Generator(device=DEV).manual_seed(M + K + 2 * (prec == "fp32"))
    Ad = (torch.rand(K, M, generator=g, device=DEV) < 0.1).float()
    Bd = torch.randn(K, N, generator=g, device=DEV) * 1e-3
    bias = torch.randn(N, generator=g, device=DEV)
    words = myelin.pack_spikes(Ad).data
    # the same words in rows with 3 slack words (an odd pitch: one word per
    # load instead of a lane's four columns in one 16-byte load)
    wide = torch.full((K, words.shape[1] + 3), -1, dtype=torch.int32, device=DEV)
    wide[:, :words.shape[1]] = words
    stream = _lib.stream(torch.device(DEV))
    for acc in (False, True):
        C0 = torch.randn(M, N, generator=g, device=DEV)
        dense, bits, bits_wide = C0.clone(), C0.clone(), C0.clone()
        _gemm(Ad, Bd, dense, M, N, K, M, N, N, True, False, acc, _lib.PREC[prec], stream, bias=bias)
        _gemm(words, Bd, bits, M, N, K, words.shape[1], N, N, True, False, acc, _lib.PREC[prec], stream, bias=bias,
              a_bits=True)
        _gemm(wide, Bd, bits_wide, M, N, K, wide.shape[1], N, N, True, False, acc, _lib.PREC[prec], stream,
              bias=bias, a_bits=True)
        assert_same_bits(bits, dense, f"transposed bits, accumulate={acc}")
        assert_same_bits(bits_wide, dense, f"transposed bits, padded rows, accumulate={acc}")
    if prec == "fp32":
        C = torch.empty(M, N, device=DEV)
        _gemm(words, Bd, C, M, N, K, words.shape[1], N, N, True, False, False, _lib.PREC[prec], stream, a_bits=True)
        ref = Ad.double().t() @ Bd.double()
        assert_norm_close(C.double(), ref, 1e-6, "transposed bits (exact split) vs float64")


def test_gemm_packed_bit_operand_checks():
    stream = _lib.stream(torch.device(DEV))
    words = torch.zeros(16, 2, dtype=torch.int32, device=DEV)
    B = torch.zeros(40, 8, device=DEV)
    C = torch.empty(16, 8, device=DEV)
    with pytest.raises(ValueError, match="words per row"):
        _gemm(words, B, C, 16, 8, 40, 1, 8, 8, False, False, False, _lib.PREC["fp32"], stream, a_bits=True)
    with pytest.raises(ValueError, match="float32 B"):
        _gemm(words, B.to(torch.bfloat16), C, 16, 8, 40, 2, 8, 8, False, False, False, _lib.PREC["bf16"], stream,
              a_bits=True)


@pytest.mark.parametrize("prec", ["fp32", "bf16"])
def test_checkpoint_recompute_reproduces_forward_trace_exactly(prec):
    """The backward recomputes each checkpoint chunk's currents over that
    chunk's rows only; its pre-reset trace must equal the forward's bit for
    bit (as the reference's per-step recompute does).  Shape chosen so the
    forward GEMM (8192 rows, 512 tiles) and a chunk's (128 rows, 8 tiles)
    would split K differently if the current GEMMs were allowed to split."""

    from myelin_amd.linear import _cast_bf16, _half, _lif_fwd, _transpose_bf16

    _print_case(test="recompute_exact", prec=prec)
    T, B, F, N, C = 1024, 8, 256, 1024, 16
    g = seeded(17)
    x = (torch.rand(T, B, F, generator=g) < 0.2).float().to(DEV)
    w = ((torch.rand(F, N, generator=g) - 0.4) * 0.2).to(DEV)
    b = (torch.rand(N, generator=g) * 0.05).to(DEV)
    stream = _lib.stream(torch.device(DEV))
    p = _lib.PREC[prec]
    half = _half(p, F, N)
    xs, wt = (_cast_bf16(x, stream), _transpose_bf16(w, stream)) if half else (x, None)
    args = (0.95, 1.0, 0.0, 5.0, _lib.RULE_THRESHOLD, p, stream)
    pre = torch.empty(T, B, N, device=DEV)
    ck = torch.empty(T // C, B, N, device=DEV)
    _lif_fwd(xs, w, b, None, 0, T, *args, pre=pre, ckpt=ck, ckpt_every=C, wt=wt, exact=True)
    scratch = torch.empty(C, B, N, device=DEV)
    for k in (0, 1, 37, T // C - 1):
        _lif_fwd(xs, w, b, ck[k], k * C, (k + 1) * C, *args, pre=scratch, wt=wt, exact=True)
        assert torch.equal(scratch, pre[k * C:(k + 1) * C]), f"chunk {k}"


@pytest.mark.parametrize("C", [5, 6])
@pytest.mark.parametrize("rate", [False, True])
@pytest.mark.parametrize("prec", ["fp32", "bf16"])
def test_small_budget_spans_and_forward_chunks_agree_with_one_span(monkeypatch, C, rate, prec):
    """With the currents budget shrunk to 20 steps, the forward walks six
    GEMM chunks (each GEMM on the side stream beside the previous chunk's
    recurrence) and keeps the last backward span's trace, and the backward
    walks spans of several chunks (C = 6: 18-step spans, so the kept trace
    starts inside a forward chunk).  Spikes, rates and dX must equal the
    one-span run bit for bit; dW and db differ only in summation order."""

    from myelin_amd import linear as L

    _print_case(test="small_budget_spans", C=C, rate=rate, prec=prec)
    T, B, F, N = 103, 4, 64, 96
    g = seeded(C * 11 + rate)
    x = (torch.rand(T, B, F, generator=g) < 0.3).float()
    w = (torch.rand(F, N, generator=g) - 0.45) * 0.5
    b = torch.rand(N, generator=g) * 0.1
    go = torch.randn((B, N) if rate else (T, B, N), generator=g)
    res = []
    for budget in (None, 20 * B * N):
        if budget is not None:
            monkeypatch.setattr(L, "_CURRENT_CHUNK_ELEMS", budget)
        xd, wd, bd = (t.to(DEV).requires_grad_() for t in (x, w, b))
        fn = myelin.linear_surrogate_lif_rate_forward if rate else myelin.linear_surrogate_lif_forward
        kw = {"reduction": "none"} if rate else {}
        _, out = fn(xd, wd, bd, P, surrogate="atan", surrogate_slope=4.0, checkpoint_size=C,
                    synapse_precision=prec, **kw)
        out.backward(go.to(DEV))
        torch.cuda.synchronize()
        res.append((to_np(out), to_np(xd.grad), to_np(wd.grad), to_np(bd.grad)))
    assert 0.0 < res[0][0].mean() < 1.0
    assert np.array_equal(res[1][0], res[0][0]) and np.array_equal(res[1][1], res[0][1])
    assert_norm_close(res[1][2], res[0][2], 1e-6, "grad_w across span sizes")
    assert_norm_close(res[1][3], res[0][3], 1e-6, "grad_b across span sizes")


@pytest.mark.parametrize("gdt", ["fp32", "bf16", "planes"])
@pytest.mark.parametrize("with_gs", [False, True])
def test_reverse_pass_two_neurons_per_lane_equals_one(gdt, with_gs):
    """linear_pre_bwd takes two neurons per lane on wide grids (>= 65536
    neurons) when every operand is 8-byte aligned; the same data one float
    off that alignment runs one neuron per lane.  G, the carried gradient
    and the bias partials agree bit for bit."""

    _print_case(test="pre_bwd_lanes", gdt=gdt, with_gs=with_gs)
    C, BN = 37, 66002
    g = seeded(41)
    pre = torch.randn(C * BN, generator=g) + 0.8
    gs = torch.randn(C * BN, generator=g)
    grate = torch.randn(BN, generator=g)
    gm0 = torch.randn(BN, generator=g)
    dt = {"fp32": _lib.DT[torch.float32], "bf16": _lib.DT[torch.bfloat16], "planes": _lib.DT_BF16X3}[gdt]
    gdtype = torch.float32 if gdt == "fp32" else torch.bfloat16
    glen = C * BN * (3 if gdt == "planes" else 1)
    stream = _lib.stream(torch.device(DEV))
    outs = []
    for off in (0, 1):
        def place(t, dtype=torch.float32):
            buf = torch.zeros(t.numel() + 2, dtype=dtype, device=DEV)
            buf[off:off + t.numel()] = t.to(DEV, dtype)
            return buf[off:off + t.numel()]
        p_, s_, r_, m_ = place(pre), place(gs), place(grate), place(gm0)
        gb = place(torch.zeros(BN))
        G = place(torch.zeros(glen), gdtype)
        _lib.call("myelin_linear_pre_bwd", _lib.ptr(p_), _lib.ptr(s_) if with_gs else None, _lib.ptr(r_),
                  _lib.ptr(m_), _lib.ptr(G), dt, _lib.ptr(gb), C, BN, 50, 0.9, 1.0, -0.1, 4.0, 2, 0, stream)
        outs.append((G.cpu(), m_.cpu(), gb.cpu()))
    for a, b in zip(outs[0], outs[1]):
        assert torch.equal(a, b)


@pytest.mark.parametrize("BN", [640, 66002])
@pytest.mark.parametrize("gdt", ["fp32", "planes"])
def test_reverse_pass_without_adjoint_buffer_equals_zero_started(BN, gdt):
    """grad_m NULL makes linear_pre_bwd a whole reverse pass: the adjoint
    starts at zero and the bias sums are written, not accumulated.  G and
    the bias sums equal a launch on zero-filled buffers bit for bit (one and
    two neurons per lane)."""

    _print_case(test="pre_bwd_whole", BN=BN, gdt=gdt)
    C = 29
    g = seeded(BN + 7)
    pre = (torch.randn(C * BN, generator=g) + 0.8).to(DEV)
    gs = torch.randn(C * BN, generator=g).to(DEV)
    dt = {"fp32": _lib.DT[torch.float32], "planes": _lib.DT_BF16X3}[gdt]
    gdtype = torch.float32 if gdt == "fp32" else torch.bfloat16
    glen = C * BN * (3 if gdt == "planes" else 1)
    stream = _lib.stream(torch.device(DEV))
    outs = []
    for whole in (False, True):
        gm = None if whole else torch.zeros(BN, device=DEV)
        gb = torch.full((BN,), float("nan"), device=DEV) if whole else torch.zeros(BN, device=DEV)
        G = torch.empty(glen, dtype=gdtype, device=DEV)
        _lib.call("myelin_linear_pre_bwd", _lib.ptr(pre), _lib.ptr(gs), None, _lib.ptr(gm), _lib.ptr(G), dt,
                  _lib.ptr(gb), C, BN, C, 0.9, 1.0, 0.0, 4.0, 4, 0, stream)
        outs.append((G.cpu(), gb.cpu()))
    for a, b in zip(outs[0], outs[1]):
        assert torch.equal(a, b)
