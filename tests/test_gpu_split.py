"""GPU parity of the exact bf16 split of the fp32 synapse.

When a layer's input is bf16-exact (spikes), ``x @ W`` runs as
``x @ W_hi + x @ W_mid + x @ W_lo`` on the bf16 MFMA, with the three planes
summing exactly to W.  Bars:
* the planes (W and the reverse pass's G) sum back to the fp32 value bit
  for bit, and the checked cast flags every non-exact input;
* the multi-part GEMM within 1e-5 (max-norm relative) of the float64
  product of the unsplit operands, so within fp32 GEMM accuracy;
* layers on the split path against the oracle as the fp32 layers are:
  rasters >= 99.99 % equal, membranes within 1e-5, gradients within 1e-5,
  and against the fp32-engine run of the same layer within 1e-5;
* a checkpointed recompute on the split path equals the forward's trace
  bit for bit.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import myelin_amd as myelin
from myelin_amd import _lib
from myelin_amd import linear as L
from oracle import torch_ref as R
from tests.helpers import assert_elementwise_close, assert_norm_close, norm_rel_err, raster_agreement, seeded, to_np

pytestmark = pytest.mark.gpu
DEV = "cuda"
P = myelin.LIFParams(tau_mem=9.0, threshold=0.7, reset=-0.2)


def _print_case(**kw):
    print("case:", " ".join(f"{k}={v}" for k, v in kw.items()), flush=True)


def _planes_sum(planes):
    """float(hi) + float(mid) + float(lo) in fp32, in that order."""

    f = planes.float()
    return (f[0] + f[1]) + f[2]


@pytest.mark.parametrize("transpose", [0, 1])
def test_split_planes_sum_back_exactly(transpose):
    _print_case(test="split_planes", transpose=transpose)
    g = seeded(31 + transpose)
    rows, cols = 130, 77
    w = torch.randn(rows, cols, generator=g) * torch.exp2(torch.randint(-40, 40, (rows, cols), generator=g).float())
    w[0, :4] = torch.tensor([0.0, -0.0, 1.0, -3.0])
    wd = w.to(DEV)
    out = torch.empty(3 * rows * cols, dtype=torch.bfloat16, device=DEV)
    _lib.call("myelin_split_bf16x3", _lib.ptr(wd), _lib.ptr(out), rows, cols, transpose, _lib.stream(wd.device))
    planes = out.view(3, cols, rows) if transpose else out.view(3, rows, cols)
    back = _planes_sum(planes).cpu()
    assert torch.equal(back.t() if transpose else back, w)
    # the high plane is the nearest bf16 value, as torch rounds
    hi = planes[0].cpu()
    assert torch.equal(hi.t() if transpose else hi, w.to(torch.bfloat16))


def test_split_of_non_finite_values_keeps_them_in_the_high_plane():
    _print_case(test="split_non_finite")
    w = torch.tensor([[float("inf"), -float("inf"), 2.5, float("nan")]], device=DEV)
    out = torch.empty(12, dtype=torch.bfloat16, device=DEV)
    _lib.call("myelin_split_bf16x3", _lib.ptr(w), _lib.ptr(out), 1, 4, 0, _lib.stream(w.device))
    p = out.view(3, 4).float().cpu()
    assert p[0, 0] == float("inf") and p[0, 1] == -float("inf") and p[0, 2] == 2.5 and torch.isnan(p[0, 3])
    assert torch.equal(p[1:, :2], torch.zeros(2, 2))


@pytest.mark.parametrize("case", ["spikes", "integers", "odd_integer", "random", "denormal", "nan", "tail"])
def test_checked_cast_flags_exactly_the_inexact_inputs(case):
    _print_case(test="checked_cast", case=case)
    g = seeded(7)
    n = 4099 if case == "tail" else 4096
    x = (torch.rand(n, generator=g) < 0.1).float()
    expect = 0
    if case == "integers":
        x = torch.randint(-256, 257, (n,), generator=g).float()  # 8 significant bits: |k| <= 256 are exact
    elif case == "odd_integer":
        x[9] = 257.0  # needs 9 significant bits
        expect = 1
    elif case == "random":
        x = torch.randn(n, generator=g)
        expect = 1
    elif case == "denormal":
        x[17] = 1e-40
        expect = 1
    elif case == "nan":
        x[4000] = float("nan")
        expect = 1
    elif case == "tail":
        x[n - 1] = 0.1  # in the scalar tail of the last thread
        expect = 1
    xd = x.to(DEV)
    xb = torch.empty(n, dtype=torch.bfloat16, device=DEV)
    flag = torch.zeros(1, dtype=torch.int32, device=DEV)
    _lib.call("myelin_cast_bf16_checked", _lib.ptr(xd), _lib.ptr(xb), n, _lib.ptr(flag), _lib.stream(xd.device))
    assert int(flag.item()) == expect
    got, want = xb.cpu(), x.to(torch.bfloat16)
    nan = torch.isnan(want)
    assert torch.equal(torch.isnan(got), nan) and torch.equal(got[~nan], want[~nan])


# bf16 rows: k-contiguous ones a multiple of 8 elements, mn-contiguous ones of 4
@pytest.mark.parametrize("M,N,K", [(128, 128, 64), (300, 260, 1000), (136, 132, 72), (64, 200, 3000),
                                   (1000, 136, 24)])
@pytest.mark.parametrize("ta,tb", [(False, False), (False, True), (True, False), (True, True)])
@pytest.mark.parametrize("parts", [1, 3])
def test_gemm_parts_matches_float64(M, N, K, ta, tb, parts):
    _print_case(test="gemm_parts", M=M, N=N, K=K, ta=ta, tb=tb, parts=parts)
    g = seeded(M + 3 * N + 7 * K + parts)
    A = torch.randn((K, M) if ta else (M, K), generator=g).to(torch.bfloat16)
    Bs = torch.randn((parts, N, K) if tb else (parts, K, N), generator=g).to(torch.bfloat16)
    bias = torch.randn(N, generator=g)
    C0 = torch.randn(M, N, generator=g)
    a64 = (A.t() if ta else A).double()
    ref = sum(a64 @ (Bs[p].t() if tb else Bs[p]).double() for p in range(parts))
    stream = _lib.stream(torch.device(DEV))
    Ad, Bd = A.to(DEV), Bs.to(DEV)
    for acc in (False, True):
        for split in (False, True):
            C = C0.clone().to(DEV)
            L._gemm_parts(Ad, Bd, parts, Bs[0].numel(), C, M, N, K, M if ta else K, K if tb else N, N, ta, tb, acc,
                          stream, bias=bias.to(DEV), split=split)
            want = ref + bias.double() + (C0.double() if acc else 0.0)
            assert_norm_close(to_np(C), want.numpy(), 1e-5, f"acc={acc} split={split}")


def test_gemm_parts_equals_the_concatenated_k_product():
    """Three parts sum like one product over K' = 3K whose A repeats and whose
    B stacks the parts last to first (each part's k range in turn, from the
    last part, K a whole number of 64-wide stages): the same stages in the
    same order, so bit for bit."""

    _print_case(test="gemm_parts_concat")
    M, N, K = 512, 384, 512
    g = seeded(99)
    A = (torch.rand(M, K, generator=g) < 0.3).to(torch.bfloat16)
    Bs = torch.randn(3, K, N, generator=g).to(torch.bfloat16)
    stream = _lib.stream(torch.device(DEV))
    C1 = torch.empty(M, N, device=DEV)
    L._gemm_parts(A.to(DEV), Bs.to(DEV), 3, K * N, C1, M, N, K, K, N, N, False, False, False, stream, split=False)
    A3 = torch.cat([A, A, A], dim=1).to(DEV)
    C2 = torch.empty(M, N, device=DEV)
    L._gemm(A3, Bs.flip(0).reshape(3 * K, N).to(DEV), C2, M, N, 3 * K, 3 * K, N, N, False, False, False,
            _lib.PREC["bf16"], stream, split=False)
    assert torch.equal(C1, C2)


def test_split_synapse_sums_the_smallest_plane_first():
    """The three planes of an exact split summed smallest first: spike inputs
    [8000 x 1024] times an fp32 W [1024 x 4096] (config 4's hidden synapse
    on 4 batch rows) lie within 1.5e-7 (max-norm relative) of the float64
    product, closer than a plain fp32 GEMM of the same operands (torch's on
    the GPU: 3.7e-7 measured; the planes summed largest first: 5.3e-7;
    smallest first: 6.8e-8)."""

    _print_case(test="split_order_accuracy")
    g = seeded(40)
    M, K, N = 8000, 1024, 4096
    x = (torch.rand(M, K, generator=g) < 0.05).float()
    w = torch.empty(K, N).uniform_(-(6 / K) ** 0.5, (6 / K) ** 0.5, generator=g)
    ref = x.double() @ w.double()
    stream = _lib.stream(torch.device(DEV))
    wd = w.to(DEV)
    w3 = torch.empty((3, N, K), dtype=torch.bfloat16, device=DEV)
    _lib.call("myelin_split_bf16x3", wd.data_ptr(), w3.data_ptr(), K, N, 1, stream)
    cur = torch.empty(M, N, device=DEV)
    L._gemm_parts(x.to(DEV).to(torch.bfloat16), w3, 3, N * K, cur, M, N, K, K, K, N, False, True, False, stream,
                  split=False)
    plain = x.to(DEV) @ wd
    torch.cuda.synchronize()
    e_split = norm_rel_err(cur.cpu(), ref)
    e_plain = norm_rel_err(plain.cpu(), ref)
    print(f"split {e_split:.2e}, plain fp32 GEMM {e_plain:.2e}", flush=True)
    assert e_split <= 1.5e-7
    assert e_split < e_plain


def test_reverse_pass_planes_sum_to_the_fp32_gradient():
    _print_case(test="pre_bwd_planes")
    C, BN = 37, 3000
    g = seeded(5)
    pre = (torch.randn(C, BN, generator=g) + 0.7).to(DEV)
    gs = torch.randn(C, BN, generator=g).to(DEV)
    stream = _lib.stream(torch.device(DEV))
    outs = []
    for dt in (_lib.DT[torch.float32], _lib.DT_BF16X3):
        gm = torch.zeros(BN, device=DEV)
        G = torch.empty(C * BN * (3 if dt == _lib.DT_BF16X3 else 1), device=DEV,
                        dtype=torch.bfloat16 if dt == _lib.DT_BF16X3 else torch.float32)
        _lib.call("myelin_linear_pre_bwd", _lib.ptr(pre), _lib.ptr(gs), None, _lib.ptr(gm), _lib.ptr(G), dt, None,
                  C, BN, C, 0.9, 1.0, 0.0, 5.0, 2, 0, stream)
        outs.append((G, gm))
    assert torch.equal(_planes_sum(outs[1][0].view(3, C, BN)), outs[0][0].view(C, BN))
    assert torch.equal(outs[1][1], outs[0][1])


def _flips(r1, r2, T):
    """Spikes by which two rate tensors (counts / T) differ."""

    return float(np.rint(np.abs(to_np(r1).astype(np.float64) - to_np(r2).astype(np.float64)) * T).sum())


def _layer_inputs(T, B, F, N, seed):
    g = seeded(seed)
    x = (torch.rand(T, B, F, generator=g) < 0.3).float()
    w = (torch.rand(F, N, generator=g) - 0.45) * 0.5
    b = torch.rand(N, generator=g) * 0.1
    return x, w, b, g


def _run_layer(x, w, b, go, ck, rate, need_x):
    xd = x.to(DEV).requires_grad_(need_x)
    wd, bd = w.to(DEV).requires_grad_(), b.to(DEV).requires_grad_()
    if rate:
        st, out = myelin.linear_surrogate_lif_rate_forward(xd, wd, bd, P, surrogate="atan", surrogate_slope=4.0,
                                                           checkpoint_size=ck, reduction="none")
    else:
        st, out = myelin.linear_surrogate_lif_forward(xd, wd, bd, P, surrogate="atan", surrogate_slope=4.0,
                                                      checkpoint_size=ck)
    out.backward(go.to(DEV))
    return (to_np(out), to_np(st.membrane), None if not need_x else to_np(xd.grad), to_np(wd.grad),
            to_np(bd.grad))


@pytest.mark.parametrize("ck,rate", [(None, False), (5, False), (7, True)])
@pytest.mark.parametrize("need_x", [False, True])
def test_split_layer_matches_oracle_and_fp32_engine(monkeypatch, ck, rate, need_x):
    """A 64 -> 72 layer on binary inputs, split path forced on (no minimum
    size): against the CPU oracle at the fp32 bars, and against the same
    layer on the fp32 engine."""

    _print_case(test="split_layer", ck=ck, rate=rate, need_x=need_x)
    T, B, F, N = 37, 5, 64, 72
    x, w, b, g = _layer_inputs(T, B, F, N, 40 + (ck or 0) + rate)
    go = torch.randn((B, N) if rate else (T, B, N), generator=g)
    calls = []
    real = L._split_synapse
    monkeypatch.setattr(L, "_split_synapse", lambda *a, **k: calls.append(1) or real(*a, **k))
    monkeypatch.setattr(L, "_SPLIT_MIN_MACS", 0)
    got = _run_layer(x, w, b, go, ck, rate, need_x)
    assert calls, "the split path did not run"
    monkeypatch.setattr(L, "_SPLIT_MIN_MACS", 1 << 62)
    fp32 = _run_layer(x, w, b, go, ck, rate, need_x)
    if rate:
        assert _flips(got[0], fp32[0], T) <= 1e-4 * T * B * N
    else:
        assert raster_agreement(got[0], fp32[0]) >= 0.9999
    for i, what in ((1, "membrane"), (3, "grad_w"), (4, "grad_b")) + (((2, "grad_x"),) if need_x else ()):
        assert_norm_close(got[i], fp32[i], 1e-5, f"{what} vs fp32 engine")
    xr, wr, br = (t.clone().requires_grad_() for t in (x, w, b))
    if rate:
        mT, r = R.linear_surrogate_lif_rate(xr, wr, br, 9.0, 0.7, -0.2, "atan", 4.0, ck, "none")
        r.backward(go)
        assert _flips(got[0], r.detach(), T) <= 1e-4 * T * B * N
    else:
        if ck is None:
            mT, s = R.linear_surrogate_lif_stream(xr, wr, br, 9.0, 0.7, -0.2, "atan", 4.0)
        else:
            mT, s = R.linear_surrogate_lif_checkpoint(xr, wr, br, 9.0, 0.7, -0.2, "atan", 4.0, ck)
        s.backward(go)
        assert raster_agreement(got[0], s) >= 0.9999
    assert_norm_close(got[1], mT.detach(), 1e-5, "membrane vs oracle")
    assert_norm_close(got[3], wr.grad, 1e-5, "grad_w vs oracle")
    assert_norm_close(got[4], br.grad, 1e-5, "grad_b vs oracle")
    if need_x:
        assert_norm_close(got[2], xr.grad, 1e-5, "grad_x vs oracle")


def test_non_exact_inputs_fall_back_to_the_fp32_engine(monkeypatch):
    _print_case(test="split_fallback")
    T, B, F, N = 21, 4, 64, 72
    x, w, b, g = _layer_inputs(T, B, F, N, 77)
    x[3, 1, 5] = 0.3  # not a bf16 value
    go = torch.randn(T, B, N, generator=g)
    monkeypatch.setattr(L, "_SPLIT_MIN_MACS", 0)
    got = _run_layer(x, w, b, go, 4, False, True)
    monkeypatch.setattr(L, "_SPLIT_MIN_MACS", 1 << 62)
    fp32 = _run_layer(x, w, b, go, 4, False, True)
    for a, c in zip(got, fp32):
        assert np.array_equal(a, c)


def test_split_recompute_reproduces_forward_trace_exactly(monkeypatch):
    """The checkpointed backward's recompute on the split path (unsplit K,
    chunk rows only) equals the forward's trace bit for bit."""

    _print_case(test="split_recompute_exact")
    T, B, F, N, C = 512, 8, 256, 1024, 16
    g = seeded(17)
    x = (torch.rand(T, B, F, generator=g) < 0.2).float().to(DEV)
    w = ((torch.rand(F, N, generator=g) - 0.4) * 0.2).to(DEV)
    b = (torch.rand(N, generator=g) * 0.05).to(DEV)
    stream = _lib.stream(torch.device(DEV))
    sp = L._split_synapse(x, w, stream)
    assert sp.exact()
    xb, w3 = sp.xb, sp.w3
    args = (0.95, 1.0, 0.0, 5.0, _lib.RULE_THRESHOLD, _lib.PREC["fp32"], stream)
    pre = torch.empty(T, B, N, device=DEV)
    ck = torch.empty(T // C, B, N, device=DEV)
    L._lif_fwd(xb, w, b, None, 0, T, *args, pre=pre, ckpt=ck, ckpt_every=C, wt=w3, exact=True)
    scratch = torch.empty(C, B, N, device=DEV)
    for k in (0, 1, 17, T // C - 1):
        L._lif_fwd(xb, w, b, ck[k], k * C, (k + 1) * C, *args, pre=scratch, wt=w3, exact=True)
        assert torch.equal(scratch, pre[k * C:(k + 1) * C]), f"chunk {k}"


@pytest.mark.parametrize("variant", ["recompute", "packed"])
@pytest.mark.parametrize("need_x", [False, True])
def test_two_layer_hidden_split_matches_fp32_engine_and_oracle(monkeypatch, variant, need_x):
    """The two-layer network's hidden synapse on the split path (binary
    inputs, forced on): rates and gradients against the fp32-engine run and
    the oracle."""

    from myelin_amd import two_layer as TL

    _print_case(test="two_layer_split", variant=variant, need_x=need_x)
    T, B, F, H, O, C = 23, 4, 64, 136, 10, 4
    g = seeded(61 + need_x)
    x = (torch.rand(T, B, F, generator=g) < 0.3).float()
    wh = (torch.rand(F, H, generator=g) - 0.4) * 0.5
    bh = torch.rand(H, generator=g) * 0.1
    wo = (torch.rand(H, O, generator=g) - 0.4) * 0.4
    bo = torch.rand(O, generator=g) * 0.1
    grate = torch.randn(B, O, generator=g)
    fn = {"recompute": myelin.two_layer_surrogate_lif_rate_recompute_forward,
          "packed": myelin.two_layer_surrogate_lif_rate_packed_hidden_forward}[variant]
    p = myelin.LIFParams(tau_mem=8.0, threshold=0.7, reset=-0.2)
    calls = []
    real = TL._split_synapse
    monkeypatch.setattr(TL, "_split_synapse", lambda *a, **k: calls.append(1) or real(*a, **k))
    res = []
    for min_macs in (0, 1 << 62):
        monkeypatch.setattr(L, "_SPLIT_MIN_MACS", min_macs)
        leaves = [x.to(DEV).requires_grad_(need_x)] + [t.to(DEV).requires_grad_() for t in (wh, bh, wo, bo)]
        r = fn(*leaves, p, surrogate="fast_sigmoid", surrogate_slope=5.0, checkpoint_size=C)
        r.backward(grate.to(DEV))
        res.append([to_np(r)] + [None if t.grad is None else to_np(t.grad) for t in leaves])
    assert len(calls) == 1, "the split path ran once (the first run)"
    assert _flips(res[0][0], res[1][0], T) <= 1e-4 * T * B * O
    for name, a, b in zip(("x", "wh", "bh", "wo", "bo"), res[0][1:], res[1][1:]):
        if a is not None:
            assert_norm_close(a, b, 1e-5, f"grad_{name} vs fp32 engine")
    lv = [x.clone().requires_grad_(need_x)] + [t.clone().requires_grad_() for t in (wh, bh, wo, bo)]
    rr = R.two_layer_rate(*lv, 8.0, 0.7, -0.2, "fast_sigmoid", 5.0, C)
    rr.backward(grate)
    assert _flips(res[0][0], rr.detach(), T) <= 1e-4 * T * B * O
    if np.array_equal(res[0][0], rr.detach().numpy()):
        for name, a, t in zip(("x", "wh", "bh", "wo", "bo"), res[0][1:], lv):
            if a is not None:
                assert_norm_close(a, t.grad, 1e-5, f"grad_{name} vs oracle")


@pytest.mark.parametrize("parts,K,N,M", [(1, 1000, 1024, 8192), (3, 1000, 1024, 8192), (2, 1024, 1024, 8192),
                                           (3, 1024, 1024, 8192), (3, 1024, 4096, 8192), (3, 1024, 4096, 7200)])
def test_parts_products_do_not_depend_on_the_rows_computed(parts, K, N, M):
    """A 128-row slice of a bf16 product of `parts` parts (no K split)
    equals the same rows of the M-row product bit for bit, as a
    checkpointed recompute needs; and the product is within 1e-5 of float64.
    K = 1000 ends in a partial stage (register-staged tiles throughout);
    with K = 1024 and two or three parts the full product runs on the
    256 x 128 tiles staged by direct global -> LDS loads (N = 1024) or on
    the 256 x 256 ones (N = 4096; at M = 7200, a long-horizon layer's last
    backward span, the last row of tiles is ragged), while the slices run on
    the 128 x 128 register-staged tiles."""

    _print_case(test="parts_rows", parts=parts, K=K, N=N, M=M)
    g = seeded(123 + parts)
    A = torch.randn(M, K, generator=g).to(torch.bfloat16)
    Bs = torch.randn(parts, N, K, generator=g).to(torch.bfloat16)
    bias = torch.randn(N, generator=g)
    Ad, Bd, bd = A.to(DEV), Bs.to(DEV), bias.to(DEV)
    stream = _lib.stream(torch.device(DEV))
    full = torch.empty(M, N, device=DEV)
    L._gemm_parts(Ad, Bd, parts, N * K, full, M, N, K, K, K, N, False, True, False, stream, bias=bd, split=False)
    for r0 in (0, 4000, M - 128):
        sub = torch.empty(128, N, device=DEV)
        L._gemm_parts(Ad[r0:r0 + 128], Bd, parts, N * K, sub, 128, N, K, K, K, N, False, True, False, stream,
                      bias=bd, split=False)
        assert torch.equal(full[r0:r0 + 128], sub), f"rows {r0}"
    rows = torch.tensor([0, 1, 255, 256, 4097, M - 1])
    ref = sum(A[rows].double() @ Bs[p].double().t() for p in range(parts)) + bias.double()
    assert_norm_close(to_np(full[rows.to(DEV)]), ref.numpy(), 1e-5, "parts product vs float64")


@pytest.mark.parametrize("M,N,K,parts,accumulate", [
    (1024, 4096, 1440, 3, True),   # the 1024 -> 4096 layer's span dW at one 45-step chunk, B=32
    (784, 2048, 2560, 1, False),   # the 784 -> 2048 layer's dW shape: split, it runs on 256 x 256 tiles
    (784, 2048, 2600, 3, False),   # the same on three parts, K ending in a partial stage
    (1024, 2048, 1000, 3, True),   # three parts on 256 x 256 tiles, accumulating, partial stage
    (264, 1032, 1000, 3, True),    # ragged tiles, K ending in a partial stage
    (136, 200, 104, 2, False),     # K = 64 + a partial stage of 40
    (128, 128, 40, 3, False),      # a single partial stage per part
    (8, 8, 64, 1, False),          # one piece of columns, clamped reads
])
def test_mn_contiguous_products_equal_the_k_contiguous_ones(M, N, K, parts, accumulate):
    """C (+)= sum_p A^T B_p with A [K, M] and B_p [K, N] stored as the
    weight-gradient products store them (both mn-contiguous: staged into LDS
    as stored and read through the transposing LDS read) equals the same
    product with both operands transposed to k-contiguous first (the other
    staging) bit for bit: without a K split both sum every element over the
    same k sequence.  And it is within 1e-5 of float64."""

    _print_case(test="mn_vs_kc", M=M, N=N, K=K, parts=parts)
    g = seeded(900 + M + parts)
    A = (torch.rand(K, M, generator=g) < 0.2).to(torch.bfloat16)
    Bs = torch.randn(parts, K, N, generator=g).to(torch.bfloat16)
    C0 = torch.randn(M, N, generator=g)
    Ad, Bd = A.to(DEV), Bs.to(DEV)
    At, Bt = Ad.t().contiguous(), Bd.transpose(1, 2).contiguous()
    stream = _lib.stream(torch.device(DEV))
    mn = C0.to(DEV)
    kc = C0.to(DEV)
    L._gemm_parts(Ad, Bd, parts, K * N, mn, M, N, K, M, N, N, True, False, accumulate, stream, split=False)
    L._gemm_parts(At, Bt, parts, N * K, kc, M, N, K, K, K, N, False, True, accumulate, stream, split=False)
    assert torch.equal(mn, kc), "mn-contiguous and k-contiguous products differ"
    ref = sum(A.double().t() @ Bs[p].double() for p in range(parts)) + (C0.double() if accumulate else 0)
    assert_norm_close(to_np(mn), ref.numpy(), 1e-5, "mn-contiguous product vs float64")
    # with a K split (the weight-gradient route; 256 x 256 tiles where the
    # 128 x 128 grid is under one round): within 1e-5 of float64 too, and
    # per element within summation-order noise of the unsplit product (a
    # tile summing the wrong rows or k range is off by O(1))
    sp = C0.to(DEV)
    L._gemm_parts(Ad, Bd, parts, K * N, sp, M, N, K, M, N, N, True, False, accumulate, stream, split=True)
    assert_norm_close(to_np(sp), ref.numpy(), 1e-5, "split mn-contiguous product vs float64")
    assert_elementwise_close(sp, mn, 1e-4, "split vs unsplit, per element", floor=1e-2)


@pytest.mark.parametrize("variant", ["recompute", "packed"])
def test_two_layer_non_exact_input_falls_back_to_the_fp32_engine(monkeypatch, variant):
    """The first group's GEMM runs on the split before the input check
    returns; an input that is not bf16-exact redoes it on the fp32 engine,
    so rates and gradients equal the fp32-engine run bit for bit."""

    _print_case(test="two_layer_split_fallback", variant=variant)
    T, B, F, H, O, C = 23, 4, 64, 136, 10, 4
    g = seeded(71)
    x = (torch.rand(T, B, F, generator=g) < 0.3).float()
    x[0, 2, 7] = 0.3  # not a bf16 value
    wh = (torch.rand(F, H, generator=g) - 0.4) * 0.5
    bh = torch.rand(H, generator=g) * 0.1
    wo = (torch.rand(H, O, generator=g) - 0.4) * 0.4
    bo = torch.rand(O, generator=g) * 0.1
    grate = torch.randn(B, O, generator=g)
    fn = {"recompute": myelin.two_layer_surrogate_lif_rate_recompute_forward,
          "packed": myelin.two_layer_surrogate_lif_rate_packed_hidden_forward}[variant]
    p = myelin.LIFParams(tau_mem=8.0, threshold=0.7, reset=-0.2)
    res = []
    for min_macs in (0, 1 << 62):
        monkeypatch.setattr(L, "_SPLIT_MIN_MACS", min_macs)
        leaves = [t.to(DEV).requires_grad_() for t in (x, wh, bh, wo, bo)]
        r = fn(*leaves, p, surrogate="fast_sigmoid", surrogate_slope=5.0, checkpoint_size=C)
        r.backward(grate.to(DEV))
        res.append([to_np(r)] + [to_np(t.grad) for t in leaves])
    for a, b in zip(res[0], res[1]):
        assert np.array_equal(a, b)


def test_parts_product_mn_layouts_at_a_weight_gradient_shape():
    """dW-shaped three-part product (A transposed, B planes row-major,
    1024 x 4096 x 3*2000) with and without a K split, against float64 on a
    few rows and columns."""

    _print_case(test="parts_dw_shape")
    M, N, K, parts = 1024, 4096, 2000, 3
    g = seeded(321)
    A = (torch.rand(K, M, generator=g) < 0.2).to(torch.bfloat16)  # stored [K, M]: op(A) = A^T
    Bs = torch.randn(parts, K, N, generator=g).to(torch.bfloat16)
    stream = _lib.stream(torch.device(DEV))
    Ad, Bd = A.to(DEV), Bs.to(DEV)
    rows = torch.tensor([0, 5, 511, 1023])
    cols = torch.tensor([0, 77, 2048, 4095])
    ref = sum(A[:, rows].double().t() @ Bs[p][:, cols].double() for p in range(parts))
    outs = []
    for split in (False, True):
        C = torch.empty(M, N, device=DEV)
        L._gemm_parts(Ad, Bd, parts, K * N, C, M, N, K, M, N, N, True, False, False, stream, split=split)
        got = C[rows.to(DEV)][:, cols.to(DEV)]
        assert_norm_close(to_np(got), ref.numpy(), 1e-5, f"split={split}")
        outs.append(C)
    assert_norm_close(to_np(outs[1]), to_np(outs[0]), 1e-6, "split vs unsplit")


def test_split_synapse_is_not_used_under_graph_capture():
    """A layer large enough for the split (2**32 MACs, spike inputs) keeps
    the fp32 engine while a graph is captured -- the split's choice waits on
    the host for the input check, which capture forbids.  The captured
    forward equals the eager forward on the fp32 engine value for value, on
    every replay (eager work in between)."""

    _print_case(test="split_under_capture")
    T, B, F, N = 128, 32, 1024, 1024
    assert not L._fused(B, N) and T * B * F * N >= L._SPLIT_MIN_MACS
    g = seeded(808)
    x = (torch.rand(T, B, F, generator=g) < 0.05).float().to(DEV)
    w = ((torch.rand(F, N, generator=g) - 0.45) * 0.1).to(DEV)
    p = myelin.LIFParams()

    def fwd():
        with torch.no_grad():
            return myelin.linear_surrogate_lif_forward(x, w, None, p, surrogate="superspike")

    calls = []
    real = L._split_synapse
    L._split_synapse = lambda *a, **k: calls.append(1) or real(*a, **k)
    try:
        _, s_eager_split = fwd()  # eager: the split runs
        assert calls, "the split path did not run eagerly"
        calls.clear()
        saved, L._SPLIT_MIN_MACS = L._SPLIT_MIN_MACS, 1 << 62
        try:
            st_ref, s_ref = fwd()  # eager on the fp32 engine
        finally:
            L._SPLIT_MIN_MACS = saved
        torch.cuda.synchronize()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            fwd()  # warm up on a side stream (eager: the split runs)
        torch.cuda.current_stream().wait_stream(side)
        calls.clear()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            st_cap, s_cap = fwd()
        assert not calls, "the split path ran under capture"
    finally:
        L._split_synapse = real
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(s_cap, s_ref) and torch.equal(st_cap.membrane, st_ref.membrane)
        _ = (x * 2.0).sum().item()  # eager work between replays
    assert raster_agreement(s_cap, s_eager_split) >= 0.9999
