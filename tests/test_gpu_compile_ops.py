"""GPU checks of the compile-visible rate operators: eager results equal the
default HIP rate path; ``torch.compile(fullgraph=True)`` traces through them
(fake rules + registered autograd) with the same values and gradients; and
``torch.library.opcheck`` accepts the operators."""

from __future__ import annotations

import pytest
import torch

import myelin_amd as myelin
from myelin_amd import compile_ops
from tests.helpers import assert_norm_close, seeded, to_np

pytestmark = pytest.mark.gpu
DEV = "cuda"
P = myelin.LIFParams(tau_mem=8.0, threshold=0.7, reset=-0.2)


def _print_case(**kw):
    print("case:", " ".join(f"{k}={v}" for k, v in kw.items()), flush=True)


def _net(seed, T=11, B=4, F=24, N=9):
    g = seeded(seed)
    x = (torch.rand(T, B, F, generator=g) < 0.4).float().to(DEV)
    w = ((torch.rand(F, N, generator=g) - 0.4) * 0.6).to(DEV)
    b = (torch.rand(N, generator=g) * 0.1).to(DEV)
    target = torch.rand(B, N, generator=g).to(DEV)
    return x, w, b, target


def _run(backend, x, w, b, target, ck):
    xs, ws = x.clone().requires_grad_(), w.clone().requires_grad_()
    bs = None if b is None else b.clone().requires_grad_()
    st, r = myelin.linear_surrogate_lif_rate_forward(xs, ws, bs, P, surrogate="fast_sigmoid", surrogate_slope=5.0,
                                                     checkpoint_size=ck, reduction="none", backend=backend)
    loss = ((r - target) ** 2).sum() + 0.1 * st.membrane.sum()
    loss.backward()
    return [r, st.membrane, xs.grad, ws.grad] + ([] if b is None else [bs.grad])


@pytest.mark.parametrize("bias", [False, True])
@pytest.mark.parametrize("ck", [1, 4, 11])
def test_eager_operators_equal_default_path(bias, ck):
    _print_case(test="compile_ops_eager", bias=bias, ck=ck)
    x, w, b, target = _net(ck + 10 * bias)
    b = b if bias else None
    got = _run("triton_compile", x, w, b, target, ck)
    ref = _run("hip", x, w, b, target, ck)
    for a, e in zip(got, ref):
        assert torch.equal(a, e)


@pytest.mark.parametrize("bias", [False, True])
def test_torch_compile_traces_through_the_operators(bias):
    _print_case(test="compile_ops_torch_compile", bias=bias)
    x, w, b, target = _net(3)
    b = b if bias else None

    def loss_fn(xs, ws, bs):
        st, r = myelin.linear_surrogate_lif_rate_forward(xs, ws, bs, P, surrogate="fast_sigmoid",
                                                         surrogate_slope=5.0, checkpoint_size=4, reduction="none",
                                                         backend="triton_compile")
        return ((r - target) ** 2).sum() + 0.1 * st.membrane.sum()

    compiled = torch.compile(loss_fn, backend="aot_eager", fullgraph=True)
    leaves = [x.clone().requires_grad_(), w.clone().requires_grad_()] + (
        [] if b is None else [b.clone().requires_grad_()])
    loss = compiled(*leaves, *([] if b is not None else [None]))
    loss.backward()
    ref = _run("triton_compile", x, w, b, target, 4)
    eager_loss = ((ref[0] - target) ** 2).sum() + 0.1 * ref[1].sum()
    assert_norm_close(to_np(loss), to_np(eager_loss), 1e-6, "loss")
    for leaf, e in zip(leaves, ref[2:]):
        assert torch.equal(leaf.grad, e)


def test_opcheck_accepts_the_operators():
    _print_case(test="compile_ops_opcheck")
    x, w, b, _ = _net(5, T=6, B=3, F=8, N=5)
    args = (x, w.requires_grad_(), 0.9, 0.7, -0.2, 5.0, 3, 16, 32, 32)
    torch.library.opcheck(compile_ops.linear_lif_checkpoint_rate_forward_no_bias_op, args)
    args_b = (x, w, b.requires_grad_(), 0.9, 0.7, -0.2, 5.0, 3, 16, 32, 32)
    torch.library.opcheck(compile_ops.linear_lif_checkpoint_rate_forward_bias_op, args_b)
