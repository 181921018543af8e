"""Host-side checks of the compile-visible rate operators: registration,
fake-tensor shape rules and the reference's validation wording
(triton/compile_ops.py, kernels.py:637-684).  No GPU calls."""

from __future__ import annotations

import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode

import myelin_amd as myelin
from myelin_amd import compile_ops


def test_operators_are_registered_in_their_namespace():
    for name in ("linear_lif_checkpoint_rate_forward_no_bias", "linear_lif_checkpoint_rate_forward_bias",
                 "linear_lif_checkpoint_rate_grads_no_bias", "linear_lif_checkpoint_rate_grads_bias"):
        assert hasattr(torch.ops.myelin_amd, name)


@pytest.mark.parametrize("T,ck,chunks", [(7, 3, 3), (6, 3, 2), (1, 5, 1)])
def test_fake_shapes(T, ck, chunks):
    with FakeTensorMode():
        x, w, b = torch.empty(T, 3, 5), torch.empty(5, 4), torch.empty(4)
        m, r, c = compile_ops.linear_lif_checkpoint_rate_forward_bias_op(x, w, b, 0.9, 1.0, 0.0, 5.0, ck, 16, 32, 32)
        assert m.shape == (3, 4) and r.shape == (3, 4) and c.shape == (chunks, 3, 4)
        gx, gw, gb = compile_ops.linear_lif_checkpoint_rate_grads_bias_op(
            x, w, b, c, m, r, 0.9, 1.0, 0.0, 5.0, ck, 16, 32, 32)
        assert gx.shape == x.shape and gw.shape == w.shape and gb.shape == b.shape


def test_triton_compile_backend_validation_matches_reference():
    x, w = torch.zeros(4, 2, 3), torch.zeros(3, 5)
    p = myelin.LIFParams()
    with pytest.raises(ValueError, match="only surrogate='fast_sigmoid'"):
        myelin.linear_surrogate_lif_rate_forward(x, w, None, p, surrogate="atan", backend="triton_compile")
    with pytest.raises(ValueError, match="only hard_forward=True"):
        myelin.linear_surrogate_lif_rate_forward(x, w, None, p, surrogate="fast_sigmoid", hard_forward=False,
                                                 backend="triton_compile")
