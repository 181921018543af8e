"""A whole training step (streamed-synapse hidden layer + rate readout +
cross-entropy, forward and backward) captured in one HIP graph: every
replay must equal the eager step bit for bit (loss and all gradients),
with eager work and synchronisations between the replays.  bench.py times
the 784 -> 2048 -> 10 step this way.
"""

from __future__ import annotations

import pytest
import torch

import myelin_amd as myelin
from tests.helpers import assert_same_bits, seeded

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _print_case(**kw):
    print("case:", " ".join(f"{k}={v}" for k, v in kw.items()), flush=True)


@pytest.mark.parametrize("T,B,F,H,O,prec", [(12, 64, 96, 256, 10, "bf16"), (20, 32, 64, 128, 7, "fp32")])
def test_training_step_replays_equal_eager(T, B, F, H, O, prec):
    _print_case(test="graph_capture", T=T, B=B, F=F, H=H, O=O, prec=prec)
    g = seeded(T * B + F + H)
    x = (torch.rand(T, B, F, generator=g) < 0.2).float().to(DEV)
    labels = torch.randint(0, O, (B,), generator=g).to(DEV)
    torch.manual_seed(5)
    hidden = myelin.LinearSurrogateLIF(F, H, surrogate=myelin.atan_surrogate, stream_synapse=True,
                                       synapse_precision=prec).to(DEV)
    readout = myelin.LinearSurrogateLIFRate(H, O, surrogate=myelin.atan_surrogate, checkpoint_size=T,
                                            synapse_precision=prec).to(DEV)
    with torch.no_grad():
        for mod, fan in ((hidden, F), (readout, H)):
            mod.synapse.weight.uniform_(-(6.0 / fan) ** 0.5, (6.0 / fan) ** 0.5)
    params = list(hidden.parameters()) + list(readout.parameters())

    def body():
        rates = readout(hidden(x))
        loss = torch.nn.functional.cross_entropy(rates * T, labels)
        loss.backward()
        return loss

    for q in params:
        q.grad = None
    loss_e = body().detach().clone()
    grads_e = [q.grad.clone() for q in params]
    assert bool(loss_e.isfinite())

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            for q in params:
                q.grad = None
            body()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    for q in params:
        q.grad = None
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        loss_g = body()
    for rep in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert_same_bits(loss_g, loss_e, f"loss, replay {rep}")
        for i, (q, ge) in enumerate(zip(params, grads_e)):
            assert_same_bits(q.grad, ge, f"grad {i}, replay {rep}")
        _ = float((x * 2.0).sum())  # eager work between replays
