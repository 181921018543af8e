"""Write golden input/output vectors from djsaunde/myelin's torch backend.

Run in the build container only (it reads the reference checkout):

    python tests/golden/make_golden.py [/path/to/reference]

Covers the functions whose results no closed form or library routine pins
on its own: the linear stream / checkpoint / checkpoint-rate autograd
Functions (autograd.py:445-923) at chunk edges with and without bias and
with both reductions, the surrogate LIF / ALIF unroll gradients for every
surrogate (functional.py:115-189), and every dim variant of
packed_spike_count / packed_spike_rate (packing.py:84-162), and the
two-layer whole-model-recompute rate network (autograd.py:926-1126,
kernels.py:779-808) at several checkpoint sizes.  The fixtures
are plain arrays (inputs and the reference's outputs) in .npz files next to
this script; nothing from the reference is copied.
"""

from __future__ import annotations

import itertools
import pathlib
import sys

import numpy as np
import torch

HERE = pathlib.Path(__file__).resolve().parent


def _np(t):
    return t.detach().cpu().numpy()


def main(ref_root: str) -> None:
    src = pathlib.Path(ref_root).resolve() / "src"
    sys.path.insert(0, str(src))
    import myelin

    # this repository's `myelin` alias package must not stand in for the reference here
    if not pathlib.Path(myelin.__file__).resolve().is_relative_to(src):
        raise RuntimeError(f"`import myelin` resolved to {myelin.__file__}, not the reference under {src}")
    from myelin import packing as P
    from myelin.functional import surrogate_alif_unroll, surrogate_lif_unroll
    from myelin.kernels import linear_surrogate_lif_forward, linear_surrogate_lif_rate_forward
    from myelin.neurons import ALIFParams, ALIFState, LIFParams, LIFState
    from myelin.surrogates import SURROGATE_NAMES, surrogate_from_name

    # ---------------------------------------------------------------- packing
    out = {}
    for i, shape in enumerate([(3, 2, 35), (2, 3, 5, 33), (4, 64)]):
        g = torch.Generator().manual_seed(100 + i)
        s = (torch.rand(shape, generator=g) < 0.3).float()
        pk = P.pack_spikes(s)
        out[f"s{i}"] = _np(s)
        out[f"words{i}"] = _np(pk.data)
        nd = len(shape)
        dims_list = [None] + [d for r in range(1, nd + 1) for d in itertools.combinations(range(nd), r)]
        for dims in dims_list:
            tag = "none" if dims is None else "_".join(map(str, dims))
            c = P.packed_spike_count(pk, dim=dims)
            out[f"count{i}_{tag}"] = _np(c)
            out[f"rate{i}_{tag}"] = _np(P.packed_spike_rate(pk, dim=dims))
            out[f"rate64{i}_{tag}"] = _np(P.packed_spike_rate(pk, dim=dims, dtype=torch.float64))
            if dims is None or (nd - 1) in dims:
                out[f"counts{i}_{tag}"] = _np(P.packed_spike_counts(pk, dim=dims))
        out[f"unpack{i}"] = _np(P.unpack_spikes(pk))
    np.savez_compressed(HERE / "packing_counts.npz", **out)

    # ---------------------------------------------------------------- unrolls
    out = {}
    g = torch.Generator().manual_seed(7)
    T, B, N = 12, 2, 9
    x = 0.25 + 0.6 * torch.randn(T, B, N, generator=g)
    m0 = 0.1 * torch.randn(B, N, generator=g)
    a0 = 0.2 * torch.rand(B, N, generator=g)
    gs = torch.randn(T, B, N, generator=g)
    gm = torch.randn(B, N, generator=g)
    ga = torch.randn(B, N, generator=g)
    for k, v in dict(x=x, m0=m0, a0=a0, gs=gs, gm=gm, ga=ga).items():
        out[k] = _np(v)
    ap = ALIFParams(tau_mem=20.0, tau_adaptation=50.0, threshold=1.0, reset=0.0, beta=1.8)
    lp = LIFParams(tau_mem=8.0, threshold=0.7, reset=-0.2)
    for name in SURROGATE_NAMES:
        xr, mr, ar = (t.clone().requires_grad_() for t in (x, m0, a0))
        st, s = surrogate_alif_unroll(xr, ALIFState(mr, ar), ap, surrogate=surrogate_from_name(name),
                                      surrogate_slope=10.0)
        torch.autograd.backward([s, st.membrane, st.adaptation], [gs, gm, ga])
        for k, v in dict(s=s, mT=st.membrane, aT=st.adaptation, gx=xr.grad, gm0=mr.grad, ga0=ar.grad).items():
            out[f"alif_{name}_{k}"] = _np(v)
        xr, mr = x.clone().requires_grad_(), m0.clone().requires_grad_()
        st, s = surrogate_lif_unroll(xr, LIFState(mr), lp, surrogate=surrogate_from_name(name), surrogate_slope=4.0)
        torch.autograd.backward([s, st.membrane], [gs, gm])
        for k, v in dict(s=s, mT=st.membrane, gx=xr.grad, gm0=mr.grad).items():
            out[f"lif_{name}_{k}"] = _np(v)
    np.savez_compressed(HERE / "surrogate_unrolls.npz", **out)

    # ---------------------------------------------------------------- linear
    out = {}
    g = torch.Generator().manual_seed(11)
    T, B, F, N = 9, 3, 11, 17
    x = (torch.rand(T, B, F, generator=g) < 0.3).float()
    w = (torch.rand(F, N, generator=g) - 0.5) * 0.6
    b = torch.rand(N, generator=g) * 0.1
    gsp = torch.randn(T, B, N, generator=g)
    gfin = torch.randn(B, N, generator=g)
    grate = torch.randn(B, N, generator=g)
    for k, v in dict(x=x, w=w, b=b, gs=gsp, gfin=gfin, grate=grate).items():
        out[k] = _np(v)
    p = LIFParams(tau_mem=9.0, threshold=0.7, reset=-0.2)

    def leaves(bias: bool):
        xr, wr = x.clone().requires_grad_(), w.clone().requires_grad_()
        br = b.clone().requires_grad_() if bias else None
        return xr, wr, br

    for bias in (False, True):
        bt = "b" if bias else "nob"
        # streamed (checkpoint_size=None) and checkpointed spike outputs
        for ck in (None, 1, 4, 9):
            for with_final in (False, True):
                xr, wr, br = leaves(bias)
                st, s = linear_surrogate_lif_forward(xr, wr, br, p, surrogate="atan", surrogate_slope=5.0,
                                                     backend="torch", checkpoint_size=ck)
                outs, grads = [s], [gsp]
                if with_final:
                    outs.append(st.membrane)
                    grads.append(gfin)
                torch.autograd.backward(outs, grads)
                tag = f"spk_{bt}_c{ck}_f{int(with_final)}"
                out[f"{tag}_s"] = _np(s)
                out[f"{tag}_mT"] = _np(st.membrane)
                out[f"{tag}_gx"] = _np(xr.grad)
                out[f"{tag}_gw"] = _np(wr.grad)
                if bias:
                    out[f"{tag}_gb"] = _np(br.grad)
        # rate readout
        for ck in (1, 4, 9):
            for red in ("none", "mean"):
                xr, wr, br = leaves(bias)
                st, r = linear_surrogate_lif_rate_forward(xr, wr, br, p, surrogate="superspike", surrogate_slope=5.0,
                                                          backend="torch", checkpoint_size=ck, reduction=red)
                if red == "none":
                    r.backward(grate)
                else:
                    r.backward()
                tag = f"rate_{bt}_c{ck}_{red}"
                out[f"{tag}_r"] = _np(r)
                out[f"{tag}_mT"] = _np(st.membrane)
                out[f"{tag}_gx"] = _np(xr.grad)
                out[f"{tag}_gw"] = _np(wr.grad)
                if bias:
                    out[f"{tag}_gb"] = _np(br.grad)
    np.savez_compressed(HERE / "linear_paths.npz", **out)

    # ------------------------------------------------------ two-layer rate
    from myelin.kernels import two_layer_surrogate_lif_rate_recompute_forward

    out = {}
    g = torch.Generator().manual_seed(12)
    T, B, F, H, O = 11, 3, 13, 37, 5
    x = (torch.rand(T, B, F, generator=g) < 0.35).float()
    wh = (torch.rand(F, H, generator=g) - 0.3) * 0.9
    bh = torch.rand(H, generator=g) * 0.1
    wo = (torch.rand(H, O, generator=g) - 0.45) * 0.6
    bo = torch.rand(O, generator=g) * 0.1
    grate = torch.randn(B, O, generator=g)
    for k, v in dict(x=x, wh=wh, bh=bh, wo=wo, bo=bo, grate=grate).items():
        out[k] = _np(v)
    p = LIFParams(tau_mem=6.0, threshold=0.6, reset=-0.1)
    for bias in (False, True):
        for ck in (1, 4, 11):
            for sg in ("fast_sigmoid", "superspike"):
                xr, whr, wor = (t.clone().requires_grad_() for t in (x, wh, wo))
                bhr = bh.clone().requires_grad_() if bias else None
                bor = bo.clone().requires_grad_() if bias else None
                r = two_layer_surrogate_lif_rate_recompute_forward(
                    xr, whr, bhr, wor, bor, p, surrogate=sg, surrogate_slope=5.0, checkpoint_size=ck)
                r.backward(grate)
                tag = f"{'b' if bias else 'nob'}_c{ck}_{sg}"
                out[f"{tag}_r"] = _np(r)
                out[f"{tag}_gx"] = _np(xr.grad)
                out[f"{tag}_gwh"] = _np(whr.grad)
                out[f"{tag}_gwo"] = _np(wor.grad)
                if bias:
                    out[f"{tag}_gbh"] = _np(bhr.grad)
                    out[f"{tag}_gbo"] = _np(bor.grad)
    np.savez_compressed(HERE / "two_layer_rate.npz", **out)
    print("wrote", sorted(p.name for p in HERE.glob("*.npz")))


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
