"""Pin the oracle (CPU) against the reference's own vectors, independent
library routines and brute force.  No GPU needed."""

from __future__ import annotations

import json
import pathlib

import numpy as np
import pytest
import torch

from oracle import c_ref
from oracle import torch_ref as R
from tests.helpers import seeded

VEC = json.loads((pathlib.Path(__file__).parent / "golden" / "reference_vectors.json").read_text())


def test_lif_step_vector():
    v = VEC["lif_step"]
    x = torch.tensor([v["inputs"]])
    m, s = R.lif_unroll(x, torch.tensor(v["membrane"]), v["tau_mem"], v["threshold"], v["reset"])
    assert torch.equal(s[0], torch.tensor(v["spikes"]))
    assert torch.allclose(m, torch.tensor(v["next_membrane"]))
    cm, cs = c_ref.lif_fwd(x.numpy(), np.array(v["membrane"], np.float32),
                           np.float32(R.decay_from_tau(v["tau_mem"])), v["threshold"], v["reset"])
    assert np.array_equal(cs[0], np.array(v["spikes"], np.float32))
    assert np.array_equal(cm, m.numpy())


@pytest.mark.parametrize("key", ["alif_step_no_spike", "alif_step_spike"])
def test_alif_step_vectors(key):
    v = VEC[key]
    x = torch.tensor([v["inputs"]])
    m, a, s = R.alif_unroll(x, torch.tensor(v["membrane"]), torch.tensor(v["adaptation"]),
                            v["tau_mem"], v["tau_adaptation"], v["threshold"], v["reset"], v["beta"])
    assert torch.equal(s[0], torch.tensor(v["spikes"]))
    assert torch.allclose(m, torch.tensor(v["next_membrane"]))
    assert torch.allclose(a, torch.tensor(v["next_adaptation"]))
    cm, ca, cs = c_ref.alif_fwd(
        x.numpy(), np.array(v["membrane"], np.float32), np.array(v["adaptation"], np.float32),
        np.float32(R.decay_from_tau(v["tau_mem"])), np.float32(R.decay_from_tau(v["tau_adaptation"])),
        v["threshold"], v["beta"], v["reset"],
    )
    assert np.array_equal(cm, m.numpy()) and np.array_equal(ca, a.numpy()) and np.array_equal(cs, s.numpy())


def _f32(v: float) -> float:
    return float(np.float32(v))


def _brute_alif(x, m0, a0, d, rho, thr, beta, reset):
    """Python-float loop, rounding to fp32 after every operation."""

    T, B, N = x.shape
    s = np.zeros_like(x)
    m = m0.copy()
    a = a0.copy()
    for b in range(B):
        for n in range(N):
            mm, aa = float(m[b, n]), float(a[b, n])
            for t in range(T):
                mm = _f32(_f32(mm * d) + float(x[t, b, n]))
                th = _f32(thr + _f32(beta * aa))
                sp = mm >= th
                s[t, b, n] = 1.0 if sp else 0.0
                if sp:
                    mm = reset
                aa = _f32(_f32(aa * rho) + (1.0 if sp else 0.0))
            m[b, n], a[b, n] = mm, aa
    return m, a, s


def test_alif_unroll_matches_brute_force():
    g = seeded(11)
    x = 0.25 + 0.6 * torch.randn(40, 2, 7, generator=g)
    m0 = 0.2 * torch.randn(2, 7, generator=g)
    a0 = 0.3 * torch.rand(2, 7, generator=g)
    d = _f32(R.decay_from_tau(20.0))
    rho = _f32(R.decay_from_tau(50.0))
    m, a, s = R.alif_unroll(x, m0, a0, 20.0, 50.0, 1.0, 0.0, 1.8)
    bm, ba, bs = _brute_alif(x.numpy(), m0.numpy(), a0.numpy(), d, rho, 1.0, _f32(1.8), 0.0)
    assert np.array_equal(bs, s.numpy())
    assert np.array_equal(bm, m.numpy())
    assert np.array_equal(ba, a.numpy())


@pytest.mark.parametrize("seed", [0, 1])
def test_c_and_torch_oracles_agree_bitwise(seed):
    g = seeded(seed)
    x = 0.3 + 0.5 * torch.randn(100, 4, 65, generator=g)
    m0 = 0.1 * torch.randn(4, 65, generator=g)
    m, s = R.lif_unroll(x, m0, 10.0, 1.0, 0.0)
    cm, cs = c_ref.lif_fwd(x.numpy(), m0.numpy(), np.float32(R.decay_from_tau(10.0)), 1.0, 0.0)
    assert np.array_equal(cs, s.numpy()) and np.array_equal(cm, m.numpy())
    a0 = 0.2 * torch.rand(4, 65, generator=g)
    m, a, s = R.alif_unroll(x, m0, a0, 20.0, 50.0, 1.0, 0.0, 1.8)
    cm, ca, cs = c_ref.alif_fwd(x.numpy(), m0.numpy(), a0.numpy(), np.float32(R.decay_from_tau(20.0)),
                                np.float32(R.decay_from_tau(50.0)), 1.0, 1.8, 0.0)
    assert np.array_equal(cs, s.numpy()) and np.array_equal(cm, m.numpy()) and np.array_equal(ca, a.numpy())


def test_surrogate_forward_decision_matches_plain_unroll():
    """slope*(m' - th) >= 0 is the same decision as m' >= th for slope > 0."""

    g = seeded(5)
    x = 0.25 + 0.6 * torch.randn(50, 3, 33, generator=g)
    z = torch.zeros(3, 33)
    _, _, s_plain = R.alif_unroll(x, z, z, 20.0, 50.0, 1.0, 0.0, 1.8)
    _, _, s_sur = R.surrogate_alif_unroll(x, z, z, 20.0, 50.0, 1.0, 0.0, 1.8, "fast_sigmoid", 10.0)
    # the straight-through value is (H + sigma) - sigma, within 1 ulp of H
    assert torch.all((s_sur - s_plain).abs() <= 6e-8)


def test_checkpoint_policy_vectors():
    v = VEC["checkpoint_policy"]
    assert R.recommended_checkpoint_size(v["T"], "memory") == v["memory"]
    assert R.recommended_checkpoint_size(v["T"], "balanced") == v["balanced"]
    assert R.recommended_checkpoint_size(v["T"], "speed") == v["speed"]
    assert R.resolve_checkpoint_size(v["resolve_T"], v["resolve_size"]) == v["resolved"]
    assert R.recommended_checkpoint_size(2000, "memory") == 45  # ceil(sqrt(2000))
    with pytest.raises(ValueError, match="positive"):
        R.resolve_checkpoint_size(10, 0)


# ---------------------------------------------------------------- surrogates
HAND = {
    # sigma'(c) at c = 0.5 from the closed forms, evaluated by hand
    "fast_sigmoid": 0.5 / 1.5**2,
    "superspike": 1.0 / 1.5**2,
    "atan": 0.5 / (1.0 + (np.pi * 0.5 / 2.0) ** 2),
    "sigmoid": (1 / (1 + np.exp(-0.5))) * (1 - 1 / (1 + np.exp(-0.5))),
    "triangular": -1.0,
    "multi_gaussian": 0.6 * np.exp(-0.5) / (0.5 * np.sqrt(2 * np.pi))
    + 0.2 * np.exp(-0.125) / np.sqrt(2 * np.pi)
    + 0.2 * np.exp(-1.125) / np.sqrt(2 * np.pi),
}


@pytest.mark.parametrize("name", R.SURROGATE_NAMES)
def test_surrogate_derivative_is_derivative_of_primitive(name):
    c = torch.linspace(-3.0, 3.0, 601, dtype=torch.float64)
    c = c[(c.abs() - 1.0).abs() > 1e-9]  # triangular kinks at |c| = 1
    c = c[c != 0]
    cc = c.clone().requires_grad_()
    (auto,) = torch.autograd.grad(R.surrogate_primitive(name, cc).sum(), cc)
    closed = R.surrogate_derivative(name, c)
    assert torch.allclose(auto, closed, rtol=1e-10, atol=1e-12)
    assert abs(float(R.surrogate_derivative(name, torch.tensor([0.5], dtype=torch.float64))) - HAND[name]) < 1e-12


@pytest.mark.parametrize("name", ["fast_sigmoid", "superspike", "atan"])
def test_surrogate_derivative_of_huge_arguments_is_zero(name):
    """fp32 sigma'(c) once (1 + |c|)^2 (or 1 + (pi c / 2)^2) overflows: 0,
    not NaN, in both restatements (the kernels' reciprocal is held to the
    same on the GPU)."""

    c = torch.tensor([3e19, -3e19, 1e30, -1e38, float("inf")], dtype=torch.float32)
    d = R.surrogate_derivative(name, c)
    assert torch.equal(d, torch.zeros_like(d))
    x = np.array([[[1e20]], [[0.0]]], dtype=np.float32)  # c = 10 (m' - 1) ~ 1e21 at step 0
    zeros = np.zeros((1, 1), dtype=np.float32)
    gx, _ = c_ref.lif_bwd(x, zeros, np.ones_like(x), zeros, np.float32(R.decay_from_tau(20.0)), 1.0, 0.0, 10.0,
                          name)
    assert np.isfinite(gx).all()
    assert gx[0, 0, 0] == 0.0


def test_multi_gaussian_derivative_integrates_to_one():
    c = torch.linspace(-12, 12, 240001, dtype=torch.float64)
    area = torch.trapezoid(R.surrogate_derivative("multi_gaussian", c), c)
    assert abs(float(area) - 1.0) < 1e-9


# ---------------------------------------------------------------- packing
def test_pack_high_bit_vector():
    v = VEC["pack_high_bit"]
    s = torch.zeros(v["spikes_shape"])
    s[tuple(v["one_at"])] = 1.0
    data, shape = R.pack_spikes(s)
    assert data.item() == v["word"]
    assert c_ref.pack(s.numpy()).item() == v["word"]
    assert torch.equal(R.unpack_spikes(data, shape), s)


def test_pack_nonzero_vector():
    v = VEC["pack_nonzero"]
    data, shape = R.pack_spikes(torch.tensor(v["spikes"]))
    assert torch.equal(R.unpack_spikes(data, shape), torch.tensor(v["unpacked"]))


def test_count_ignores_padding_vector():
    v = VEC["count_ignores_padding"]
    data = torch.tensor(v["words"], dtype=torch.int32)
    shape = tuple(v["original_shape"])
    assert torch.equal(R.packed_spike_counts(data, shape), torch.tensor(v["row_counts"]))
    assert R.packed_spike_count(data, shape).item() == v["total"]
    assert R.packed_spike_rate(data, shape).item() == v["rate"]
    assert np.array_equal(c_ref.row_counts(data.numpy(), shape[-1]), np.array(v["row_counts"]))


@pytest.mark.parametrize("n", [1, 5, 31, 32, 33, 35, 64, 65, 100])
def test_pack_matches_numpy_packbits(n):
    g = seeded(n)
    s = (torch.rand(3, 4, n, generator=g) < 0.3).float()
    data, shape = R.pack_spikes(s)
    w = (n + 31) // 32
    bits = np.zeros((3, 4, w * 32), np.uint8)
    bits[..., :n] = s.numpy().astype(np.uint8)
    ref = np.packbits(bits, axis=-1, bitorder="little").view("<i4").reshape(3, 4, w)
    assert np.array_equal(data.numpy(), ref)
    assert np.array_equal(c_ref.pack(s.numpy()), ref)
    assert torch.equal(R.unpack_spikes(data, shape), s)
    assert np.array_equal(c_ref.unpack(ref, n), s.numpy())
    # counts against numpy popcount of the dense bits
    assert np.array_equal(R.packed_spike_counts(data, shape).numpy(), s.numpy().sum(-1).astype(np.int64))
    assert np.array_equal(c_ref.row_counts(ref, n), s.numpy().sum(-1).astype(np.int64))


def test_count_dims_vectors():
    v = VEC["count_dims"]
    s = torch.zeros(v["shape"])
    for idx in v["ones"]:
        s[tuple(idx)] = 1.0
    data, shape = R.pack_spikes(s)
    for dim in [0, 1, -1, (0, 1), (0, -1), (1, -1), (0, 1, 2)]:
        dims = (dim,) if isinstance(dim, int) else dim
        dims = tuple(d % 3 for d in dims)
        assert torch.equal(R.packed_spike_count(data, shape, dim), s.sum(dim=dims).to(torch.int64))
    assert R.packed_spike_count(data, shape).item() == len(v["ones"])
    with pytest.raises(ValueError, match="last dimension"):
        R.packed_spike_counts(data, shape, 0)
    with pytest.raises(ValueError, match="duplicate"):
        R.packed_spike_count(data, shape, (0, -3))


def test_compression_vector():
    v = VEC["compression"]
    n = v["shape"][-1]
    assert v["shape"][0] * v["shape"][1] * n * 4 == v["dense_bytes"]
    assert v["shape"][0] * v["shape"][1] * R.packed_words(n) * 4 == v["packed_bytes"]
    assert v["dense_bytes"] / v["packed_bytes"] == v["ratio"]
