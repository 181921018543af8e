"""GPU parity of the bitpacking kernels: bit-exact against the oracle
(oracle.torch_ref restating myelin.packing) for words, unpacked values,
counts (int64) and rates."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import myelin_amd as myelin
from oracle import torch_ref as R
from tests.helpers import seeded

pytestmark = pytest.mark.gpu
DEV = "cuda"
SHAPES = [(1,), (3, 2, 1), (3, 2, 31), (3, 2, 32), (3, 2, 33), (2, 3, 35), (4, 65), (2, 2, 2, 100), (5, 64),
          (7, 3, 130)]


def _print_case(**kw):
    print("case:", " ".join(f"{k}={v}" for k, v in kw.items()), flush=True)


def _spikes(shape, seed, p=0.3):
    g = seeded(seed)
    return (torch.rand(shape, generator=g) < p).float()


@pytest.mark.parametrize("shape", SHAPES)
def test_pack_unpack_round_trip_bit_exact(shape):
    _print_case(test="pack", shape=shape)
    s = _spikes(shape, sum(shape))
    words, oshape = R.pack_spikes(s)
    pk = myelin.pack_spikes(s.to(DEV))
    assert pk.original_shape == oshape
    assert pk.data.dtype == torch.int32
    assert torch.equal(pk.data.cpu(), words)
    assert torch.equal(myelin.unpack_spikes(pk).cpu(), s)


@pytest.mark.parametrize(
    "dtype", [torch.float32, torch.float16, torch.bfloat16, torch.bool, torch.uint8, torch.int8, torch.int32,
              torch.int64, torch.float64]
)
def test_pack_dtypes(dtype):
    _print_case(test="pack_dtype", dtype=dtype)
    g = seeded(3)
    v = (torch.rand(4, 3, 45, generator=g) * 3).floor() - 1.0  # values in {-1, 0, 1}
    s = v.to(dtype)
    words, _ = R.pack_spikes(s)
    pk = myelin.pack_spikes(s.to(DEV))
    assert torch.equal(pk.data.cpu(), words)
    out = myelin.unpack_spikes(pk, dtype=dtype)
    assert out.dtype == dtype
    assert torch.equal(out.cpu(), R.unpack_spikes(words, tuple(s.shape), dtype))


def test_pack_signed_zero_nan_and_high_bit():
    _print_case(test="pack_special")
    s = torch.zeros(2, 64)
    s[0, 1] = -0.0
    s[0, 2] = float("nan")
    s[0, 3] = 2.0
    s[0, 31] = 1.0
    s[1, 63] = -3.0
    words, _ = R.pack_spikes(s)
    pk = myelin.pack_spikes(s.to(DEV))
    assert torch.equal(pk.data.cpu(), words)
    assert pk.data[0, 0].item() == (1 << 2) + (1 << 3) - (1 << 31)
    h = s.to(torch.bfloat16)
    assert torch.equal(myelin.pack_spikes(h.to(DEV)).data.cpu(), R.pack_spikes(h)[0])


# the last three reduce >= 16 rows onto each output, which takes the
# atomic-free block kernel when the kept leading dims are contiguous
@pytest.mark.parametrize("shape", [(3, 2, 35), (4, 3, 64), (2, 3, 5, 33), (6, 100), (40, 6, 5, 70), (300, 4, 100),
                                   (64, 3, 2100)])
def test_counts_and_rates_every_dim_bit_exact(shape):
    _print_case(test="counts", shape=shape)
    s = _spikes(shape, 11 + len(shape))
    words, oshape = R.pack_spikes(s)
    pk = myelin.pack_spikes(s.to(DEV))
    nd = len(shape)
    dims_list = [None, -1, 0]
    import itertools

    for r in range(1, nd + 1):
        dims_list += list(itertools.combinations(range(nd), r))
    for dims in dims_list:
        ref = R.packed_spike_count(words, oshape, dims)
        got = myelin.packed_spike_count(pk, dim=dims)
        assert got.dtype == torch.int64
        assert torch.equal(got.cpu(), ref), dims
        for dt in (torch.float32, torch.float64):
            assert torch.equal(myelin.packed_spike_rate(pk, dim=dims, dtype=dt).cpu(),
                               R.packed_spike_rate(words, oshape, dims, dt)), (dims, dt)
        if dims is None or (nd - 1) in [d % nd for d in ((dims,) if isinstance(dims, int) else dims)]:
            assert torch.equal(myelin.packed_spike_counts(pk, dim=dims).cpu(),
                               R.packed_spike_counts(words, oshape, dims))


def test_counts_ignore_padding_bits():
    _print_case(test="padding")
    pk = myelin.PackedSpikes(data=torch.tensor([[[-1, -1]]], dtype=torch.int32, device=DEV),
                             original_shape=(1, 1, 35))
    assert myelin.packed_spike_counts(pk).cpu().tolist() == [[35]]
    assert myelin.packed_spike_count(pk).item() == 35
    assert myelin.packed_spike_rate(pk).item() == 1.0
    assert myelin.packed_spike_count(pk, dim=0).cpu().tolist() == [[1] * 35]


def test_counts_many_rows_use_atomic_blocks():
    """More rows than one block covers (2040) in the keep-last count path."""

    _print_case(test="keep_last_many_rows")
    s = _spikes((4100, 3, 40), 5, p=0.5)
    words, oshape = R.pack_spikes(s)
    pk = myelin.pack_spikes(s.to(DEV))
    assert torch.equal(myelin.packed_spike_count(pk, dim=0).cpu(), R.packed_spike_count(words, oshape, 0))
    assert torch.equal(myelin.packed_spike_count(pk, dim=(0, 1)).cpu(),
                       R.packed_spike_count(words, oshape, (0, 1)))


def test_bitpack_config_full_size():
    """Spikes [512, 64, 8192], Bernoulli with per-neuron rate LogNormal(-3, 1)
    clipped to [0, 1]: pack, unpack round trip, per-neuron counts over T,
    per-sample rates.  Size-independent properties over the whole tensor,
    oracle equality on a slice of samples."""

    _print_case(test="bitpack_full")
    T, B, N = 512, 64, 8192
    g = seeded(5)
    rate = torch.exp(-3.0 + torch.randn(N, generator=g)).clamp(0.0, 1.0)
    gd = torch.Generator(device=DEV).manual_seed(5)
    s = (torch.rand((T, B, N), generator=gd, device=DEV) < rate.to(DEV)).float()
    pk = myelin.pack_spikes(s)
    assert torch.equal(myelin.unpack_spikes(pk), s)
    counts = myelin.packed_spike_count(pk, dim=0)
    assert torch.equal(counts, s.sum(0).to(torch.int64))
    rates = myelin.packed_spike_rate(pk, dim=(0, -1))
    assert torch.equal(rates, s.sum((0, 2)).to(torch.int64).to(torch.float32) / (T * N))
    rows = [0, 31, 63]
    ss = s[:, rows].cpu()
    words, oshape = R.pack_spikes(ss)
    assert torch.equal(pk.data[:, rows].cpu(), words)
    assert torch.equal(counts[rows].cpu(), R.packed_spike_count(words, oshape, 0))
    assert torch.equal(rates[rows].cpu(), R.packed_spike_rate(words, oshape, (0, -1)))
    bits = np.packbits(ss.numpy().astype(np.uint8), axis=-1, bitorder="little").view("<i4")
    assert np.array_equal(pk.data[:, rows].cpu().numpy(), bits)
