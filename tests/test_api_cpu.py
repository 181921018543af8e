"""Host-side behaviour of the public API that needs no GPU: validation,
registries, policies, and the absence of any CPU fallback."""

from __future__ import annotations

import pytest
import torch

import myelin_amd as myelin
from myelin_amd import checkpointing, kernels, packing, surrogates


def test_cpu_tensors_are_rejected_not_run_on_cpu():
    x = torch.zeros(3, 2, 4)
    with pytest.raises(ValueError, match="ROCm device"):
        myelin.lif_forward(x, myelin.LIFState(torch.zeros(2, 4)), myelin.LIFParams())
    with pytest.raises(ValueError, match="ROCm device"):
        myelin.surrogate_alif_forward(
            x, myelin.ALIFState(torch.zeros(2, 4), torch.zeros(2, 4)), myelin.ALIFParams()
        )
    with pytest.raises(ValueError, match="ROCm device"):
        myelin.pack_spikes(x)


def test_shape_and_backend_errors_match_reference_wording():
    with pytest.raises(ValueError, match=r"\[T, B, N\]"):
        myelin.lif_forward(torch.zeros(2, 3), myelin.LIFState(torch.zeros(3)), myelin.LIFParams())
    with pytest.raises(ValueError, match="unsupported backend"):
        myelin.lif_forward(torch.zeros(2, 3, 4), myelin.LIFState(torch.zeros(3, 4)), myelin.LIFParams(),
                           backend="cuda")
    with pytest.raises(ValueError, match="unknown surrogate"):
        myelin.surrogate_lif_forward(torch.zeros(2, 3, 4), myelin.LIFState(torch.zeros(3, 4)),
                                     myelin.LIFParams(), surrogate="relu")


def test_smooth_forward_on_triton_backends_raises_reference_message():
    """hard_forward=False is the torch route in the reference; its Triton
    backends refuse it with these messages (kernels.py:273-276,290-293)."""

    x, st = torch.zeros(2, 3, 4), myelin.LIFState(torch.zeros(3, 4))
    with pytest.raises(ValueError, match="^Triton surrogate LIF currently supports only hard_forward=True$"):
        myelin.surrogate_lif_forward(x, st, myelin.LIFParams(), hard_forward=False, backend="triton")
    with pytest.raises(ValueError, match="^generated Triton surrogate LIF currently supports only hard_forward"):
        myelin.surrogate_lif_forward(x, st, myelin.LIFParams(), hard_forward=False, backend="triton_generated")


def test_backend_selects_the_arithmetic():
    """torch / hard_forward=False / ALIF auto: autograd's arithmetic; the
    fused-kernel arithmetic otherwise (codes per include/myelin_hip.h)."""

    from myelin_amd import _lib

    assert kernels._surrogate_codes(1, True, True) == (_lib.RULE_STRAIGHT_THROUGH + 1, _lib.SG_AUTOGRAD + 1)
    assert kernels._surrogate_codes(2, False, True) == (_lib.RULE_SMOOTH + 2, _lib.SG_AUTOGRAD_SMOOTH + 2)
    assert kernels._surrogate_codes(4, True, False) == (_lib.RULE_SURROGATE, 4)


def test_params_match_reference_properties():
    p = myelin.LIFParams(tau_mem=10.0)
    assert p.decay == 1.0 - 1.0 / 10.0
    a = myelin.ALIFParams(tau_mem=20.0, tau_adaptation=50.0, beta=1.8)
    assert a.decay == 0.95 and a.adaptation_decay == 1.0 - 1.0 / 50.0
    with pytest.raises(ValueError, match="tau_mem must be positive"):
        myelin.LIFParams(tau_mem=0.0).decay


def test_surrogate_registry_round_trips():
    for name in surrogates.SURROGATE_NAMES:
        fn = surrogates.surrogate_from_name(name)
        assert surrogates.surrogate_name(fn) == name
        assert getattr(myelin, f"{name}_surrogate") is fn
    assert surrogates.SURROGATE_IDS["fast_sigmoid"] == 1
    with pytest.raises(ValueError, match="built-in surrogate functions"):
        surrogates.surrogate_name(lambda c: c)


def test_checkpoint_policy():
    assert checkpointing.recommended_checkpoint_size(100, policy="memory") == 10
    assert checkpointing.recommended_checkpoint_size(100, policy="balanced") == 25
    assert checkpointing.recommended_checkpoint_size(100, policy="speed") == 50
    assert checkpointing.resolve_checkpoint_size(2000, "memory") == 45
    assert checkpointing.resolve_checkpoint_size(10, 25) == 10
    assert checkpointing.parse_checkpoint_size("balanced") == "balanced"
    assert checkpointing.parse_checkpoint_size("12") == 12
    with pytest.raises(ValueError, match="positive integer"):
        checkpointing.parse_checkpoint_size("nope")
    with pytest.raises(ValueError, match="positive"):
        checkpointing.resolve_checkpoint_size(10, 0)


def test_packing_host_validation():
    with pytest.raises(ValueError, match="at least one dimension"):
        packing.pack_spikes(torch.tensor(1.0))
    with pytest.raises(ValueError, match="empty last dimension"):
        packing.pack_spikes(torch.empty(2, 0))
    bad = packing.PackedSpikes(data=torch.zeros((2, 2), dtype=torch.int32), original_shape=(2, 65))
    with pytest.raises(ValueError, match="shape"):
        packing.unpack_spikes(bad)
    empty = packing.PackedSpikes(data=torch.zeros((2, 0), dtype=torch.int32), original_shape=(2, 0))
    with pytest.raises(ValueError, match="non-empty last dimension"):
        packing.packed_spike_count(empty, dim=-1)
    p = packing.PackedSpikes(data=torch.zeros((3, 2, 2), dtype=torch.int32), original_shape=(3, 2, 35))
    with pytest.raises(ValueError, match="duplicate"):
        packing.packed_spike_count(p, dim=(0, -3))
    with pytest.raises(IndexError, match="out of range"):
        packing.packed_spike_count(p, dim=3)
    assert packing.packed_last_dim_size(33) == 2
    s = torch.zeros(100, 64, 2048)
    pk = packing.PackedSpikes(data=torch.zeros(100, 64, 64, dtype=torch.int32), original_shape=(100, 64, 2048))
    assert packing.spike_compression_ratio(s, pk) == 32.0


def test_every_backend_name_is_accepted():
    for b in ("auto", "torch", "hip", "triton", "triton_generated", "triton_compile"):
        kernels._check_backend(b)


def test_two_layer_entry_points_validate_like_the_reference():
    x, wh, wo = torch.zeros(4, 2, 3), torch.zeros(3, 5), torch.zeros(5, 2)
    p = myelin.LIFParams()
    with pytest.raises(ValueError, match="ROCm device"):
        myelin.two_layer_surrogate_lif_rate_recompute_forward(x, wh, None, wo, None, p)
    with pytest.raises(ValueError, match="requires CUDA tensors"):
        myelin.two_layer_surrogate_lif_rate_packed_hidden_forward(x, wh, None, wo, None, p)
    with pytest.raises(ValueError, match="only hard_forward=True"):
        myelin.two_layer_surrogate_lif_rate_recompute_forward(x, wh, None, wo, None, p, hard_forward=False)
    with pytest.raises(ValueError, match="only hard_forward=True"):
        myelin.two_layer_surrogate_lif_rate_packed_hidden_forward(x, wh, None, wo, None, p, hard_forward=False)
    with pytest.raises(ValueError, match="unknown surrogate"):
        myelin.two_layer_surrogate_lif_rate_recompute_forward(x, wh, None, wo, None, p, surrogate="relu")
