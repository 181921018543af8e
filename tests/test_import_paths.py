"""The reference's import paths (`import myelin`, `from myelin.kernels import
...`) resolve to the HIP implementation (reference src/myelin/__init__.py:3-320,
kernels.py:52-846, packing.py:45-162, modules.py:706-943).  Host-only."""

from __future__ import annotations

import importlib

import pytest
import torch

import myelin_amd

KERNELS = ("lif_forward", "alif_forward", "surrogate_lif_forward", "surrogate_alif_forward",
           "lif_forward_packed_spikes", "linear_surrogate_lif_forward", "linear_surrogate_lif_rate_forward",
           "linear_surrogate_lif_packed_forward", "two_layer_surrogate_lif_rate_recompute_forward",
           "two_layer_surrogate_lif_rate_packed_hidden_forward", "fused_lif_unroll")
PACKING = ("PackedSpikes", "pack_spikes", "unpack_spikes", "packed_spike_count", "packed_spike_counts",
           "packed_spike_rate", "packed_last_dim_size", "packed_spike_bytes", "dense_spike_bytes",
           "spike_compression_ratio")
MODULES = ("LinearSynapse", "LIFCell", "ALIFCell", "SurrogateLIFCell", "SurrogateALIFCell", "TimeUnroll",
           "LinearSurrogateLIF", "LinearSurrogateLIFRate", "LinearSurrogateLIFPacked", "RateReadoutClassifier")


@pytest.mark.parametrize("module,names", [("kernels", KERNELS), ("packing", PACKING), ("modules", MODULES),
                                          ("neurons", ("LIFParams", "LIFState", "ALIFParams", "ALIFState")),
                                          ("surrogates", ("SURROGATE_NAMES", "surrogate_from_name",
                                                          "fast_sigmoid_surrogate", "atan_surrogate")),
                                          ("checkpointing", ("recommended_checkpoint_size",
                                                             "resolve_checkpoint_size"))])
def test_reference_submodule_paths_resolve_to_the_hip_modules(module, names):
    mod = importlib.import_module(f"myelin.{module}")
    assert mod is importlib.import_module(f"myelin_amd.{module}")
    for name in names:
        assert getattr(mod, name) is getattr(myelin_amd, name), f"myelin.{module}.{name}"


def test_top_level_names():
    import myelin

    for name in myelin_amd.__all__:
        assert getattr(myelin, name) is getattr(myelin_amd, name), name
    from myelin import LinearSurrogateLIF, surrogate_alif_forward  # noqa: F401


def test_no_cpu_fallback_through_the_reference_path():
    from myelin.kernels import surrogate_alif_forward
    from myelin.neurons import ALIFParams, ALIFState

    x = torch.zeros(4, 2, 3)
    z = torch.zeros(2, 3)
    with pytest.raises(ValueError, match="ROCm device tensor"):
        surrogate_alif_forward(x, ALIFState(z, z), ALIFParams())
