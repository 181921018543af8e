"""djsaunde/myelin's import paths for the HIP spiking-neuron path.

Callers of the reference keep their imports unchanged::

    import myelin
    from myelin.kernels import surrogate_alif_forward
    from myelin.packing import pack_spikes, packed_spike_count
    from myelin.modules import LinearSurrogateLIF, LinearSurrogateLIFRate

and get the gfx950 kernels of ``myelin_amd``.  Each submodule below is the
``myelin_amd`` module of the same name (the same module object, so classes
and functions are identical whichever path imported them).  Only the hot
path's modules exist here (reference ``__init__.py:3-320`` also exports the
DSL, code generation, hardware export, online learning and the torch
reference functions, which this package does not provide).
"""

from __future__ import annotations

import importlib
import sys

import myelin_amd
from myelin_amd import *  # noqa: F401,F403
from myelin_amd import __all__  # noqa: F401

# reference module -> implementation (reference src/myelin/<name>.py)
SUBMODULES = ("checkpointing", "kernels", "modules", "neurons", "packing", "surrogates")

for _name in SUBMODULES:
    _mod = importlib.import_module(f"myelin_amd.{_name}")
    sys.modules[f"{__name__}.{_name}"] = _mod
    globals()[_name] = _mod

del _name, _mod
