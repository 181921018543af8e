"""MI355X-native fused-time spiking-neuron path with myelin's public API.

``import myelin_amd as myelin`` gives the names callers of djsaunde/myelin
use on this path (kernels, packing, neuron types, surrogates, checkpoint
policy, and the streamed-synapse / rate modules); every compute call runs a
hand-written gfx950 HIP kernel from ``libmyelin_hip.so``.
"""

from myelin_amd.checkpointing import (
    CheckpointPolicy,
    CheckpointSize,
    parse_checkpoint_size,
    recommended_checkpoint_size,
    resolve_checkpoint_size,
)
from myelin_amd.kernels import (
    Backend,
    alif_forward,
    fused_lif_unroll,
    lif_forward,
    lif_forward_packed_spikes,
    surrogate_alif_forward,
    surrogate_lif_forward,
)
from myelin_amd.neurons import ALIFParams, ALIFState, LIFParams, LIFState
from myelin_amd.packing import (
    BITS_PER_WORD,
    PackedSpikes,
    dense_spike_bytes,
    pack_spikes,
    packed_last_dim_size,
    packed_spike_bytes,
    packed_spike_count,
    packed_spike_counts,
    packed_spike_rate,
    spike_compression_ratio,
    unpack_spikes,
)
from myelin_amd.surrogates import (
    SURROGATE_NAMES,
    SurrogateFn,
    SurrogateName,
    atan_surrogate,
    fast_sigmoid_surrogate,
    multi_gaussian_surrogate,
    sigmoid_surrogate,
    superspike_surrogate,
    surrogate_from_name,
    surrogate_name,
    triangular_surrogate,
)

__all__ = [
    "ALIFParams",
    "ALIFState",
    "BITS_PER_WORD",
    "Backend",
    "CheckpointPolicy",
    "CheckpointSize",
    "LIFParams",
    "LIFState",
    "PackedSpikes",
    "SURROGATE_NAMES",
    "SurrogateFn",
    "SurrogateName",
    "alif_forward",
    "atan_surrogate",
    "dense_spike_bytes",
    "fast_sigmoid_surrogate",
    "fused_lif_unroll",
    "lif_forward",
    "lif_forward_packed_spikes",
    "multi_gaussian_surrogate",
    "pack_spikes",
    "packed_last_dim_size",
    "packed_spike_bytes",
    "packed_spike_count",
    "packed_spike_counts",
    "packed_spike_rate",
    "parse_checkpoint_size",
    "recommended_checkpoint_size",
    "resolve_checkpoint_size",
    "sigmoid_surrogate",
    "spike_compression_ratio",
    "superspike_surrogate",
    "surrogate_alif_forward",
    "surrogate_from_name",
    "surrogate_lif_forward",
    "surrogate_name",
    "triangular_surrogate",
    "unpack_spikes",
]
