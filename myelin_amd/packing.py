"""Bitpacked spike tensors on the GPU (drop-in for ``myelin.packing``,
packing.py:1-273).

``PackedSpikes.data`` holds signed int32 words along the last dimension:
bit ``i`` of word ``w`` is element ``32*w + i`` (LSB first); padding bits
are zero after packing and ignored by every count.  All compute runs in the
HIP kernels of ``csrc/packing.hip``: a wave ballot packs 64 elements into two
words, unpack writes 4 elements per lane, counts use popcount.
"""

from __future__ import annotations

import contextlib
import ctypes

from collections.abc import Sequence
from dataclasses import dataclass
from typing import Union

import torch

from myelin_amd import _lib

BITS_PER_WORD = 32
CountDim = Union[int, Sequence[int], None]


@dataclass(frozen=True)
class PackedSpikes:
    """Spike tensor packed into signed int32 words along the last dimension (packing.py:19-34)."""

    data: torch.Tensor
    original_shape: tuple[int, ...]

    @property
    def packed_shape(self) -> tuple[int, ...]:
        return tuple(self.data.shape)

    @property
    def original_numel(self) -> int:
        numel = 1
        for size in self.original_shape:
            numel *= size
        return numel


def _device_of(t: torch.Tensor):
    """The tensor's device as the current device for a launch (no switch
    when it already is)."""

    if t.device.index == torch.cuda.current_device():
        return contextlib.nullcontext()
    return torch.cuda.device(t.device)


def packed_last_dim_size(size: int) -> int:
    """Words needed for a last dimension of ``size`` (packing.py:36-42)."""

    if size < 0:
        raise ValueError("size must be non-negative")
    return (size + BITS_PER_WORD - 1) // BITS_PER_WORD


def _dtype_code(dtype: torch.dtype) -> int:
    try:
        return _lib.DT[dtype]
    except KeyError:
        raise ValueError(f"unsupported spike dtype {dtype}") from None


def pack_spikes(spikes: torch.Tensor) -> PackedSpikes:
    """Pack nonzero elements into int32 words along the last dim (packing.py:45-71)."""

    if spikes.ndim == 0:
        raise ValueError("spikes must have at least one dimension")
    if spikes.shape[-1] == 0:
        raise ValueError("cannot pack an empty last dimension")
    _lib.require_device(spikes, "spikes")
    code = _dtype_code(spikes.dtype)
    src = spikes.contiguous()
    n = src.shape[-1]
    rows = src.numel() // n
    words = torch.empty((*src.shape[:-1], packed_last_dim_size(n)), dtype=torch.int32, device=src.device)
    with _device_of(src):
        _lib.call("myelin_pack", _lib.ptr(src), code, _lib.ptr(words), rows, n, _lib.stream(src.device))
    return PackedSpikes(data=words, original_shape=tuple(spikes.shape))


def unpack_spikes(packed: PackedSpikes, *, dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """Unpack to 0/1 values of ``dtype`` in the original shape (packing.py:74-81)."""

    _validate_packed_spikes(packed)
    _lib.require_device(packed.data, "packed.data")
    code = _dtype_code(dtype)
    words = packed.data.contiguous()
    shape = packed.original_shape
    n = shape[-1]
    out = torch.empty(shape, dtype=dtype, device=words.device)
    rows = out.numel() // n
    with _device_of(words):
        _lib.call("myelin_unpack", _lib.ptr(words), _lib.ptr(out), code, rows, n, _lib.stream(words.device))
    return out


def packed_spike_count(packed: PackedSpikes, dim: CountDim = None) -> torch.Tensor:
    """Spike counts with dense-like reduction semantics (packing.py:84-107).

    Reductions that include the last dim run from the packed words; ones that
    keep it count bits per neuron without unpacking.  Counts are exact
    int64 (the reference's dense fallback sums in float32, which agrees while
    every count is below 2**24).
    """

    if dim is None:
        return packed_spike_counts(packed, dim=None)
    nd = len(packed.original_shape)
    dims = _normalize_count_dims(dim, ndim=nd)
    if nd - 1 in dims:
        return packed_spike_counts(packed, dim=dims)
    return _counts_keep_last(packed, dims)


def packed_spike_counts(packed: PackedSpikes, dim: CountDim = -1) -> torch.Tensor:
    """Counts over dims that include the packed last dim (packing.py:110-142).

    For ``[T, B, N]`` spikes: ``dim=-1`` -> ``[T, B]``, ``dim=(0, -1)`` ->
    ``[B]``, ``dim=None`` -> scalar.
    """

    _validate_packed_spikes(packed)
    _lib.require_device(packed.data, "packed.data")
    shape = packed.original_shape
    nd = len(shape)
    if dim is None:
        dims = tuple(range(nd))
    else:
        dims = _normalize_count_dims(dim, ndim=nd)
        if nd - 1 not in dims:
            raise ValueError(
                "packed_spike_counts requires reducing the packed/original last dimension; "
                "use packed_spike_count for dense-like reductions that keep that dimension"
            )
    lead = shape[:-1]
    mask = 0
    for d in dims:
        if d != nd - 1:
            mask |= 1 << d
    kept = tuple(s for i, s in enumerate(lead) if not (mask >> i) & 1)
    out = torch.empty(kept, dtype=torch.int64, device=packed.data.device)
    words = packed.data.contiguous()
    lead_arr = (ctypes.c_int64 * max(1, len(lead)))(*lead)
    if len(lead) > 8:
        raise ValueError("at most 8 leading dimensions are supported")
    with _device_of(words):
        _lib.call(
            "myelin_packed_counts", _lib.ptr(words), len(lead), ctypes.addressof(lead_arr), mask, shape[-1],
            _lib.ptr(out), _lib.stream(words.device),
        )
    return out


def _counts_keep_last(packed: PackedSpikes, dims: tuple[int, ...]) -> torch.Tensor:
    """Per-neuron counts over leading dims ``dims`` (last dim kept)."""

    _validate_packed_spikes(packed)
    _lib.require_device(packed.data, "packed.data")
    shape = packed.original_shape
    nd = len(shape)
    n = shape[-1]
    lead = list(range(nd - 1))
    red = sorted(dims)
    keep = [d for d in lead if d not in red]
    words = packed.data
    if red != lead[: len(red)]:
        # bring the reduced dims to the front (a layout copy of the packed words)
        words = words.permute(*red, *keep, nd - 1)
    words = words.contiguous()
    R = 1
    for d in red:
        R *= shape[d]
    K = 1
    for d in keep:
        K *= shape[d]
    out = torch.empty((*[shape[d] for d in keep], n), dtype=torch.int64, device=words.device)
    with _device_of(words):
        _lib.call(
            "myelin_packed_counts_keep_last", _lib.ptr(words), R, K, n, _lib.ptr(out),
            _lib.stream(words.device),
        )
    return out


def packed_spike_rate(
    packed: PackedSpikes, dim: CountDim = None, *, dtype: torch.dtype = torch.float32
) -> torch.Tensor:
    """``count(dim).to(dtype) / prod(reduced sizes)`` (packing.py:145-162)."""

    counts = packed_spike_count(packed, dim=dim)
    nd = len(packed.original_shape)
    dims = tuple(range(nd)) if dim is None else _normalize_count_dims(dim, ndim=nd)
    denominator = 1
    for index in dims:
        denominator *= packed.original_shape[index]
    if dtype not in (torch.float32, torch.float64):
        raise ValueError("packed_spike_rate supports dtype float32 or float64 on the HIP path")
    out = torch.empty(counts.shape, dtype=dtype, device=counts.device)
    with _device_of(counts):
        _lib.call(
            "myelin_counts_to_rate", _lib.ptr(counts), _lib.ptr(out), _lib.DT[dtype], counts.numel(),
            denominator, _lib.stream(counts.device),
        )
    return out


def _normalize_count_dims(dim: int | Sequence[int], *, ndim: int) -> tuple[int, ...]:
    """Normalize, range-check and de-duplicate dims (packing.py:223-233)."""

    raw = (dim,) if isinstance(dim, int) else tuple(dim)
    out: list[int] = []
    for d in raw:
        actual = d + ndim if d < 0 else d
        if actual < 0 or actual >= ndim:
            raise IndexError(f"dimension out of range: {d}")
        if actual in out:
            raise ValueError(f"duplicate reduction dimension: {d}")
        out.append(actual)
    return tuple(out)


def _validate_packed_spikes(packed: PackedSpikes) -> None:
    """Shape/dtype contract of a PackedSpikes (packing.py:236-252)."""

    if packed.data.dtype != torch.int32:
        raise ValueError("packed.data must have dtype torch.int32")
    if len(packed.original_shape) == 0:
        raise ValueError("packed.original_shape must have at least one dimension")
    if packed.original_shape[-1] <= 0:
        raise ValueError("packed.original_shape must have non-empty last dimension")
    expected = (*packed.original_shape[:-1], packed_last_dim_size(packed.original_shape[-1]))
    if tuple(packed.data.shape) != expected:
        raise ValueError(
            "packed.data shape does not match packed.original_shape; "
            f"got {tuple(packed.data.shape)} and expected {expected}"
        )


def dense_spike_bytes(spikes: torch.Tensor) -> int:
    """Storage bytes of a dense spike tensor (packing.py:255-258)."""

    return spikes.numel() * spikes.element_size()


def packed_spike_bytes(packed: PackedSpikes) -> int:
    """Storage bytes of the packed words (packing.py:261-264)."""

    return packed.data.numel() * packed.data.element_size()


def spike_compression_ratio(spikes: torch.Tensor, packed: PackedSpikes) -> float:
    """Dense bytes / packed bytes (packing.py:267-273)."""

    packed_bytes = packed_spike_bytes(packed)
    if packed_bytes == 0:
        raise ValueError("packed representation has zero bytes")
    return dense_spike_bytes(spikes) / packed_bytes
