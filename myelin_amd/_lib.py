"""ctypes binding of ``libmyelin_hip.so`` (declared in ``include/myelin_hip.h``).

There is no fallback: if the library is missing or a tensor is not on a
ROCm device, the calls raise.  ``torch`` is imported before the library is
loaded so that the HIP runtime torch already holds (same soname) is the one
the kernels launch through.
"""

from __future__ import annotations

import ctypes
import os
import pathlib
import threading

import torch

LIB_PATH = pathlib.Path(os.environ.get("MYELIN_HIP_LIB", pathlib.Path(__file__).with_name("libmyelin_hip.so")))

OK, EINVAL, EHIP = 0, 1, 2
RULE_THRESHOLD, RULE_SURROGATE = 0, 1
# + surrogate id: spike values of hard_surrogate_spike / the smooth primitive,
# evaluated op by op as torch does
RULE_STRAIGHT_THROUGH, RULE_SMOOTH = 16, 32
SG_NONE = 6
# + surrogate id: the backward in torch autograd's operation order, after a
# forward run with RULE_STRAIGHT_THROUGH / RULE_SMOOTH + the same id
SG_AUTOGRAD, SG_AUTOGRAD_SMOOTH = 16, 32
PREC = {"fp32": 0, "bf16": 1}
DT_BITS = 7  # packed spike bits (int32 words) as a GEMM operand
DT_BF16X3 = 8  # three bf16 planes summing exactly to an fp32 tensor
DT = {
    torch.float32: 0,
    torch.float16: 1,
    torch.bfloat16: 2,
    torch.bool: 3,
    torch.uint8: 3,
    torch.int8: 3,
    torch.int32: 4,
    torch.int64: 5,
    torch.float64: 6,
}

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_F = ctypes.c_float
_INT = ctypes.c_int

# name -> argtypes, in the order of include/myelin_hip.h
SIGNATURES: dict[str, list] = {
    "myelin_lif_fwd_f32": [_P] * 6 + [_I64] * 3 + [_F] * 4 + [_INT, _I64, _P],
    "myelin_alif_fwd_f32": [_P] * 9 + [_I64] * 3 + [_F] * 6 + [_INT, _I64, _P],
    "myelin_lif_bwd_f32": [_P] * 6 + [_I64] * 2 + [_F] * 4 + [_INT, _I64, _P],
    "myelin_alif_bwd_f32": [_P] * 9 + [_I64] * 2 + [_F] * 6 + [_INT, _I64, _P],
    "myelin_pack": [_P, _INT, _P, _I64, _I64, _P],
    "myelin_unpack": [_P, _P, _INT, _I64, _I64, _P],
    "myelin_packed_counts": [_P, _INT, _P, ctypes.c_uint32, _I64, _P, _P],
    "myelin_packed_counts_keep_last": [_P, _I64, _I64, _I64, _P, _P],
    "myelin_counts_to_rate": [_P, _P, _INT, _I64, _I64, _P],
    "myelin_gemm_f32": [_P, _P, _P, _P] + [_I64] * 6 + [_INT] * 4 + [_P, _I64, _P],
    "myelin_gemm": [_P, _INT, _P, _INT, _P, _P] + [_I64] * 6 + [_INT] * 4 + [_P, _I64, _P],
    "myelin_gemm_col_sum": [_P, _INT, _P, _INT, _P, _P] + [_I64] * 6 + [_INT] * 4 + [_P, _I64, _P, _P, _I64, _I64,
                                                                                     _P],
    "myelin_linear_lif_fwd": [_P] * 10 + [_I64] * 7 + [_F] * 4 + [_INT, _INT, _P],
    "myelin_linear_lif_fwd_bf16": [_P] * 10 + [_I64] * 7 + [_F] * 4 + [_INT, _P],
    "myelin_cast_bf16": [_P, _P, _I64, _P],
    "myelin_cast_bf16_checked": [_P, _P, _I64, _P, _P],
    "myelin_split_bf16x3": [_P, _P, _I64, _I64, _INT, _P],
    "myelin_gemm_parts": [_P, _P, _INT, _I64, _P, _P] + [_I64] * 6 + [_INT] * 3 + [_P, _I64, _P],
    "myelin_gemm_parts_col_sum": [_P, _P, _INT, _I64, _P, _P] + [_I64] * 6 + [_INT] * 3 + [_P, _I64, _P, _P, _I64,
                                                                                          _I64, _P],
    "myelin_gemm_noalloc": [_P, _INT, _P, _INT, _P, _P] + [_I64] * 6 + [_INT] * 4 + [_P],
    "myelin_transpose_bf16": [_P, _P, _I64, _I64, _P],
    "myelin_cast_transpose_bf16": [_P, _P, _I64, _P, _P, _I64, _I64, _P],
    "myelin_linear_pre_bwd": [_P] * 5 + [_INT, _P] + [_I64] * 3 + [_F] * 4 + [_INT, _INT, _P],
    "myelin_linear_pre_bwd_readout": [_P] * 3 + [_INT] + [_P] * 2 + [_INT, _P] + [_I64] * 3 + [_F] * 4
    + [_INT, _INT, _P],
    "myelin_col_sum_f32": [_P, _P, _I64, _I64, _INT, _P],
    "myelin_lif_currents_fwd": [_P] * 9 + [_I64] * 8 + [_F] * 4 + [_INT, _P],
    "myelin_linear_lif_fwd_narrow_bits": [_P] * 8 + [_I64] * 6 + [_F] * 4 + [_INT, _INT, _P],
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


class MyelinHipError(RuntimeError):
    """A HIP launch inside libmyelin_hip.so failed."""


def load() -> ctypes.CDLL:
    """Load the library once; raise ImportError with build instructions if absent."""

    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise ImportError(
                    f"{LIB_PATH} is not built; run `python -m myelin_amd.build` "
                    "(hipcc --offload-arch=gfx950). myelin_amd has no CPU fallback."
                )
            lib = ctypes.CDLL(str(LIB_PATH))
            lib.myelin_last_error.restype = ctypes.c_char_p
            lib.myelin_abi_version.restype = ctypes.c_int
            lib.myelin_gemm_workspace_elems.argtypes = [_I64, _I64, _I64, _INT]
            lib.myelin_gemm_workspace_elems.restype = ctypes.c_int64
            lib.myelin_narrow_bits_fits.argtypes = [_I64, _I64, _INT]
            lib.myelin_narrow_bits_fits.restype = ctypes.c_int
            for name, argtypes in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.argtypes = argtypes
                fn.restype = ctypes.c_int
            if lib.myelin_abi_version() != 1:
                raise ImportError("libmyelin_hip.so ABI version mismatch; rebuild it")
            _lib = lib
    return _lib


_FNS: dict = {}


def call(name: str, *args) -> None:
    """Call an entry point; map its return code to ValueError / MyelinHipError."""

    fn = _FNS.get(name)
    if fn is None:
        fn = _FNS[name] = getattr(load(), name)
    rc = fn(*args)
    if rc == OK:
        return
    msg = (load().myelin_last_error() or b"").decode(errors="replace")
    if rc == EINVAL:
        raise ValueError(f"{name}: {msg}")
    raise MyelinHipError(f"{name}: {msg}")


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream(device: torch.device) -> int:
    """The raw handle of the current stream of ``device`` (the stream torch
    launches on, also under graph capture)."""

    idx = device.index
    return torch._C._cuda_getCurrentRawStream(torch.cuda.current_device() if idx is None else idx)


def require_device(t: torch.Tensor, what: str) -> None:
    if not t.is_cuda:
        raise ValueError(
            f"{what} must be a ROCm device tensor (got device {t.device}); myelin_amd runs only "
            "the HIP path"
        )
