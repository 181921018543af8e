"""ctypes binding of ``oracle/liboracle_c.so`` (the C restatement).

TEST INFRASTRUCTURE ONLY.  Arrays are numpy float32 / int32 / int64,
C-contiguous, time-major ``[T, BN]`` for the recurrences.
"""

from __future__ import annotations

import ctypes
import pathlib
import subprocess

import numpy as np

_HERE = pathlib.Path(__file__).resolve().parent
_LIB_PATH = _HERE / "liboracle_c.so"
_lib = None

_F = ctypes.c_float
_I64 = ctypes.c_int64
_P = ctypes.c_void_p

SURROGATE_IDS = {
    "sigmoid": 0,
    "fast_sigmoid": 1,
    "atan": 2,
    "triangular": 3,
    "superspike": 4,
    "multi_gaussian": 5,
}


def build() -> pathlib.Path:
    subprocess.run(["make", "-s", "-C", str(_HERE)], check=True)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            build()
        _lib = ctypes.CDLL(str(_LIB_PATH))
        _lib.orc_lif_fwd.argtypes = [_P, _P, _P, _P, _I64, _I64, _F, _F, _F, ctypes.c_int, _F]
        _lib.orc_alif_fwd.argtypes = [_P] * 6 + [_I64, _I64] + [_F] * 5 + [ctypes.c_int, _F]
        _lib.orc_lif_bwd.argtypes = [_P] * 6 + [_I64, _I64] + [_F] * 4 + [ctypes.c_int]
        _lib.orc_alif_bwd.argtypes = [_P] * 9 + [_I64, _I64] + [_F] * 6 + [ctypes.c_int]
        _lib.orc_pack_f32.argtypes = [_P, _P, _I64, _I64]
        _lib.orc_unpack_f32.argtypes = [_P, _P, _I64, _I64]
        _lib.orc_row_counts.argtypes = [_P, _P, _I64, _I64]
    return _lib


def _p(a: np.ndarray | None) -> int | None:
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32))


def lif_fwd(x, m0, decay, thr, reset, surrogate_mode=False, slope=10.0):
    x = _f32(x)
    T = x.shape[0]
    bn = x[0].size
    m0 = _f32(m0).reshape(-1)
    mT = np.empty(bn, np.float32)
    s = np.empty_like(x)
    lib().orc_lif_fwd(_p(x), _p(m0), _p(mT), _p(s), T, bn, decay, thr, reset,
                      int(surrogate_mode), slope)
    return mT.reshape(x.shape[1:]), s


def alif_fwd(x, m0, a0, decay, rho, thr, beta, reset, surrogate_mode=False, slope=10.0):
    x = _f32(x)
    T = x.shape[0]
    bn = x[0].size
    m0 = _f32(m0).reshape(-1)
    a0 = _f32(a0).reshape(-1)
    mT = np.empty(bn, np.float32)
    aT = np.empty(bn, np.float32)
    s = np.empty_like(x)
    lib().orc_alif_fwd(_p(x), _p(m0), _p(a0), _p(mT), _p(aT), _p(s), T, bn, decay, rho,
                       thr, beta, reset, int(surrogate_mode), slope)
    return mT.reshape(x.shape[1:]), aT.reshape(x.shape[1:]), s


def lif_bwd(x, m0, gs, gmT, decay, thr, reset, slope, surrogate):
    x = _f32(x)
    T = x.shape[0]
    bn = x[0].size
    m0 = _f32(m0).reshape(-1)
    gs = None if gs is None else _f32(gs)
    gmT = None if gmT is None else _f32(gmT).reshape(-1)
    gx = np.empty_like(x)
    gm0 = np.empty(bn, np.float32)
    lib().orc_lif_bwd(_p(x), _p(m0), _p(gs), _p(gmT), _p(gx), _p(gm0), T, bn, decay, thr,
                      reset, slope, SURROGATE_IDS[surrogate])
    return gx, gm0.reshape(x.shape[1:])


def alif_bwd(x, m0, a0, gs, gmT, gaT, decay, rho, thr, beta, reset, slope, surrogate):
    x = _f32(x)
    T = x.shape[0]
    bn = x[0].size
    m0 = _f32(m0).reshape(-1)
    a0 = _f32(a0).reshape(-1)
    gs = None if gs is None else _f32(gs)
    gmT = None if gmT is None else _f32(gmT).reshape(-1)
    gaT = None if gaT is None else _f32(gaT).reshape(-1)
    gx = np.empty_like(x)
    gm0 = np.empty(bn, np.float32)
    ga0 = np.empty(bn, np.float32)
    lib().orc_alif_bwd(_p(x), _p(m0), _p(a0), _p(gs), _p(gmT), _p(gaT), _p(gx), _p(gm0),
                       _p(ga0), T, bn, decay, rho, thr, beta, reset, slope,
                       SURROGATE_IDS[surrogate])
    return gx, gm0.reshape(x.shape[1:]), ga0.reshape(x.shape[1:])


def pack(spikes) -> np.ndarray:
    s = _f32(spikes)
    n = s.shape[-1]
    rows = s.size // n
    w = (n + 31) // 32
    out = np.empty((*s.shape[:-1], w), np.int32)
    lib().orc_pack_f32(_p(s), _p(out), rows, n)
    return out


def unpack(words, n: int) -> np.ndarray:
    words = np.ascontiguousarray(words, dtype=np.int32)
    rows = words.size // words.shape[-1]
    out = np.empty((*words.shape[:-1], n), np.float32)
    lib().orc_unpack_f32(_p(words), _p(out), rows, n)
    return out


def row_counts(words, n: int) -> np.ndarray:
    words = np.ascontiguousarray(words, dtype=np.int32)
    rows = words.size // words.shape[-1]
    out = np.empty(words.shape[:-1], np.int64)
    lib().orc_row_counts(_p(words), _p(out), rows, n)
    return out


def adjoint_exact(x, m0, a0, gs, gmT, gaT, decay, rho, thr, beta, reset, slope, surrogate, alif=True):
    """Exact (float64) gradient of the fp32 surrogate forward; returns
    float64 (grad_x, grad_m0, grad_a0)."""

    x = _f32(x)
    T = x.shape[0]
    bn = x[0].size
    m0 = _f32(m0).reshape(-1)
    a0 = None if a0 is None else _f32(a0).reshape(-1)
    gs = None if gs is None else _f32(gs)
    gmT = None if gmT is None else _f32(gmT).reshape(-1)
    gaT = None if gaT is None else _f32(gaT).reshape(-1)
    gx = np.empty(x.shape, np.float64)
    gm0 = np.empty(bn, np.float64)
    ga0 = np.empty(bn, np.float64)
    fn = lib().orc_adjoint_exact
    fn.argtypes = [_P] * 9 + [_I64, _I64] + [_F] * 6 + [ctypes.c_int, ctypes.c_int]
    fn(_p(x), _p(m0), _p(a0), _p(gs), _p(gmT), _p(gaT), _p(gx), _p(gm0), _p(ga0), T, bn, decay, rho, thr, beta,
       reset, slope, SURROGATE_IDS[surrogate], int(alif))
    return gx, gm0.reshape(x.shape[1:]), ga0.reshape(x.shape[1:])
