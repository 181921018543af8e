"""The reciprocal the fused kernels use for divisions by b >= 1
(myelin::recip_rn: the hardware reciprocal plus one Newton step) equals the
IEEE quotient 1.0f / b for every fp32 significand of b, at several
exponents; and quotients formed from it (myelin::div_by) equal IEEE x / b
for numerators from 2^-60 to 2^60 of both signs.  The autograd-order
kernels' bit-for-bit agreement with torch rests on this."""

from __future__ import annotations

import ctypes
import pathlib

import pytest
import torch

pytestmark = pytest.mark.gpu
LIB = pathlib.Path(__file__).resolve().parent / "hip" / "libtest_kernels.so"


@pytest.mark.parametrize("scale", [1.0, 8.0, 1024.0, 2.0 ** 40])
def test_reciprocal_and_quotients_equal_ieee_division(scale):
    print(f"case: reciprocal scale={scale:g}", flush=True)
    lib = ctypes.CDLL(str(LIB))
    fn = lib.myelin_test_reciprocal_check
    fn.argtypes = [ctypes.c_void_p, ctypes.c_uint32, ctypes.c_float, ctypes.c_void_p]
    n = 1 << 23
    out = torch.empty(n, dtype=torch.int32, device="cuda")
    assert fn(out.data_ptr(), n, scale, torch.cuda.current_stream().cuda_stream) == 0
    flags = out.cpu().to(torch.int64)
    bad_recip = int((flags & 1).sum())
    bad_quot = int((flags >> 1).ne(0).sum())
    assert bad_recip == 0, f"{bad_recip} divisors whose reciprocal differs from 1/b"
    assert bad_quot == 0, f"{bad_quot} divisors with a quotient different from x/b"


@pytest.mark.parametrize("scale", [2.0 ** 100, 2.0 ** 127, float("inf")])
def test_reciprocal_of_large_and_infinite_divisors(scale):
    """recip_rn stays the IEEE reciprocal wherever that is a normal number
    (divisors up to 2^126), and so do quotients above 2^-100;
    recip_rn_or_zero (the closed-form surrogate derivatives' reciprocal of
    a squared 1 + |c|) gives 0 for +inf, where the Newton step alone makes
    NaN, and never more than 2^-126 from 1/b; the derivative
    0.5 / (1 + |c|)^2 is 0 once the square overflows, as in torch."""

    print(f"case: reciprocal large scale={scale:g}", flush=True)
    lib = ctypes.CDLL(str(LIB))
    fn = lib.myelin_test_reciprocal_check_large
    fn.argtypes = [ctypes.c_void_p, ctypes.c_uint32, ctypes.c_float, ctypes.c_void_p]
    n = 1 << 23
    out = torch.empty(n, dtype=torch.int32, device="cuda")
    assert fn(out.data_ptr(), n, scale, torch.cuda.current_stream().cuda_stream) == 0
    flags = out.cpu().to(torch.int64)
    names = ("recip_rn vs 1/b", "recip_rn_or_zero", "quotient", "closed-form derivative")
    for bit, what in enumerate(names):
        bad = int(((flags >> bit) & 1).sum())
        assert bad == 0, f"{bad} divisors fail: {what}"
