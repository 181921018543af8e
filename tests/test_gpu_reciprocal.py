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
