// Shared helpers for the gfx950 kernels behind include/myelin_hip.h.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/myelin_hip.h"

namespace myelin {

// Record a message for myelin_last_error() on the calling thread.
void set_error(const char *fmt, ...) __attribute__((format(printf, 1, 2)));

// Report a rejected argument: returns MYELIN_EINVAL.
int invalid(const char *fmt, ...) __attribute__((format(printf, 1, 2)));

// Check hipGetLastError() after a launch: MYELIN_OK or MYELIN_EHIP.
int launched(const char *what);

inline hipStream_t as_hip(myelin_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

inline bool aligned(const void *p, int bytes) {
  return (reinterpret_cast<uintptr_t>(p) % static_cast<uintptr_t>(bytes)) == 0;
}

constexpr int kWave = 64;

// 1/b rounded to nearest, for b >= 1: the hardware reciprocal refined by
// one Newton step (e = 1 - b*r exact in an fma, r + r*e rounded once).  On
// gfx950 this equals the IEEE quotient 1.0f / b for every fp32 significand
// of b (tests/test_gpu_reciprocal.py checks all of them), in 3 instructions
// instead of the 10 of the general division sequence.
__device__ __forceinline__ float recip_rn(float b) {
  const float r = __builtin_amdgcn_rcpf(b);
  return __builtin_fmaf(__builtin_fmaf(-b, r, 1.0f), r, r);
}

// recip_rn for a divisor that may overflow to +inf (a squared 1 + |c|):
// there the Newton step would form inf * 0 = NaN, and IEEE division gives
// 0.  Finite divisors past 2^126 have a subnormal reciprocal, returned as 0
// or that subnormal (never NaN).
__device__ __forceinline__ float recip_rn_or_zero(float b) {
  const float y = recip_rn(b);
  return b < __builtin_huge_valf() ? y : 0.0f;
}

// x / b from y = recip_rn(b): q0 = x*y, e = x - b*q0 (exact in an fma),
// q = q0 + e*y rounded once.  With y within half an ulp of 1/b and q0
// within one ulp of x/b this is x/b rounded to nearest (Markstein's
// theorem), i.e. the IEEE quotient, while the residual stays normal: |x| >=
// 2^-100 and x/b normal.  x = 0 gives a zero of possibly the other sign.
// (Checked against IEEE division on the host for every fp32 significand of
// b with numerators in that range, and on the GPU.)
__device__ __forceinline__ float div_by(float x, float b, float y) {
  const float q0 = x * y;
  const float e = __builtin_fmaf(-b, q0, x);
  return __builtin_fmaf(e, y, q0);
}

}  // namespace myelin
