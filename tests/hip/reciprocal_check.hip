// Test-only kernels: the reciprocal and quotient helpers of
// myelin_amd/csrc/common.h against IEEE division on the GPU, for every fp32
// significand of the divisor.  One lane per significand, one result word
// per lane (bit flags), no atomics.  Built by tests/hip/build.py.
#include "../../myelin_amd/csrc/common.h"

namespace {

__global__ void reciprocal_check(uint32_t *out, uint32_t n, float scale) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float b = __uint_as_float(0x3f800000u | i) * scale;
  const float y = myelin::recip_rn(b);
  uint32_t f = (y != 1.0f / b) ? 1u : 0u;
  // quotients of hashed numerators (both signs, spread over exponents)
  uint32_t h = i * 2654435761u + 12345u;
  for (int j = 0; j < 16; ++j) {
    h = h * 1664525u + 1013904223u;
    const int ex = static_cast<int>(h % 120u) - 60;
    float x = __uint_as_float(0x3f800000u | (h >> 9)) * ldexpf(1.0f, ex);
    if (j & 1) x = -x;
    if (j == 0) x = 1.0f;
    if (j == 1) x = b;
    f |= (myelin::div_by(x, b, y) != x / b) ? (2u << j) : 0u;
  }
  out[i] = f;
}

// Divisors of 2^100 and beyond (scale 2^100, 2^127, +inf):
//   bit 0: recip_rn(b) differs from 1/b where 1/b is a normal number;
//   bit 1: recip_rn_or_zero(b) is not a number, or is more than 2^-126
//          from 1/b (it may flush a subnormal 1/b to 0);
//   bit 2: a quotient differs from x / b where x / b >= 2^-100;
//   bit 3: a closed-form derivative 0.5 * recip_rn_or_zero(d * d) is not a
//          number, or is more than 2^-126 from 0.5 / (d * d).
__global__ void reciprocal_check_large(uint32_t *out, uint32_t n, float scale) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float b = __uint_as_float(0x3f800000u | i) * scale;
  const float ieee = 1.0f / b;
  const float y = myelin::recip_rn(b);
  uint32_t f = 0u;
  if (ieee >= 0x1p-126f && y != ieee) f |= 1u;
  const float z = myelin::recip_rn_or_zero(b);
  if (z != z || fabsf(z - ieee) > 0x1p-126f) f |= 2u;
  if (ieee >= 0x1p-126f) {
    uint32_t h = i * 2654435761u + 777u;
    for (int j = 0; j < 8; ++j) {
      h = h * 1664525u + 1013904223u;
      float x = b * (__uint_as_float(0x3f800000u | (h >> 9)) * ldexpf(1.0f, -static_cast<int>(h % 90u)));
      if (j & 1) x = -x;
      if (myelin::div_by(x, b, y) != x / b) f |= 4u;
    }
  }
  const float d = 1.0f + b;  // 1 + |c| for c = b
  const float want = 0.5f / (d * d);
  const float got = 0.5f * myelin::recip_rn_or_zero(d * d);
  if (got != got || fabsf(got - want) > 0x1p-126f) f |= 8u;
  out[i] = f;
}

}  // namespace

extern "C" int myelin_test_reciprocal_check(uint32_t *out, uint32_t n, float scale, hipStream_t stream) {
  reciprocal_check<<<dim3((n + 255) / 256), dim3(256), 0, stream>>>(out, n, scale);
  return hipGetLastError() == hipSuccess ? 0 : 1;
}

extern "C" int myelin_test_reciprocal_check_large(uint32_t *out, uint32_t n, float scale, hipStream_t stream) {
  reciprocal_check_large<<<dim3((n + 255) / 256), dim3(256), 0, stream>>>(out, n, scale);
  return hipGetLastError() == hipSuccess ? 0 : 1;
}
