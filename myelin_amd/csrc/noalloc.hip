// myelin_gemm_noalloc: myelin_gemm for callers that cannot allocate device
// memory (code under HIP graph capture, tight serving loops, harnesses that
// forbid hipMalloc).  The K split's partial tiles go to `scratch`, a static
// device array of MYELIN_NOALLOC_SCRATCH_ELEMS floats that every GPU the
// library runs on holds until the process ends, instead of a caller
// workspace.  The kernels are myelin_gemm's: the array's device address is
// passed to them as the workspace pointer.
//
// In host code `scratch` names a host-side stand-in, not device memory, so
// its device address is looked up once per device (with that device
// current) by hipGetSymbolAddress and kept per device; only that address is
// ever handed to a kernel.
//
// Every split writes its whole [M, N] plane before the reduce reads it, so
// nothing in the array needs clearing between calls.  All calls on one GPU
// share its array: calls that overlap in time on one GPU (two streams, two
// host threads) race on it.

#include <mutex>

#include "common.h"

namespace {

__device__ __align__(256) float scratch[MYELIN_NOALLOC_SCRATCH_ELEMS];

constexpr int kMaxDevices = 64;
std::mutex g_mu;
float *g_scratch[kMaxDevices] = {};

// This device's address of `scratch`: the device of `stream` (the current
// device for the null stream), looked up on its first call.
int device_scratch(myelin_stream_t stream, float **out) {
  int dev = -1;
  hipError_t e = stream != nullptr ? hipStreamGetDevice(myelin::as_hip(stream), &dev) : hipGetDevice(&dev);
  if (e != hipSuccess) {
    myelin::set_error("gemm_noalloc: cannot find the stream's device: %s", hipGetErrorString(e));
    return MYELIN_EHIP;
  }
  if (dev < 0 || dev >= kMaxDevices) return myelin::invalid("gemm_noalloc: device %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_mu);
  if (g_scratch[dev] == nullptr) {
    int cur = -1;
    if ((e = hipGetDevice(&cur)) == hipSuccess && cur != dev) e = hipSetDevice(dev);
    void *p = nullptr;
    if (e == hipSuccess) e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (cur >= 0 && cur != dev) {
      const hipError_t back = hipSetDevice(cur);
      if (e == hipSuccess) e = back;
    }
    if (e != hipSuccess || p == nullptr) {
      myelin::set_error("gemm_noalloc: hipGetSymbolAddress(scratch) on device %d: %s", dev,
                        hipGetErrorString(e != hipSuccess ? e : hipErrorInvalidSymbol));
      return MYELIN_EHIP;
    }
    g_scratch[dev] = static_cast<float *>(p);
  }
  *out = g_scratch[dev];
  return MYELIN_OK;
}

}  // namespace

extern "C" int myelin_gemm_noalloc(const void *A, int a_dtype, const void *B, int b_dtype, const float *bias,
                                   float *C, int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb, int64_t ldc,
                                   int trans_a, int trans_b, int accumulate, int precision, myelin_stream_t stream) {
  if (M < 0 || N < 0 || K < 0) return myelin::invalid("gemm_noalloc: negative size");
  const int64_t need = myelin_gemm_workspace_elems(M, N, K, precision);
  if (need > MYELIN_NOALLOC_SCRATCH_ELEMS)
    return myelin::invalid(
        "gemm_noalloc: the K split of a %lld x %lld x %lld product needs %lld floats of scratch, more than the %lld "
        "this entry point holds; call myelin_gemm with a workspace instead",
        (long long)M, (long long)N, (long long)K, (long long)need, (long long)MYELIN_NOALLOC_SCRATCH_ELEMS);
  float *ws = nullptr;
  if (need > 0) {
    if (int rc = device_scratch(stream, &ws)) return rc;
  }
  return myelin_gemm(A, a_dtype, B, b_dtype, bias, C, M, N, K, lda, ldb, ldc, trans_a, trans_b, accumulate,
                     precision, ws, need, stream);
}
