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

}  // namespace myelin
