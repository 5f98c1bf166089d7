// common.hpp — shared plumbing of the fakhip C ABI: status codes, the current stream, the
// grow-only device workspace.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "fakhip.h"

namespace fhip {

// The stream every launch and async copy goes to (fhip_set_stream; nullptr = default stream).
hipStream_t stream();

// Record a failure message for fhip_last_error and return `code`.
int fail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
// Map a HIP error to 1000 + hipError_t with a message naming the failing call.
int hip_fail(hipError_t e, const char *what);
// Clear the per-thread error message at the start of an entry point.
void clear_error();

// Device scratch owned by the library, grown on demand. A grow allocates a new buffer and
// keeps the old one (queued kernels and captured graphs may still use it). Returns nullptr
// (and records the error) on failure.
void *workspace(size_t bytes);

// Device properties cached by fhip_init.
int cu_count();
// Largest dynamic LDS allocation one workgroup may request (bytes).
int lds_limit();

}  // namespace fhip

#define FHIP_CHECK(expr)                                    \
  do {                                                      \
    hipError_t fhip_e_ = (expr);                            \
    if (fhip_e_ != hipSuccess) return fhip::hip_fail(fhip_e_, #expr); \
  } while (0)

#define FHIP_CHECK_LAUNCH(what)                             \
  do {                                                      \
    hipError_t fhip_e_ = hipGetLastError();                 \
    if (fhip_e_ != hipSuccess) return fhip::hip_fail(fhip_e_, what); \
  } while (0)
