// common.hpp — shared plumbing of the fakhip C ABI: status codes, the current stream, device
// scratch, the tuning knobs and the registry of tiled weights.
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

// Device scratch for the launches of one call, `bytes` long. Normally the current stream's
// workspace: one grow-only buffer per stream, so work queued on different streams never shares
// scratch (a grow allocates a new buffer and keeps the old one: queued kernels and captured
// graphs may still use it). Inside a ScratchScope it is the scope's region instead, and nothing
// is allocated; a request larger than that region fails. Returns nullptr (and records the
// error) on failure.
void *workspace(size_t bytes);

// Routes workspace() to [base, base + cap) until destroyed (scopes nest).
class ScratchScope {
 public:
  ScratchScope(void *base, size_t cap);
  ~ScratchScope();
  ScratchScope(const ScratchScope &) = delete;
  ScratchScope &operator=(const ScratchScope &) = delete;

 private:
  void *prev_base_;
  size_t prev_cap_;
  bool prev_on_;
};

// Resolves the device address of the no-allocation entry's static scratch on the current
// device (noalloc.hip); called by fhip_init.
int noalloc_setup();

// Events set by fhip_time_next_launch, handed to (and cleared by) the next launch that takes
// them (the one-token GEMV); both null when none are pending.
void take_launch_events(hipEvent_t *start, hipEvent_t *stop);

// Device properties cached by fhip_init.
int cu_count();
// Largest dynamic LDS allocation one workgroup may request (bytes).
int lds_limit();

// Launch-shape overrides, read once from the environment by fhip_init (0 = the built-in rule).
// None of them changes a result except gemm32_sk, which reorders the GEMM's K-range sums.
struct Tuning {
  int gemv_tw, gemv_kw;   // FAK_HIP_GEMV_TW / _KW: 1..4-token GEMV workgroup shape
  int gemv_globalx;       // FAK_HIP_GEMV_GLOBALX: activation operands in global memory
  int gemv16_from;        // FAK_HIP_GEMV16_FROM: first width on the 5..16-token kernel (1..5)
  int gemm32_form;        // FAK_HIP_GEMM32_FORM: 1 = four-wave 2x2 (else the staged kernel)
  int gemm32_nt;          // FAK_HIP_GEMM32_NT: 32-row tiles per wave of the staged kernel
  int gemm32_sk;          // FAK_HIP_GEMM32_SK: K ranges of the prefill GEMM
  int gemm32_nwb;         // FAK_HIP_GEMM32_NWB: weight buffers of the 2x2 form (1 or 2)
  int i8r_kw;             // FAK_HIP_I8R_KW: waves per tile of the int8 route
  int i8r_tw;             // FAK_HIP_I8R_TW: tiles per workgroup of the int8 route (one wave each)
  int q8_tw, q8_kw;       // FAK_HIP_Q8_TW / _KW: Q8_0 GEMV workgroup shape
};
const Tuning &tuning();

// Registry of tiled weights: every repack records the buffer's format and shape, and the matmul
// entries refuse a pointer that does not start a tiled weight of the format and shape asked for
// (a raw GGUF upload or a stale pointer would otherwise produce plausible garbage). Any other
// write through the ABI into a recorded range (copies, memsets, the outputs of unpack, dequant,
// quantize, matmul and MLP calls, frees) drops the record; a device-to-device copy of a whole
// recorded weight records the copy.
enum WeightKind { kWeightQ4K = 1, kWeightQ8_0 = 2, kWeightQ6K = 3 };
void tag_weight(const void *p, size_t bytes, int kind, int out, int in);
void untag_range(const void *p, size_t bytes);
int check_weight(const char *who, const void *p, int kind, int out, int in);

// FHIP_EINVAL unless [a, a + na) and [b, b + nb) are disjoint (an input that lives in the
// scratch a launch is about to overwrite).
int check_disjoint(const char *who, const void *a, size_t na, const void *b, size_t nb);

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
