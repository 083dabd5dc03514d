// Host-side helpers shared by the C entry points: error reporting, workspace
// carving and the status-word clear kernel.
#pragma once

#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stddef.h>
#include <stdint.h>
#include <stdio.h>

#include "pararnn_amd.h"
#include "prnn_common.h"

namespace prnn {

// Thread-local message of the last failing call.
char* last_error_buffer();

inline int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(last_error_buffer(), 512, fmt, ap);
  va_end(ap);
  return code;
}

// f(TX{}) with TX the storage type of a checked dtype code.
template <typename F>
inline int with_storage(int dtype, F&& f) {
  if (dtype == PRNN_F32) return f(float{});
  if (dtype == PRNN_F16) return f(f16{});
  return f(bf16{});
}

// The dtype check every entry point runs.
inline int check_dtype(int dtype) {
  if (dtype != PRNN_F32 && dtype != PRNN_BF16 && dtype != PRNN_F16)
    return fail(PRNN_ERR_TYPE, "dtype code %d is not float32 (0), bfloat16 (1) or float16 (2)",
                dtype);
  return PRNN_OK;
}

inline int hip_fail(hipError_t e, const char* what) {
  return fail(PRNN_ERR_RUNTIME, "%s: %s", what, hipGetErrorString(e));
}

#define PRNN_HIP(call)                                   \
  do {                                                   \
    hipError_t e_ = (call);                              \
    if (e_ != hipSuccess) return prnn::hip_fail(e_, #call); \
  } while (0)

// Bump allocator over the caller's workspace; every block 256-byte aligned.
struct Carver {
  char* base;
  size_t used;
  explicit Carver(void* p) : base(static_cast<char*>(p)), used(0) {}
  void* take(size_t bytes) {
    used = (used + 255) & ~static_cast<size_t>(255);
    void* p = base ? base + used : nullptr;
    used += bytes;
    return p;
  }
};

// Process-wide deterministic look-back switch (prnn_set_deterministic).
int deterministic();

// Polling rounds a look-back or hand-off wait may spend before it gives up
// (prnn_set_spin_limit; default kSpinLimitDefault).
constexpr int kSpinLimitDefault = 1 << 22;
int spin_limit();

// Optional timing of an entry point's main kernel(s) (prnn_set_kernel_timing):
// when on, HIP events are recorded on the caller's stream right before and
// right after them; prnn_last_kernel_ms reads the last pair.
void timing_begin(hipStream_t stream);
void timing_end(hipStream_t stream);

// Zero `n` 32-bit words on `stream` with a kernel (no memset node, so the
// sequence stays replay-safe under HIP graph capture).
int clear_words(int* p, size_t n, hipStream_t stream);

}  // namespace prnn
