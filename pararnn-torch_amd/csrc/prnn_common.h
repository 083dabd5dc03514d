// Shared device helpers for the pararnn_amd HIP kernels (gfx950 / CDNA4).
//
// * bf16 storage as raw 16-bit words with round-to-nearest-even conversion;
// * transcendentals built on the hardware v_exp_f32 / v_rcp_f32 instructions;
// * the decoupled look-back status words (agent-scope release / acquire, which
//   the compiler lowers to an L2 write-back / invalidate so tiles on different
//   XCDs see each other's payloads).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace prnn {

struct bf16 {
  uint16_t bits;
};

__device__ __forceinline__ float to_f32(float v) { return v; }
__device__ __forceinline__ float to_f32(bf16 v) {
  return __uint_as_float(static_cast<uint32_t>(v.bits) << 16);
}

// Round-to-nearest-even, NaN kept quiet (matches torch's float -> bfloat16).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

template <typename T>
__device__ __forceinline__ T from_f32(float v);
template <>
__device__ __forceinline__ float from_f32<float>(float v) { return v; }
template <>
__device__ __forceinline__ bf16 from_f32<bf16>(float v) { return bf16{f32_to_bf16_bits(v)}; }

// Value after a round trip through storage type T (identity for fp32).
template <typename T>
__device__ __forceinline__ float round_to(float v) { return to_f32(from_f32<T>(v)); }

template <typename T>
__device__ __forceinline__ float ld(const T* p) { return to_f32(*p); }
template <typename T>
__device__ __forceinline__ void st(T* p, float v) { *p = from_f32<T>(v); }

// exp(x) = 2^(x log2 e) on the hardware exp2 (1 ulp); exp(-inf) = 0.
__device__ __forceinline__ float fexp(float x) {
  return __builtin_amdgcn_exp2f(x * 1.4426950408889634f);
}
__device__ __forceinline__ float frcp(float x) { return __builtin_amdgcn_rcpf(x); }

__device__ __forceinline__ float fsigmoid(float x) { return frcp(1.0f + fexp(-x)); }

// tanh from exp(-2|x|) in (0, 1]: no overflow, absolute error ~1e-7.
__device__ __forceinline__ float ftanh(float x) {
  float e = fexp(-2.0f * fabsf(x));
  float t = (1.0f - e) * frcp(1.0f + e);
  return copysignf(t, x);
}

// Exactly-rounded product / sum with no FMA contraction: the reference's eager
// path evaluates ``wx + R * h`` as two torch ops.
__device__ __forceinline__ float mul_rn(float a, float b) { return __fmul_rn(a, b); }
__device__ __forceinline__ float add_rn(float a, float b) { return __fadd_rn(a, b); }

// ---- decoupled look-back status words -------------------------------------
// A status word holds (epoch << 2) | state.  The epoch is the index of the
// launch within one solver call; the workspace is zeroed at the start of every
// call, so a word left by an earlier launch of the same call (smaller epoch)
// or by an earlier call (zeroed) never reads as ready.
enum : int { kStatusAgg = 1, kStatusIncl = 2 };

// Called by every lane of the publishing wave after its payload stores: the
// release fence orders each lane's own stores, then lane 0 sets the word.
__device__ __forceinline__ void publish(int* flag, int epoch, int state, int lane) {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
  if (lane == 0)
    __hip_atomic_store(flag, (epoch << 2) | state, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Spin until the word carries this epoch; return its state.  Every tile that
// is waited on has a smaller ticket than the waiter, so it is already resident
// and finishes without waiting on the waiter: the spin always ends.
__device__ __forceinline__ int wait_status(const int* flag, int epoch) {
  int v;
  while (true) {
    v = __hip_atomic_load(flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if ((v >> 2) == epoch) break;
    __builtin_amdgcn_s_sleep(1);
  }
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  return v & 3;
}

// Payload loads after the acquire fence; plain loads are enough there.
__device__ __forceinline__ float ld_payload(const float* p) { return *p; }

}  // namespace prnn
