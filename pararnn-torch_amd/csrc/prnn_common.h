// Shared device helpers for the pararnn_amd HIP kernels (gfx950 / CDNA4).
//
// * bf16 and fp16 storage as raw 16-bit words with round-to-nearest-even
//   conversion;
// * transcendentals built on the hardware v_exp_f32 / v_rcp_f32 instructions;
// * the decoupled look-back's tagged words (device-coherent atomics);
// * buffer-resource loads / stores with wave-uniform offsets, and packed bf16.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace prnn {

struct bf16 {
  uint16_t bits;
};
// IEEE binary16 storage (the algebra stays fp32; 65504 is the largest finite
// value, so wider values round to +-inf as in the tensor dtype).
struct f16 {
  uint16_t bits;
};

__device__ __forceinline__ float to_f32(float v) { return v; }
__device__ __forceinline__ float to_f32(bf16 v) {
  return __uint_as_float(static_cast<uint32_t>(v.bits) << 16);
}
__device__ __forceinline__ float to_f32(f16 v) {
  return static_cast<float>(__builtin_bit_cast(_Float16, v.bits));
}

template <typename T>
__device__ __forceinline__ T from_f32(float v);
template <>
__device__ __forceinline__ float from_f32<float>(float v) { return v; }
// gfx950 converts with round-to-nearest-even in hardware (v_cvt_pk_bf16_f32).
template <>
__device__ __forceinline__ bf16 from_f32<bf16>(float v) {
  const __bf16 h = static_cast<__bf16>(v);
  return bf16{__builtin_bit_cast(uint16_t, h)};
}

template <>
__device__ __forceinline__ f16 from_f32<f16>(float v) {
  return f16{__builtin_bit_cast(uint16_t, static_cast<_Float16>(v))};
}

// Value after a round trip through storage type T (identity for fp32).
template <typename T>
__device__ __forceinline__ float round_to(float v) { return to_f32(from_f32<T>(v)); }
template <>
__device__ __forceinline__ float round_to<bf16>(float v) {
  return static_cast<float>(static_cast<__bf16>(v));
}

template <>
__device__ __forceinline__ float round_to<f16>(float v) {
  return static_cast<float>(static_cast<_Float16>(v));
}

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
  // e^{-2|x|} = 2^{|x| * (-2 log2 e)}: one multiply feeds the exp2.
  float e = __builtin_amdgcn_exp2f(fabsf(x) * -2.8853900817779268f);
  float t = (1.0f - e) * frcp(1.0f + e);
  return copysignf(t, x);
}

// tanh(x) = 1 - 2 / (e^{2x} + 1): five operations instead of seven, the same
// absolute error (~1e-7; the cancellation near 0 is the one of ftanh).
// e^{2x} = inf gives 1 and e^{2x} = 0 gives -1, so no input overflows.  The
// Newton and backward cell evaluations use it; in the frozen-gate passes it
// measured slower than ftanh (2.06 against 1.97 ms for the config-3 warm
// start), so those keep ftanh.
__device__ __forceinline__ float ftanh5(float x) {
  const float e = __builtin_amdgcn_exp2f(x * 2.8853900817779268f);
  return fmaf(-2.0f, frcp(1.0f + e), 1.0f);
}

// Separately rounded product / sum: never contracted into an FMA, for the
// places that restate two eager torch ops (``wx + R * h`` of the frozen-gate
// passes).  Elsewhere the kernels let the compiler contract, as the
// reference's fused kernels do.
__device__ __forceinline__ float mul_rn(float a, float b) {
#pragma clang fp contract(off)
  return a * b;
}
__device__ __forceinline__ float add_rn(float a, float b) {
#pragma clang fp contract(off)
  return a + b;
}

// ---- decoupled look-back ----------------------------------------------------
// Cross-tile data moves through agent-scope relaxed atomics: the compiler
// lowers them to vector loads / stores with the sc1 bit, which write through
// and bypass the per-XCD L2, so a tile on one XCD sees another XCD's data at
// the device-coherent level (the memory-side cache) without any L2 write-back
// or invalidate.  Every published value is a "tagged word": 64-bit
// {float bits, tag} written and read as one atomic word.  A word whose tag
// equals the current epoch is valid, so no status flag or store ordering is
// needed and one load both tests and fetches a value.
//
// The epoch is the index of the launch within one solver call (>= 1).  The
// tagged words are cleared at the start of every call, so nothing left by an
// earlier call or an earlier launch reads as valid.

__device__ __forceinline__ void st_tagged(unsigned long long* p, float v, int tag) {
  const unsigned long long w =
      (static_cast<unsigned long long>(static_cast<uint32_t>(tag)) << 32) | __float_as_uint(v);
  __hip_atomic_store(p, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// True (and v set) when the word carries this tag.
__device__ __forceinline__ bool ld_tagged(const unsigned long long* p, int tag, float& v) {
  const unsigned long long w = __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  v = __uint_as_float(static_cast<uint32_t>(w));
  return static_cast<int>(w >> 32) == tag;
}

// ---- buffer access ----------------------------------------------------------
// Streams are read and written through buffer resources: the per-step offset
// is a wave-uniform SGPR (soffset), so a step costs no 64-bit address
// arithmetic.  A lane whose offset is kOOB is outside every resource: its
// loads return 0 and its stores are dropped, which masks channels past d.
using rsrc_t = __amdgpu_buffer_rsrc_t;
constexpr uint32_t kOOB = 0x80000000u;

// Raw (stride 0) resource over `bytes` bytes from `base` (CDNA dword 3).
// Callers pass wave-uniform values; readfirstlane keeps the descriptor in
// SGPRs even where the compiler has copied a uniform operand into a VGPR
// (otherwise every buffer access through it becomes a readfirstlane loop).
__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(a));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(a >> 32));
  void* p = reinterpret_cast<void*>((static_cast<uint64_t>(hi) << 32) | lo);
  return __builtin_amdgcn_make_buffer_rsrc(p, static_cast<short>(0),
                                           static_cast<int>(__builtin_amdgcn_readfirstlane(bytes)),
                                           0x00020000);
}

// Raw storage bits of one element (bf16: zero-extended 16-bit word).
__device__ __forceinline__ uint32_t ldb_bits(bf16*, rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b16(r, voff, soff, 0);
}
__device__ __forceinline__ uint32_t ldb_bits(float*, rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0);
}
__device__ __forceinline__ uint32_t ldb_bits(f16*, rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b16(r, voff, soff, 0);
}
__device__ __forceinline__ float bits_to_f32(bf16*, uint32_t b) { return __uint_as_float(b << 16); }
__device__ __forceinline__ float bits_to_f32(f16*, uint32_t b) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(b)));
}
__device__ __forceinline__ float bits_to_f32(float*, uint32_t b) { return __uint_as_float(b); }

template <typename T>
__device__ __forceinline__ float ldb(rsrc_t r, uint32_t voff, uint32_t soff) {
  return bits_to_f32(static_cast<T*>(nullptr), ldb_bits(static_cast<T*>(nullptr), r, voff, soff));
}
template <typename T>
__device__ __forceinline__ void stb(rsrc_t r, uint32_t voff, uint32_t soff, float v);
template <>
__device__ __forceinline__ void stb<bf16>(rsrc_t r, uint32_t voff, uint32_t soff, float v) {
  __builtin_amdgcn_raw_buffer_store_b16(from_f32<bf16>(v).bits, r, voff, soff, 0);
}
template <>
__device__ __forceinline__ void stb<f16>(rsrc_t r, uint32_t voff, uint32_t soff, float v) {
  __builtin_amdgcn_raw_buffer_store_b16(from_f32<f16>(v).bits, r, voff, soff, 0);
}
template <>
__device__ __forceinline__ void stb<float>(rsrc_t r, uint32_t voff, uint32_t soff, float v) {
  __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), r, voff, soff, 0);
}

// Two floats rounded to bf16 (RNE) and packed low | high << 16 in one
// v_cvt_pk_bf16_f32; unpacked halves are exact floats.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float float2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(float2_t{lo, hi}, bf16x2_t));
}
__device__ __forceinline__ float lo_bf16(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi_bf16(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_f16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(float2_t{lo, hi}, f16x2_t));
}
__device__ __forceinline__ float lo_f16(uint32_t w) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w)));
}
__device__ __forceinline__ float hi_f16(uint32_t w) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w >> 16)));
}

// Two values of a 16-bit storage type in one register (low | high << 16):
// pack rounds two floats (RNE), lo / hi read one back exactly, and val reads
// one zero-extended raw storage word.
template <typename T>
struct Narrow;

template <>
struct Narrow<bf16> {
  static __device__ __forceinline__ uint32_t pack(float lo, float hi) {
    return pack_bf16x2(lo, hi);
  }
  static __device__ __forceinline__ float lo(uint32_t w) { return lo_bf16(w); }
  static __device__ __forceinline__ float hi(uint32_t w) { return hi_bf16(w); }
  static __device__ __forceinline__ float val(uint32_t bits) { return __uint_as_float(bits << 16); }
};

template <>
struct Narrow<f16> {
  static __device__ __forceinline__ uint32_t pack(float lo, float hi) {
    return pack_f16x2(lo, hi);
  }
  static __device__ __forceinline__ float lo(uint32_t w) { return lo_f16(w); }
  static __device__ __forceinline__ float hi(uint32_t w) { return hi_f16(w); }
  static __device__ __forceinline__ float val(uint32_t bits) { return lo_f16(bits); }
};

}  // namespace prnn
