// T = 1 decode: one recurrent step per call, for the serving loop
// (reference kernels/decode.py:119-597).  The input projection W_x(x) stays a
// library GEMM; these kernels are the rest of cell.step: read the state row
// (or the pool slot block_table[b]), the recurrent parameters (clamped to
// +-cap in-kernel, as the reference does so a captured graph allocates
// nothing) and the step's wx, and write the next state row.  fp32 algebra,
// 16-bit storage (bf16, fp16) widened on load and rounded on store.
//
//  slstm_decode_kernel     ParaSLSTM mix='diag': one thread per channel.
//  gru_diag_decode_kernel  ParaGRU mix='diag': one thread per channel.
//  gru_head_decode_kernel  ParaGRU mix='head' (d_head = 64): one wave per
//                          (b, head); lane j forms column j of h A_z, h A_r,
//                          (h r) A_n from the head's A columns with h broadcast
//                          through LDS.  (The reference runs this mix through
//                          the eager cell.step.)
#include "prnn_common.h"
#include "pararnn_amd.h"
#include "prnn_host.h"

namespace prnn {
namespace decode {

__device__ __forceinline__ float cap_to(float v, float cap, bool has_cap) {
  return has_cap ? fminf(fmaxf(v, -cap), cap) : v;
}

__device__ __forceinline__ int slot_of(const int* bt, int b) { return bt ? bt[b] : b; }

// torch.lerp(start, end, weight) for fp32 (the head cell's update).
__device__ __forceinline__ float lerp_t(float s, float e, float w) {
  return w < 0.5f ? s + w * (e - s) : e - (e - s) * (1.f - w);
}

template <typename TX>
__global__ __launch_bounds__(256) void slstm_decode_kernel(
    const TX* __restrict__ state, const TX* __restrict__ wx, const TX* __restrict__ r,
    TX* __restrict__ out, const int* __restrict__ bt, int d, float eps, float cap, int has_cap) {
  const int b = blockIdx.y;
  const int j = blockIdx.x * 256 + threadIdx.x;
  if (j >= d) return;
  const size_t row = static_cast<size_t>(slot_of(bt, b)) * 4 * d;
  const float c = ld(state + row + j), n = ld(state + row + d + j);
  const float m = ld(state + row + 2 * d + j), h = ld(state + row + 3 * d + j);
  const TX* x = wx + static_cast<size_t>(b) * 4 * d + j;
  float z[4];
#pragma unroll
  for (int g = 0; g < 4; ++g) z[g] = cap_to(ld(r + g * d + j), cap, has_cap) * h + ld(x + g * d);
  const float left = z[1] + m;
  const float mn = fmaxf(left, z[0]);
  // one of f, i is exactly e^0 = 1 (the larger exponent is the stabiliser)
  const float e = fexp(-fabsf(left - z[0]));
  const bool lf = left >= z[0];
  const float f = lf ? 1.f : e, i = lf ? e : 1.f;
  const float nn = f * n + i;
  const float cn = f * c + i * ftanh(z[2]);
  const float hn = fsigmoid(z[3]) * (cn / (nn + eps));
  st(out + row + j, cn);
  st(out + row + d + j, nn);
  st(out + row + 2 * d + j, mn);
  st(out + row + 3 * d + j, hn);
}

template <typename TX>
__global__ __launch_bounds__(256) void gru_diag_decode_kernel(
    const TX* __restrict__ hin, const TX* __restrict__ wx, const TX* __restrict__ a_z,
    const TX* __restrict__ a_r, const TX* __restrict__ a_n, TX* __restrict__ out,
    const int* __restrict__ bt, int d, float cap, int has_cap) {
  const int b = blockIdx.y;
  const int j = blockIdx.x * 256 + threadIdx.x;
  if (j >= d) return;
  const size_t row = static_cast<size_t>(slot_of(bt, b)) * d;
  const float h = ld(hin + row + j);
  const TX* x = wx + static_cast<size_t>(b) * 3 * d + j;
  const float z = fsigmoid(cap_to(ld(a_z + j), cap, has_cap) * h + ld(x));
  const float rr = fsigmoid(cap_to(ld(a_r + j), cap, has_cap) * h + ld(x + d));
  const float n = ftanh(cap_to(ld(a_n + j), cap, has_cap) * (h * rr) + ld(x + 2 * d));
  st(out + row + j, (1.f - z) * h + z * n);
}

constexpr int DH = 64;

template <typename TX>
__global__ __launch_bounds__(64) void gru_head_decode_kernel(
    const TX* __restrict__ hin, const TX* __restrict__ wx, const TX* __restrict__ a_z,
    const TX* __restrict__ a_r, const TX* __restrict__ a_n, TX* __restrict__ out,
    const int* __restrict__ bt, int H, float cap, int has_cap) {
  __shared__ float s_v[DH];
  const int b = blockIdx.y, head = blockIdx.x, j = threadIdx.x;
  const int d = H * DH;
  const size_t row = static_cast<size_t>(slot_of(bt, b)) * d + head * DH;
  const float h = ld(hin + row + j);
  const TX* x = wx + static_cast<size_t>(b) * 3 * d + head * DH + j;
  const size_t hoff = static_cast<size_t>(head) * DH * DH + j;  // column j of the head's (in, out) matrices
  s_v[j] = h;
  __syncthreads();
  float gz = 0.f, gr = 0.f;
#pragma unroll 8
  for (int i = 0; i < DH; ++i) {
    const float v = s_v[i];
    gz += v * cap_to(ld(a_z + hoff + i * DH), cap, has_cap);
    gr += v * cap_to(ld(a_r + hoff + i * DH), cap, has_cap);
  }
  const float z = fsigmoid(gz + ld(x));
  const float rr = fsigmoid(gr + ld(x + d));
  __syncthreads();
  s_v[j] = h * rr;
  __syncthreads();
  float gn = 0.f;
#pragma unroll 8
  for (int i = 0; i < DH; ++i) gn += s_v[i] * cap_to(ld(a_n + hoff + i * DH), cap, has_cap);
  const float n = ftanh(gn + ld(x + 2 * d));
  st(out + row + j, lerp_t(h, n, z));
}

static int check(int B, int d, int dtype) {
  if (B < 1 || d < 1) return fail(PRNN_ERR_VALUE, "B and d must be >= 1, got B=%d d=%d", B, d);
  if (check_dtype(dtype) != PRNN_OK) return PRNN_ERR_TYPE;
  if (B > 65535) return fail(PRNN_ERR_VALUE, "batch %d exceeds 65535", B);
  return PRNN_OK;
}

}  // namespace decode
}  // namespace prnn

using namespace prnn;

extern "C" PRNN_API int prnn_slstm_decode(const void* state, const void* wx, const void* r,
                                          void* out, const int* block_table, int B, int d,
                                          float eps, float cap, int has_cap, int dtype,
                                          void* stream) {
  int rc = decode::check(B, d, dtype);
  if (rc != PRNN_OK) return rc;
  if (!state || !wx || !r || !out)
    return fail(PRNN_ERR_VALUE, "state, wx, r and out must be non-null");
  const dim3 grid((d + 255) / 256, B);
  hipStream_t s = static_cast<hipStream_t>(stream);
  with_storage(dtype, [&](auto tag) {
    using TX = decltype(tag);
    decode::slstm_decode_kernel<TX><<<grid, dim3(256), 0, s>>>(
        static_cast<const TX*>(state), static_cast<const TX*>(wx), static_cast<const TX*>(r),
        static_cast<TX*>(out), block_table, d, eps, cap, has_cap);
    return PRNN_OK;
  });
  PRNN_HIP(hipGetLastError());
  return PRNN_OK;
}

extern "C" PRNN_API int prnn_gru_decode(const void* h, const void* wx, const void* a_z,
                                        const void* a_r, const void* a_n, void* out,
                                        const int* block_table, int B, int d, int n_heads,
                                        float cap, int has_cap, int dtype, void* stream) {
  int rc = decode::check(B, d, dtype);
  if (rc != PRNN_OK) return rc;
  if (!h || !wx || !a_z || !a_r || !a_n || !out)
    return fail(PRNN_ERR_VALUE, "h, wx, a_z, a_r, a_n and out must be non-null");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (n_heads > 0) {
    if (d != n_heads * decode::DH)
      return fail(PRNN_ERR_TYPE, "head decode needs d_head = 64, got d=%d n_heads=%d", d,
                  n_heads);
    const dim3 grid(n_heads, B);
    with_storage(dtype, [&](auto tag) {
      using TX = decltype(tag);
      decode::gru_head_decode_kernel<TX><<<grid, dim3(64), 0, s>>>(
          static_cast<const TX*>(h), static_cast<const TX*>(wx), static_cast<const TX*>(a_z),
          static_cast<const TX*>(a_r), static_cast<const TX*>(a_n), static_cast<TX*>(out),
          block_table, n_heads, cap, has_cap);
      return PRNN_OK;
    });
  } else {
    const dim3 grid((d + 255) / 256, B);
    with_storage(dtype, [&](auto tag) {
      using TX = decltype(tag);
      decode::gru_diag_decode_kernel<TX><<<grid, dim3(256), 0, s>>>(
          static_cast<const TX*>(h), static_cast<const TX*>(wx), static_cast<const TX*>(a_z),
          static_cast<const TX*>(a_r), static_cast<const TX*>(a_n), static_cast<TX*>(out),
          block_table, d, cap, has_cap);
      return PRNN_OK;
    });
  }
  PRNN_HIP(hipGetLastError());
  return PRNN_OK;
}
