// ParaGRU mix='head' with wide heads (64 < d_head <= 128): the Newton
// iteration's linear solve and the eq. 2.6 adjoint as walks over time, one
// workgroup per (sequence, head).
//
// This is the tier of the reference's streamed head kernel
// (kernels/newton_gru_head.py:765-960, _newton_head_stream_a_kernel: one
// program per (b, head), a serial walk over T per Newton iteration, A_* read
// in fp32).  Here the parts of an iteration that do not depend on the walk
// run beforehand as wide parallel work (the gates z, r, n at the iterate:
// three GEMMs over all B*T rows and elementwise ops, issued by the host), so a
// walk step is only the Jacobian applied to the previous delta,
//     J delta = (1-z) delta + d2 (A_z^T delta) + d3 A_n^T (r delta + d5 (A_r^T delta))
// with d2 = (n-h) z(1-z), d3 = z(1-n^2), d5 = h r(1-r) (reference
// cells/para_gru.py:385-412), three 128-wide mat-vecs.
//
// Workgroup: 512 lanes = 128 channels x 4 quarters of the contraction index.
// Lane (c, q) keeps 32 entries of each A in registers -- column c (forward:
// A^T products) or row c (adjoint: A products) over k in [32 q, 32 q + 32) --
// and the quarters' partial sums meet in LDS in a fixed order (the result
// does not depend on scheduling).  fp32 throughout; lanes c >= d_head and
// entries k >= d_head hold zeros.
#include "prnn_common.h"
#include "pararnn_amd.h"
#include "prnn_host.h"

namespace prnn {
namespace gruw {

constexpr int DW = 128;       // widest head
constexpr int kQ = 4;         // quarters of the contraction index
constexpr int kK = DW / kQ;   // entries per lane and matrix
constexpr int kThreads = DW * kQ;

// torch.lerp(start, end, weight) for fp32 (the cell's update).
__device__ __forceinline__ float lerp_t(float s, float e, float w) {
  return w < 0.5f ? s + w * (e - s) : e - (e - s) * (1.f - w);
}

// Steps [t0, t1) of batch row `row` that workgroup `seq / H` walks: a batch
// row (rectangular) or a packed sequence of one stream (cu != nullptr).
struct Span {
  int row, t0, t1, seq;
};
__device__ __forceinline__ Span span_of(int s, int T, const int* cu) {
  if (cu == nullptr) return Span{s, 0, T, s};
  return Span{0, cu[s], cu[s + 1], s};
}

// Entries k in [32 q, 32 q + 32) of column c (COL) or row c of a head's A
// ((in, out) layout, d_head x d_head), zero outside the head.
template <typename TX, bool COL>
__device__ __forceinline__ void load_quarter(const TX* A, int dh, int c, int q, float a[kK]) {
#pragma unroll
  for (int kk = 0; kk < kK; ++kk) {
    const int k = q * kK + kk;
    const bool in = c < dh && k < dh;
    a[kk] = in ? ld(A + (COL ? static_cast<size_t>(k) * dh + c : static_cast<size_t>(c) * dh + k))
               : 0.f;
  }
}

// One step's per-channel inputs, loaded two steps ahead of their use: a walk
// step is short, so a load issued at the step that needs it would wait for
// the full memory latency every step.
struct StepIn {
  float z, r, n, hp, x;  // x: the iterate (forward) or dL/dH (adjoint)
};

template <typename TG>
__device__ __forceinline__ StepIn load_step(const float* __restrict__ z, const float* __restrict__ r,
                                            const float* __restrict__ n,
                                            const float* __restrict__ hp, const TG* __restrict__ x,
                                            size_t at, bool ok) {
  StepIn v{0.f, 0.f, 0.f, 0.f, 0.f};
  if (ok) {
    v.z = z[at];
    v.r = r[at];
    v.n = n[at];
    v.hp = hp[at];
    v.x = ld(x + at);
  }
  return v;
}

__device__ __forceinline__ float dot_quarter(const float a[kK], const float* __restrict__ v) {
  float acc = 0.f;
#pragma unroll
  for (int kk = 0; kk < kK; kk += 4) {
    const float4 x = *reinterpret_cast<const float4*>(v + kk);
    acc = fmaf(a[kk], x.x, acc);
    acc = fmaf(a[kk + 1], x.y, acc);
    acc = fmaf(a[kk + 2], x.z, acc);
    acc = fmaf(a[kk + 3], x.w, acc);
  }
  return acc;
}

// Forward walk of one Newton iteration: delta_t = J_t delta_{t-1} + F_t with
// F_t = lerp(hp, n, z) - H_t, then H_t + omega delta_t.  z, r, n and hp (the
// iterate's previous state, the sequence's h0 at its first step) are fp32
// (B, T, d); hin is the iterate (fp32), out receives the next one (TOUT).
// The Jacobian of a sequence's first step multiplies delta = 0, so nothing
// crosses a sequence start.
template <typename TX, typename TOUT>
__global__ __launch_bounds__(kThreads) void gruw_walk_kernel(
    const float* __restrict__ z, const float* __restrict__ r, const float* __restrict__ n,
    const float* __restrict__ hp, const float* __restrict__ hin, const TX* __restrict__ a_z,
    const TX* __restrict__ a_r, const TX* __restrict__ a_n, TOUT* __restrict__ out, int T,
    int H, int dh, float omega, const int* __restrict__ cu) {
  __shared__ __attribute__((aligned(16))) float s_d[DW];
  __shared__ __attribute__((aligned(16))) float s_w[DW];
  __shared__ float s_p[3][kQ][DW];
  const int c = threadIdx.x & (DW - 1), q = threadIdx.x / DW;
  const int head = blockIdx.x % H;
  const Span sp = span_of(blockIdx.x / H, T, cu);
  const size_t hoff = static_cast<size_t>(head) * dh * dh;
  float az[kK], ar[kK], an[kK];
  load_quarter<TX, true>(a_z + hoff, dh, c, q, az);
  load_quarter<TX, true>(a_r + hoff, dh, c, q, ar);
  load_quarter<TX, true>(a_n + hoff, dh, c, q, an);
  const int d = H * dh;
  const bool live = c < dh;
  const size_t col = static_cast<size_t>(head) * dh + c;
  if (q == 0) s_d[c] = 0.f;
  float delta = 0.f;
  __syncthreads();
  const size_t base = static_cast<size_t>(sp.row) * T * d + col;
  StepIn p0 = load_step(z, r, n, hp, hin, base + static_cast<size_t>(sp.t0) * d,
                        live && sp.t0 < sp.t1);
  StepIn p1 = load_step(z, r, n, hp, hin, base + static_cast<size_t>(sp.t0 + 1) * d,
                        live && sp.t0 + 1 < sp.t1);
  for (int t = sp.t0; t < sp.t1; ++t) {
    const size_t at = base + static_cast<size_t>(t) * d;
    const StepIn cur = p0;
    p0 = p1;
    p1 = load_step(z, r, n, hp, hin, at + 2 * static_cast<size_t>(d), live && t + 2 < sp.t1);
    const float zt = cur.z, rt = cur.r, nt = cur.n, ht = cur.hp, hv = cur.x;
    // stage 1: A_r^T delta and A_z^T delta, this quarter of k
    s_p[0][q][c] = dot_quarter(ar, s_d + q * kK);
    s_p[1][q][c] = dot_quarter(az, s_d + q * kK);
    __syncthreads();
    const float sr = ((s_p[0][0][c] + s_p[0][1][c]) + s_p[0][2][c]) + s_p[0][3][c];
    const float sz = ((s_p[1][0][c] + s_p[1][1][c]) + s_p[1][2][c]) + s_p[1][3][c];
    const float d5 = ht * rt * (1.f - rt);
    if (q == 0) s_w[c] = rt * delta + d5 * sr;
    __syncthreads();
    // stage 2: A_n^T (r delta + d5 A_r^T delta)
    s_p[2][q][c] = dot_quarter(an, s_w + q * kK);
    __syncthreads();
    const float sn = ((s_p[2][0][c] + s_p[2][1][c]) + s_p[2][2][c]) + s_p[2][3][c];
    const float d2 = (nt - ht) * zt * (1.f - zt);
    const float d3 = zt * (1.f - nt * nt);
    const float f = lerp_t(ht, nt, zt) - hv;
    delta = (1.f - zt) * delta + d2 * sz + d3 * sn + f;
    if (!live) delta = 0.f;
    if (q == 0) {
      s_d[c] = delta;
      if (live) st(out + at, hv + omega * delta);
    }
    __syncthreads();
  }
}

// Adjoint walk at H* (eq. 2.6): from the last step down,
//   mu_t = g_t + nu_{t+1},  nu_t = J_t^T mu_t
// through the cell's VJP (reference kernels/gru_head_factor.py:68-112):
//   d_zpre = mu (n - h) z(1-z),  d_npre = mu z(1-n^2),  d_u = A_n d_npre,
//   d_rpre = d_u h r(1-r),  nu = (1-z) mu + A_z d_zpre + r d_u + A_r d_rpre.
// Writes the pre-activation gradients (dL/dwx, gate blocks z, r, n) in fp32
// and, at each sequence's first step, nu = dL/dh0 of that sequence's row.
template <typename TX, typename TG>
__global__ __launch_bounds__(kThreads) void gruw_reverse_kernel(
    const float* __restrict__ z, const float* __restrict__ r, const float* __restrict__ n,
    const float* __restrict__ hp, const TG* __restrict__ grad, const TX* __restrict__ a_z,
    const TX* __restrict__ a_r, const TX* __restrict__ a_n, float* __restrict__ g_wx,
    float* __restrict__ g_h0, int T, int H, int dh, const int* __restrict__ cu) {
  __shared__ __attribute__((aligned(16))) float s_dz[DW];
  __shared__ __attribute__((aligned(16))) float s_dn[DW];
  __shared__ __attribute__((aligned(16))) float s_dr[DW];
  __shared__ float s_p[3][kQ][DW];
  const int c = threadIdx.x & (DW - 1), q = threadIdx.x / DW;
  const int head = blockIdx.x % H;
  const Span sp = span_of(blockIdx.x / H, T, cu);
  const size_t hoff = static_cast<size_t>(head) * dh * dh;
  float az[kK], ar[kK], an[kK];
  load_quarter<TX, false>(a_z + hoff, dh, c, q, az);
  load_quarter<TX, false>(a_r + hoff, dh, c, q, ar);
  load_quarter<TX, false>(a_n + hoff, dh, c, q, an);
  const int d = H * dh;
  const bool live = c < dh;
  const size_t col = static_cast<size_t>(head) * dh + c;
  float nu = 0.f;
  const size_t base = static_cast<size_t>(sp.row) * T * d + col;
  StepIn p0 = load_step(z, r, n, hp, grad, base + static_cast<size_t>(sp.t1 - 1) * d,
                        live && sp.t1 - 1 >= sp.t0);
  StepIn p1 = load_step(z, r, n, hp, grad, base + static_cast<size_t>(sp.t1 - 2) * d,
                        live && sp.t1 - 2 >= sp.t0);
  for (int t = sp.t1 - 1; t >= sp.t0; --t) {
    const size_t at = base + static_cast<size_t>(t) * d;
    const StepIn cur = p0;
    p0 = p1;
    p1 = load_step(z, r, n, hp, grad, at - 2 * static_cast<size_t>(d), live && t - 2 >= sp.t0);
    const float zt = cur.z, rt = cur.r, nt = cur.n, ht = cur.hp, g = cur.x;
    const float mu = g + nu;
    const float dz = mu * (nt - ht) * zt * (1.f - zt);
    const float dn = mu * zt * (1.f - nt * nt);
    if (q == 0) {
      s_dz[c] = dz;
      s_dn[c] = dn;
    }
    __syncthreads();
    s_p[0][q][c] = dot_quarter(an, s_dn + q * kK);
    s_p[1][q][c] = dot_quarter(az, s_dz + q * kK);
    __syncthreads();
    const float du = ((s_p[0][0][c] + s_p[0][1][c]) + s_p[0][2][c]) + s_p[0][3][c];
    const float azdz = ((s_p[1][0][c] + s_p[1][1][c]) + s_p[1][2][c]) + s_p[1][3][c];
    const float dr = du * ht * rt * (1.f - rt);
    if (q == 0) s_dr[c] = dr;
    __syncthreads();
    s_p[2][q][c] = dot_quarter(ar, s_dr + q * kK);
    __syncthreads();
    const float ardr = ((s_p[2][0][c] + s_p[2][1][c]) + s_p[2][2][c]) + s_p[2][3][c];
    nu = (1.f - zt) * mu + azdz + rt * du + ardr;
    if (q == 0 && live) {
      float* gw = g_wx + (static_cast<size_t>(sp.row) * T + t) * 3 * d + col;
      gw[0] = dz;
      gw[d] = dr;
      gw[2 * static_cast<size_t>(d)] = dn;
      if (t == sp.t0 && g_h0 != nullptr) g_h0[static_cast<size_t>(sp.seq) * d + col] = nu;
    }
  }
}

static int check(int B, int T, int H, int dh, int dtype, const int* cu, int n_seq) {
  if (B < 1 || T < 1 || H < 1)
    return fail(PRNN_ERR_VALUE, "B, T, n_heads must be >= 1, got B=%d T=%d n_heads=%d", B, T, H);
  if (dh < 1 || dh > DW) return fail(PRNN_ERR_TYPE, "d_head must be in [1, %d], got %d", DW, dh);
  if (check_dtype(dtype) != PRNN_OK) return PRNN_ERR_TYPE;
  if (cu != nullptr && (B != 1 || n_seq < 1 || n_seq > T))
    return fail(PRNN_ERR_VALUE, "a packed stream has B = 1 and n_seq in [1, T], got B=%d n_seq=%d",
                B, n_seq);
  return PRNN_OK;
}

}  // namespace gruw
}  // namespace prnn

using namespace prnn;

extern "C" PRNN_API int prnn_gru_wide_walk(const float* z, const float* r, const float* n,
                                           const float* hp, const float* hin, const void* a_z,
                                           const void* a_r, const void* a_n, void* out,
                                           int out_f32, int B, int T, int n_heads, int d_head,
                                           float omega, int dtype, const int* cu_seqlens,
                                           int n_seq, void* stream) {
  int rc = gruw::check(B, T, n_heads, d_head, dtype, cu_seqlens, n_seq);
  if (rc != PRNN_OK) return rc;
  if (!z || !r || !n || !hp || !hin || !a_z || !a_r || !a_n || !out)
    return fail(PRNN_ERR_VALUE, "z, r, n, hp, hin, a_z, a_r, a_n and out must be non-null");
  if (!out_f32 && static_cast<const void*>(hin) == out)
    return fail(PRNN_ERR_VALUE, "a narrow out must not alias hin");
  const int seqs = (cu_seqlens ? n_seq : B) * n_heads;
  hipStream_t s = static_cast<hipStream_t>(stream);
  with_storage(dtype, [&](auto tag) {
    using TX = decltype(tag);
    const TX* az = static_cast<const TX*>(a_z);
    const TX* ar = static_cast<const TX*>(a_r);
    const TX* an = static_cast<const TX*>(a_n);
    if (out_f32)
      gruw::gruw_walk_kernel<TX, float><<<dim3(seqs), dim3(gruw::kThreads), 0, s>>>(
          z, r, n, hp, hin, az, ar, an, static_cast<float*>(out), T, n_heads, d_head, omega,
          cu_seqlens);
    else
      gruw::gruw_walk_kernel<TX, TX><<<dim3(seqs), dim3(gruw::kThreads), 0, s>>>(
          z, r, n, hp, hin, az, ar, an, static_cast<TX*>(out), T, n_heads, d_head, omega,
          cu_seqlens);
    return PRNN_OK;
  });
  PRNN_HIP(hipGetLastError());
  return PRNN_OK;
}

extern "C" PRNN_API int prnn_gru_wide_reverse(const float* z, const float* r, const float* n,
                                              const float* hp, const void* grad, int grad_f32,
                                              const void* a_z, const void* a_r, const void* a_n,
                                              float* g_wx, float* g_h0, int B, int T,
                                              int n_heads, int d_head, int dtype,
                                              const int* cu_seqlens, int n_seq, void* stream) {
  int rc = gruw::check(B, T, n_heads, d_head, dtype, cu_seqlens, n_seq);
  if (rc != PRNN_OK) return rc;
  if (!z || !r || !n || !hp || !grad || !a_z || !a_r || !a_n || !g_wx)
    return fail(PRNN_ERR_VALUE, "z, r, n, hp, grad, a_z, a_r, a_n and g_wx must be non-null");
  const int seqs = (cu_seqlens ? n_seq : B) * n_heads;
  hipStream_t s = static_cast<hipStream_t>(stream);
  with_storage(dtype, [&](auto tag) {
    using TX = decltype(tag);
    const TX* az = static_cast<const TX*>(a_z);
    const TX* ar = static_cast<const TX*>(a_r);
    const TX* an = static_cast<const TX*>(a_n);
    if (grad_f32)
      gruw::gruw_reverse_kernel<TX, float><<<dim3(seqs), dim3(gruw::kThreads), 0, s>>>(
          z, r, n, hp, static_cast<const float*>(grad), az, ar, an, g_wx, g_h0, T, n_heads,
          d_head, cu_seqlens);
    else
      gruw::gruw_reverse_kernel<TX, TX><<<dim3(seqs), dim3(gruw::kThreads), 0, s>>>(
          z, r, n, hp, static_cast<const TX*>(grad), az, ar, an, g_wx, g_h0, T, n_heads,
          d_head, cu_seqlens);
    return PRNN_OK;
  });
  PRNN_HIP(hipGetLastError());
  return PRNN_OK;
}
