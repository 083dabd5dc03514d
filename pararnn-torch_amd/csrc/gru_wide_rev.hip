// The eq. 2.6 adjoint walk of the wide-head tier (64 < d_head <= 128), in a
// translation unit of its own: the build compiles it with the iterative ILP
// scheduler, which shortens its per-step chain (the forward walks run slower
// under that scheduler).
#include "gru_wide.h"

namespace prnn {
namespace gruw {

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
  __shared__ __attribute__((aligned(16))) float s_dz[kVec];
  __shared__ __attribute__((aligned(16))) float s_dn[kVec];
  __shared__ __attribute__((aligned(16))) float s_dr[kVec];
  __shared__ float s_in[2][kIn][kS][DW];
  const Role rl = role();
  const int c = rl.c;
  const int sc = slot(c);
  const int head = blockIdx.x % H;
  const Span sp = span_of(blockIdx.x / H, T, cu);
  const size_t hoff = static_cast<size_t>(head) * dh * dh;
  float az[kK], ar[kK], an[kK];
  load_pair<TX, false>(a_z + hoff, dh, rl, az);
  load_pair<TX, false>(a_r + hoff, dh, rl, ar);
  load_pair<TX, false>(a_n + hoff, dh, rl, an);
  const int d = H * dh;
  const bool live = c < dh;
  const size_t col = static_cast<size_t>(head) * dh + c;
  float nu = 0.f;
  if (sp.t0 >= sp.t1) return;
  const size_t row_base = static_cast<size_t>(sp.row) * T * d;
  const rsrc_t rg = make_rsrc(g_wx + row_base * 3,
                              static_cast<uint32_t>(static_cast<size_t>(T) * 3 * d * sizeof(float)));
  const uint32_t vg = (live && rl.wr) ? static_cast<uint32_t>(col * sizeof(float)) : kOOB;
  store_block(s_in[0], load_block(z, r, n, hp, grad, row_base, d, head, dh, sp.t1 - 1, -1,
                                  sp.t0, sp.t1 - 1), dh);
  __syncthreads();
  int buf = 0;
  for (int tb = sp.t1 - 1; tb >= sp.t0; tb -= kS) {
    const bool more = tb - kS >= sp.t0;
    Staged next;
    if (more)
      next = load_block(z, r, n, hp, grad, row_base, d, head, dh, tb - kS, -1, sp.t0, sp.t1 - 1);
    const int ns = min(kS, tb - sp.t0 + 1);
    for (int s = 0; s < ns; ++s) {
      const int t = tb - s;
      const float zt = s_in[buf][0][s][c], rt = s_in[buf][1][s][c], nt = s_in[buf][2][s][c];
      const float ht = s_in[buf][3][s][c], g = s_in[buf][4][s][c];
      const float mu = g + nu;
      const float dz = mu * (nt - ht) * zt * (1.f - zt);
      const float dn = mu * zt * (1.f - nt * nt);
      if (rl.wr) {
        s_dz[sc] = dz;
        s_dn[sc] = dn;
      }
      __syncthreads();
      const float du = dot_pair(an, s_dn, rl);
      const float azdz = dot_pair(az, s_dz, rl);
      const float dr = du * ht * rt * (1.f - rt);
      if (rl.wr) s_dr[sc] = dr;
      __syncthreads();
      const float ardr = dot_pair(ar, s_dr, rl);
      nu = (1.f - zt) * mu + azdz + rt * du + ardr;
      // buffer stores, dropped for the other lanes
      const uint32_t so = static_cast<uint32_t>(t) * (3 * d * sizeof(float));
      stb<float>(rg, vg, so, dz);
      stb<float>(rg, vg, so + d * sizeof(float), dr);
      stb<float>(rg, vg, so + 2 * d * sizeof(float), dn);
    }
    // (the other staging buffer was last read a block ago, before this
    // block's barriers)
    if (more) {
      store_block(s_in[buf ^ 1], next, dh);
      __syncthreads();
    }
    buf ^= 1;
  }
  // nu at the sequence's first step: dL/dh0 of its row
  if (rl.wr && live && g_h0 != nullptr) g_h0[static_cast<size_t>(sp.seq) * d + col] = nu;
}

}  // namespace gruw
}  // namespace prnn

using namespace prnn;

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
