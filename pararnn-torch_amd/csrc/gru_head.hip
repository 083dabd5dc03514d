// ParaGRU mix='head' Newton + scan kernels for gfx950 (CDNA4).
//
// Each (batch b, head) pair is an independent 64-dimensional recurrence
// ("sequence").  One Newton iteration solves delta_t = J_t delta_{t-1} + F_t
// over T steps with J_t the dense 64x64 head Jacobian
//     J = diag(1-z) + diag((n-h) z(1-z)) A_z^T
//         + diag(z (1-n^2)) A_n^T (diag(r) + diag(h r(1-r)) A_r^T)
// (reference cells/para_gru.py:385-412, solvers/scan.py:103-123).  Time is cut
// into chunks of kChunk steps:
//
//  gru_chunk_kernel   per chunk: gates of all steps, then the chunk transfer
//                     Phi = J_last ... J_first and the zero-carry local solution
//                     e (e <- J e + F).  Per step two 64x64x64 products on MFMA
//                     (v_mfma_f32_16x16x32_bf16, fp32 accumulate): the
//                     Jacobian's A_n^T D A_r^T term and J Phi; e is an fp32
//                     mat-vec on the assembled J;
//  gru_carry_kernel   per sequence: carry_c = Phi_c carry_{c-1} + e_c over the
//                     chunks, serially (one 64x64 mat-vec per chunk, fp32);
//  gru_replay_kernel  per chunk: the exact fp32 recurrence from the chunk's
//                     carry with the factorised J v (three 64-wide mat-vecs),
//                     then H += omega delta.
//
// Phi is composed from bf16-rounded operands and only multiplies the carry
// entering a chunk; e and every delta_t are fp32, so the bf16 rounding reaches
// the result only through Phi times the carry (measured ~1e-7 at K = 3).
#include "prnn_common.h"
#include "pararnn_amd.h"
#include "prnn_host.h"

namespace prnn {
namespace gru {

constexpr int DH = 64;      // head width handled by these kernels
constexpr int kChunk = 32;  // time steps per chunk
constexpr int kPad = 72;    // bf16 row stride of the LDS operand tiles (16-byte aligned rows)

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

// D(16x16) += A(16x32) B(32x16).  Lane l holds A[l%16][8(l/16)+q],
// B[8(l/16)+q][l%16] (q = 0..7) and D[4(l/16)+v][l%16] (v = 0..3).
__device__ __forceinline__ floatx4 mfma(bf16x8 a, bf16x8 b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// torch.lerp(start, end, weight) for fp32.
__device__ __forceinline__ float lerp_t(float s, float e, float w) {
  return w < 0.5f ? s + w * (e - s) : e - (e - s) * (1.f - w);
}

struct Geo {
  int n_seq, n_chunks;
};

// Index helpers.  wx is (B, T, 3d) with gate blocks (z, r, n); states (B, T, d).
__device__ __forceinline__ size_t wx_at(int b, int t, int T, int d, int gate, int head, int j) {
  return (static_cast<size_t>(b) * T + t) * 3 * d + static_cast<size_t>(gate) * d + head * DH + j;
}
__device__ __forceinline__ size_t h_at(int b, int t, int T, int d, int head, int j) {
  return (static_cast<size_t>(b) * T + t) * d + head * DH + j;
}

// Column j of a head's (in, out) matrix, i.e. A[i][j] for i = 0..63.
template <typename TX>
__device__ __forceinline__ void load_col(const TX* A, int head, int j, float col[DH]) {
  const TX* p = A + static_cast<size_t>(head) * DH * DH + j;
#pragma unroll
  for (int i = 0; i < DH; ++i) col[i] = ld(p + i * DH);
}

// (v @ A)[j] = sum_i v[i] A[i][j]; v broadcast from LDS, column j in registers.
__device__ __forceinline__ float vec_col(const float* __restrict__ v, const float col[DH]) {
  float acc = 0.f;
#pragma unroll
  for (int i = 0; i < DH; i += 4) {
    const float4 x = *reinterpret_cast<const float4*>(v + i);
    acc += x.x * col[i] + x.y * col[i + 1] + x.z * col[i + 2] + x.w * col[i + 3];
  }
  return acc;
}

// One head GRU step for lane j from h_prev (in s_h, wave-private LDS): gates
// and the new state (reference para_gru.py:443-467).  s_u is wave scratch.
struct Gates {
  float z, r, n, h_new;
};

__device__ __forceinline__ Gates gates_step(float* s_h, float* s_u, float hp_j, float zx, float rx,
                                            float nx, const float az[DH], const float ar[DH],
                                            const float an[DH], bool zero_h) {
  Gates g;
  float gz = 0.f, gr = 0.f;
  if (!zero_h) {
    gz = vec_col(s_h, az);
    gr = vec_col(s_h, ar);
  }
  g.z = fsigmoid(gz + zx);
  g.r = fsigmoid(gr + rx);
  float gn = 0.f;
  if (!zero_h) {
    s_u[threadIdx.x & 63] = hp_j * g.r;
    __builtin_amdgcn_wave_barrier();
    gn = vec_col(s_u, an);
  }
  g.n = ftanh(gn + nx);
  g.h_new = lerp_t(hp_j, g.n, g.z);
  return g;
}

// ---------------------------------------------------------------------------
// Initial guess: H_t = f(h_prev0_t, x_t), h_prev0 = 0 except h0 at t = 0
// (reference solvers/newton/__init__.py:925-940).  One wave per (sequence,
// block of 64 steps); only t = 0 with h0 needs the mat-vecs.
// ---------------------------------------------------------------------------
template <typename TX, typename TOUT>
__global__ __launch_bounds__(64) void gru_init_kernel(const TX* __restrict__ wx,
                                                     const TX* __restrict__ a_z,
                                                     const TX* __restrict__ a_r,
                                                     const TX* __restrict__ a_n,
                                                     const TX* __restrict__ h0,
                                                     TOUT* __restrict__ out, int B, int T, int H) {
  __shared__ float s_h[DH], s_u[DH];
  const int j = threadIdx.x;
  const int d = H * DH;
  const int n_blk = (T + 63) / 64;
  const int seq = blockIdx.x / n_blk, blk = blockIdx.x % n_blk;
  const int b = seq / H, head = seq % H;
  const int t0 = blk * 64, t1 = min(T, t0 + 64);
  for (int t = t0; t < t1; ++t) {
    const float zx = ld(wx + wx_at(b, t, T, d, 0, head, j));
    const float rx = ld(wx + wx_at(b, t, T, d, 1, head, j));
    const float nx = ld(wx + wx_at(b, t, T, d, 2, head, j));
    Gates g;
    if (t == 0 && h0 != nullptr) {
      float az[DH], ar[DH], an[DH];
      load_col(a_z, head, j, az);
      load_col(a_r, head, j, ar);
      load_col(a_n, head, j, an);
      const float hp = ld(h0 + static_cast<size_t>(b) * d + head * DH + j);
      s_h[j] = hp;
      __builtin_amdgcn_wave_barrier();
      g = gates_step(s_h, s_u, hp, zx, rx, nx, az, ar, an, false);
    } else {
      g.z = fsigmoid(zx);
      g.n = ftanh(nx);
      g.h_new = lerp_t(0.f, g.n, g.z);
    }
    st(out + h_at(b, t, T, d, head, j), g.h_new);
  }
}

// ---------------------------------------------------------------------------
// Chunk transfer.  256 threads = 4 waves; wave w owns rows 16w..16w+15 of
// every 64-row product.
// ---------------------------------------------------------------------------
struct ChunkShared {
  float vec[kChunk][5][DH];                   // per step: h_prev, z, r, n, F
  float h[4][DH], u[4][DH];                   // per-wave gate scratch
  float e[2][DH];                                          // local solution e (fp32)
  __attribute__((aligned(16))) __bf16 J[DH][kPad];         // J rows (row-major)
  __attribute__((aligned(16))) __bf16 phiT[2][DH][kPad];   // Phi transposed ([col][row])
};

template <typename TX>
__global__ __launch_bounds__(256) void gru_chunk_kernel(
    const TX* __restrict__ wx, const TX* __restrict__ a_z, const TX* __restrict__ a_r,
    const TX* __restrict__ a_n, const TX* __restrict__ h0, const float* __restrict__ hin, int B,
    int T, int H, int n_chunks, float* __restrict__ phi_out, float* __restrict__ e_out) {
  __shared__ ChunkShared sh;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int d = H * DH;
  const int seq = blockIdx.x / n_chunks, c = blockIdx.x % n_chunks;
  const int b = seq / H, head = seq % H;
  const int t0 = c * kChunk;
  const int len = min(kChunk, T - t0);

  // Phase A: gates, prediction and residual of every step (wave w: steps w, w+4, ...).
  {
    float az[DH], ar[DH], an[DH];
    load_col(a_z, head, lane, az);
    load_col(a_r, head, lane, ar);
    load_col(a_n, head, lane, an);
    for (int s = wave; s < len; s += 4) {
      const int t = t0 + s;
      float hp = 0.f;
      bool zero_h = true;
      if (t > 0) {
        hp = hin[h_at(b, t - 1, T, d, head, lane)];
        zero_h = false;
      } else if (h0 != nullptr) {
        hp = ld(h0 + static_cast<size_t>(b) * d + head * DH + lane);
        zero_h = false;
      }
      sh.h[wave][lane] = hp;
      __builtin_amdgcn_wave_barrier();
      const Gates g = gates_step(sh.h[wave], sh.u[wave], hp, ld(wx + wx_at(b, t, T, d, 0, head, lane)),
                                 ld(wx + wx_at(b, t, T, d, 1, head, lane)),
                                 ld(wx + wx_at(b, t, T, d, 2, head, lane)), az, ar, an, zero_h);
      sh.vec[s][0][lane] = hp;
      sh.vec[s][1][lane] = g.z;
      sh.vec[s][2][lane] = g.r;
      sh.vec[s][3][lane] = g.n;
      sh.vec[s][4][lane] = g.h_new - hin[h_at(b, t, T, d, head, lane)];
      __builtin_amdgcn_wave_barrier();
    }
  }

  // Phase B constants for this wave.
  const int li = lane & 15, lq = lane >> 4;  // MFMA lane coordinates
  const int row_a = 16 * wave + li;           // A-operand row
  float anT[2][8];                            // A_n^T[row_a][k] = A_n[k][row_a]
  bf16x8 arT[4][2];                           // B operand A_r^T[k][n] = A_r[n][k]
  float azD[4][4], anD[4][4];                 // A_z[j][i], A_n[j][i] at D positions
  const size_t hoff = static_cast<size_t>(head) * DH * DH;
#pragma unroll
  for (int ks = 0; ks < 2; ++ks)
#pragma unroll
    for (int q = 0; q < 8; ++q) anT[ks][q] = ld(a_n + hoff + (32 * ks + 8 * lq + q) * DH + row_a);
#pragma unroll
  for (int tn = 0; tn < 4; ++tn)
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int q = 0; q < 8; ++q)
        arT[tn][ks][q] = static_cast<__bf16>(ld(a_r + hoff + (16 * tn + li) * DH + 32 * ks + 8 * lq + q));
#pragma unroll
  for (int tn = 0; tn < 4; ++tn)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int i = 16 * wave + 4 * lq + v, j = 16 * tn + li;
      azD[tn][v] = ld(a_z + hoff + j * DH + i);
      anD[tn][v] = ld(a_n + hoff + j * DH + i);
    }
  // Phi = I, e = 0.
  for (int idx = threadIdx.x; idx < DH * DH; idx += 256) {
    const int n = idx / DH, k = idx % DH;
    sh.phiT[0][n][k] = static_cast<__bf16>(n == k ? 1.f : 0.f);
  }
  if (threadIdx.x < DH) sh.e[0][threadIdx.x] = 0.f;
  __syncthreads();

  floatx4 P[4];
  int cur = 0;
  for (int s = 0; s < len; ++s) {
    const float* hp = sh.vec[s][0];
    const float* z = sh.vec[s][1];
    const float* r = sh.vec[s][2];
    const float* n = sh.vec[s][3];
    // (a) M = (A_n^T diag(d5)) A_r^T, d5 = h r (1 - r).
    bf16x8 a[2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const int k = 32 * ks + 8 * lq + q;
        a[ks][q] = static_cast<__bf16>(anT[ks][q] * (hp[k] * r[k] * (1.f - r[k])));
      }
    floatx4 M[4];
#pragma unroll
    for (int tn = 0; tn < 4; ++tn) {
      M[tn] = floatx4{0.f, 0.f, 0.f, 0.f};
      M[tn] = mfma(a[0], arT[tn][0], M[tn]);
      M[tn] = mfma(a[1], arT[tn][1], M[tn]);
    }
    // (b) J = diag(d1) + diag(d2) A_z^T + diag(d3) (A_n^T diag(d4) + M) at the D
    // positions; e' = J e + F in fp32 (row sums over the 16 lanes of a row group).
    const float* ecur = sh.e[cur];
    float ev[4];
#pragma unroll
    for (int tn = 0; tn < 4; ++tn) ev[tn] = ecur[16 * tn + li];
    float esum[4];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int i = 16 * wave + 4 * lq + v;
      const float zi = z[i], ni = n[i];
      const float d1 = 1.f - zi;
      const float d2 = (ni - hp[i]) * zi * (1.f - zi);
      const float d3 = zi * (1.f - ni * ni);
      float part = 0.f;
#pragma unroll
      for (int tn = 0; tn < 4; ++tn) {
        const int j = 16 * tn + li;
        float Jv = d2 * azD[tn][v] + d3 * (anD[tn][v] * r[j] + M[tn][v]);
        if (i == j) Jv += d1;
        sh.J[i][j] = static_cast<__bf16>(Jv);
        part += Jv * ev[tn];
      }
      esum[v] = part;
    }
#pragma unroll
    for (int m = 1; m < 16; m <<= 1)
#pragma unroll
      for (int v = 0; v < 4; ++v) esum[v] += __shfl_xor(esum[v], m);
    __builtin_amdgcn_wave_barrier();
    // (c) Phi' = J Phi, rows of this wave.
    bf16x8 aj[2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) aj[ks] = *reinterpret_cast<const bf16x8*>(&sh.J[row_a][32 * ks + 8 * lq]);
#pragma unroll
    for (int tn = 0; tn < 4; ++tn) {
      P[tn] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const bf16x8 bp = *reinterpret_cast<const bf16x8*>(&sh.phiT[cur][16 * tn + li][32 * ks + 8 * lq]);
        P[tn] = mfma(aj[ks], bp, P[tn]);
      }
    }
    const int nxt = cur ^ 1;
#pragma unroll
    for (int tn = 0; tn < 4; ++tn)
#pragma unroll
      for (int v = 0; v < 4; ++v)
        sh.phiT[nxt][16 * tn + li][16 * wave + 4 * lq + v] = static_cast<__bf16>(P[tn][v]);
    if (li == 0) {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int i = 16 * wave + 4 * lq + v;
        sh.e[nxt][i] = esum[v] + sh.vec[s][4][i];
      }
    }
    __syncthreads();
    cur = nxt;
  }
  // Output the chunk transfer (fp32 accumulators of the last step).
  float* po = phi_out + static_cast<size_t>(blockIdx.x) * DH * DH;
  float* eo = e_out + static_cast<size_t>(blockIdx.x) * DH;
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int i = 16 * wave + 4 * lq + v;
#pragma unroll
    for (int tn = 0; tn < 4; ++tn) po[i * DH + 16 * tn + li] = P[tn][v];
  }
  if (threadIdx.x < DH) eo[threadIdx.x] = sh.e[cur][threadIdx.x];
}

// ---------------------------------------------------------------------------
// Carries over chunks: carry_0 = 0, carry_{c+1} = Phi_c carry_c + e_c.
// 256 threads: thread (i, part) sums 16 of row i's 64 products.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void gru_carry_kernel(const float* __restrict__ phi,
                                                       const float* __restrict__ e, int n_chunks,
                                                       float* __restrict__ carry_in) {
  __shared__ float s_c[2][DH];
  const int seq = blockIdx.x;
  const int i = threadIdx.x >> 2, part = threadIdx.x & 3;
  if (threadIdx.x < DH) s_c[0][threadIdx.x] = 0.f;
  __syncthreads();
  const float* P = phi + static_cast<size_t>(seq) * n_chunks * DH * DH;
  float4 row[4];
  auto load_row = [&](int c) {
    const float4* p = reinterpret_cast<const float4*>(P + (static_cast<size_t>(c) * DH + i) * DH + 16 * part);
#pragma unroll
    for (int q = 0; q < 4; ++q) row[q] = p[q];
  };
  load_row(0);
  int cur = 0;
  for (int c = 0; c < n_chunks; ++c) {
    float4 nrow[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) nrow[q] = row[q];
    if (c + 1 < n_chunks) load_row(c + 1);
    const float* v = s_c[cur] + 16 * part;
    float acc = 0.f;
#pragma unroll
    for (int q = 0; q < 4; ++q)
      acc += nrow[q].x * v[4 * q] + nrow[q].y * v[4 * q + 1] + nrow[q].z * v[4 * q + 2] +
             nrow[q].w * v[4 * q + 3];
    acc += __shfl_xor(acc, 1);
    acc += __shfl_xor(acc, 2);
    if (part == 0) {
      carry_in[(static_cast<size_t>(seq) * n_chunks + c) * DH + i] = s_c[cur][i];
      s_c[cur ^ 1][i] = acc + e[(static_cast<size_t>(seq) * n_chunks + c) * DH + i];
    }
    __syncthreads();
    cur ^= 1;
  }
}

// ---------------------------------------------------------------------------
// Replay: the exact fp32 recurrence of one chunk from its carry.  Each wave
// handles one chunk; lane j keeps column j of A_z, A_r, A_n in registers.
// ---------------------------------------------------------------------------
template <typename TX, typename TOUT>
__global__ __launch_bounds__(256) void gru_replay_kernel(
    const TX* __restrict__ wx, const TX* __restrict__ a_z, const TX* __restrict__ a_r,
    const TX* __restrict__ a_n, const TX* __restrict__ h0, const float* __restrict__ hin,
    const float* __restrict__ carry_in, TOUT* __restrict__ hout, int B, int T, int H,
    int n_chunks, float omega) {
  __shared__ float s_v[4][4][DH];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int task = blockIdx.x * 4 + wave;
  const int n_seq = B * H;
  if (task >= n_seq * n_chunks) return;  // whole wave exits together
  const int d = H * DH;
  const int seq = task / n_chunks, c = task % n_chunks;
  const int b = seq / H, head = seq % H;
  const int t0 = c * kChunk;
  const int len = min(kChunk, T - t0);
  float* s_h = s_v[wave][0];
  float* s_u = s_v[wave][1];
  float* s_d = s_v[wave][2];
  float* s_w = s_v[wave][3];
  float az[DH], ar[DH], an[DH];
  load_col(a_z, head, lane, az);
  load_col(a_r, head, lane, ar);
  load_col(a_n, head, lane, an);
  float dl = carry_in[static_cast<size_t>(task) * DH + lane];
  for (int s = 0; s < len; ++s) {
    const int t = t0 + s;
    float hp = 0.f;
    bool zero_h = true;
    if (t > 0) {
      hp = hin[h_at(b, t - 1, T, d, head, lane)];
      zero_h = false;
    } else if (h0 != nullptr) {
      hp = ld(h0 + static_cast<size_t>(b) * d + head * DH + lane);
      zero_h = false;
    }
    s_h[lane] = hp;
    s_d[lane] = dl;
    __builtin_amdgcn_wave_barrier();
    const Gates g = gates_step(s_h, s_u, hp, ld(wx + wx_at(b, t, T, d, 0, head, lane)),
                               ld(wx + wx_at(b, t, T, d, 1, head, lane)),
                               ld(wx + wx_at(b, t, T, d, 2, head, lane)), az, ar, an, zero_h);
    const float h_t = hin[h_at(b, t, T, d, head, lane)];
    // J delta = (1-z) delta + d2 (delta @ A_z) + d3 ((r delta + d5 (delta @ A_r)) @ A_n)
    const float yz = vec_col(s_d, az);
    const float yr = vec_col(s_d, ar);
    const float d5 = hp * g.r * (1.f - g.r);
    s_w[lane] = g.r * dl + d5 * yr;
    __builtin_amdgcn_wave_barrier();
    const float yn = vec_col(s_w, an);
    const float d2 = (g.n - hp) * g.z * (1.f - g.z);
    const float d3 = g.z * (1.f - g.n * g.n);
    dl = (1.f - g.z) * dl + d2 * yz + d3 * yn + (g.h_new - h_t);
    st(hout + h_at(b, t, T, d, head, lane), h_t + omega * dl);
    __builtin_amdgcn_wave_barrier();
  }
}

// ---------------------------------------------------------------------------
// Test hook: C = A B for 64x64 fp32 inputs through the bf16 MFMA operand
// layout used above (one block of 256 threads).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void mfma_probe_kernel(const float* A, const float* Bm, float* C) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int li = lane & 15, lq = lane >> 4;
#pragma unroll
  for (int tn = 0; tn < 4; ++tn) {
    floatx4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      bf16x8 a, bb;
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        a[q] = static_cast<__bf16>(A[(16 * wave + li) * DH + 32 * ks + 8 * lq + q]);
        bb[q] = static_cast<__bf16>(Bm[(32 * ks + 8 * lq + q) * DH + 16 * tn + li]);
      }
      acc = mfma(a, bb, acc);
    }
#pragma unroll
    for (int v = 0; v < 4; ++v) C[(16 * wave + 4 * lq + v) * DH + 16 * tn + li] = acc[v];
  }
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
struct Ws {
  float* phi;
  float* e;
  float* carry;
  float* work[2];
};

static Ws carve(void* base, int B, int T, int H, int K, size_t* total) {
  const int n_seq = B * H, n_chunks = (T + kChunk - 1) / kChunk;
  Carver cv(base);
  Ws w;
  w.phi = static_cast<float*>(cv.take(sizeof(float) * static_cast<size_t>(n_seq) * n_chunks * DH * DH));
  w.e = static_cast<float*>(cv.take(sizeof(float) * static_cast<size_t>(n_seq) * n_chunks * DH));
  w.carry = static_cast<float*>(cv.take(sizeof(float) * static_cast<size_t>(n_seq) * n_chunks * DH));
  const size_t hb = sizeof(float) * static_cast<size_t>(B) * T * H * DH;
  w.work[0] = K >= 1 ? static_cast<float*>(cv.take(hb)) : nullptr;
  w.work[1] = K >= 2 ? static_cast<float*>(cv.take(hb)) : nullptr;
  *total = cv.used;
  return w;
}

template <typename TX>
static int run(const TX* wx, const TX* az, const TX* ar, const TX* an, const TX* h0, TX* out,
               int B, int T, int H, int K, float omega, const Ws& w, hipStream_t stream) {
  const int n_seq = B * H, n_chunks = (T + kChunk - 1) / kChunk;
  const int n_blk64 = (T + 63) / 64;
  if (K == 0) {
    gru_init_kernel<TX, TX><<<dim3(n_seq * n_blk64), dim3(64), 0, stream>>>(wx, az, ar, an, h0, out,
                                                                            B, T, H);
    PRNN_HIP(hipGetLastError());
    return PRNN_OK;
  }
  gru_init_kernel<TX, float><<<dim3(n_seq * n_blk64), dim3(64), 0, stream>>>(wx, az, ar, an, h0,
                                                                            w.work[0], B, T, H);
  PRNN_HIP(hipGetLastError());
  const int replay_blocks = (n_seq * n_chunks + 3) / 4;
  for (int k = 1; k <= K; ++k) {
    const float* hin = w.work[(k - 1) & 1];
    gru_chunk_kernel<TX><<<dim3(n_seq * n_chunks), dim3(256), 0, stream>>>(
        wx, az, ar, an, h0, hin, B, T, H, n_chunks, w.phi, w.e);
    PRNN_HIP(hipGetLastError());
    gru_carry_kernel<<<dim3(n_seq), dim3(256), 0, stream>>>(w.phi, w.e, n_chunks, w.carry);
    PRNN_HIP(hipGetLastError());
    if (k == K) {
      gru_replay_kernel<TX, TX><<<dim3(replay_blocks), dim3(256), 0, stream>>>(
          wx, az, ar, an, h0, hin, w.carry, out, B, T, H, n_chunks, omega);
    } else {
      gru_replay_kernel<TX, float><<<dim3(replay_blocks), dim3(256), 0, stream>>>(
          wx, az, ar, an, h0, hin, w.carry, w.work[k & 1], B, T, H, n_chunks, omega);
    }
    PRNN_HIP(hipGetLastError());
  }
  return PRNN_OK;
}

static int check(int B, int T, int H, int dh, int K, int dtype) {
  if (B < 1 || T < 1 || H < 1)
    return fail(PRNN_ERR_VALUE, "B, T, n_heads must be >= 1, got B=%d T=%d n_heads=%d", B, T, H);
  if (dh != DH) return fail(PRNN_ERR_TYPE, "d_head must be %d, got %d", DH, dh);
  if (K < 0) return fail(PRNN_ERR_VALUE, "max_iters must be >= 0, got %d", K);
  if (dtype != PRNN_F32 && dtype != PRNN_BF16)
    return fail(PRNN_ERR_TYPE, "dtype code %d is not float32 (0) or bfloat16 (1)", dtype);
  if (static_cast<long long>(B) * H * ((T + kChunk - 1) / kChunk) > (1ll << 30))
    return fail(PRNN_ERR_VALUE, "problem too large");
  return PRNN_OK;
}

}  // namespace gru
}  // namespace prnn

using namespace prnn;

extern "C" PRNN_API size_t prnn_gru_head_newton_workspace_size(int B, int T, int n_heads,
                                                               int d_head, int max_iters,
                                                               int dtype) {
  if (gru::check(B, T, n_heads, d_head, max_iters, dtype) != PRNN_OK) return 0;
  size_t total = 0;
  gru::carve(nullptr, B, T, n_heads, max_iters, &total);
  return total;
}

extern "C" PRNN_API int prnn_gru_head_newton(const void* wx, const void* a_z, const void* a_r,
                                             const void* a_n, const void* h0, void* out, int B,
                                             int T, int n_heads, int d_head, int max_iters,
                                             float omega, int dtype, void* workspace,
                                             size_t workspace_bytes, void* stream) {
  int rc = gru::check(B, T, n_heads, d_head, max_iters, dtype);
  if (rc != PRNN_OK) return rc;
  if (!wx || !a_z || !a_r || !a_n || !out || !workspace)
    return fail(PRNN_ERR_VALUE, "wx, a_z, a_r, a_n, out and workspace must be non-null");
  size_t need = 0;
  const gru::Ws w = gru::carve(workspace, B, T, n_heads, max_iters, &need);
  if (workspace_bytes < need)
    return fail(PRNN_ERR_VALUE, "workspace too small: %zu < %zu bytes", workspace_bytes, need);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == PRNN_F32)
    return gru::run(static_cast<const float*>(wx), static_cast<const float*>(a_z),
                    static_cast<const float*>(a_r), static_cast<const float*>(a_n),
                    static_cast<const float*>(h0), static_cast<float*>(out), B, T, n_heads,
                    max_iters, omega, w, s);
  return gru::run(static_cast<const bf16*>(wx), static_cast<const bf16*>(a_z),
                  static_cast<const bf16*>(a_r), static_cast<const bf16*>(a_n),
                  static_cast<const bf16*>(h0), static_cast<bf16*>(out), B, T, n_heads,
                  max_iters, omega, w, s);
}

// Internal test hook (not part of the public header): C = A B, 64x64 fp32
// row-major, through the bf16 MFMA operand layout of the chunk kernel.
extern "C" PRNN_API int prnn_internal_mfma_probe(const float* A, const float* Bm, float* C,
                                                 void* stream) {
  gru::mfma_probe_kernel<<<dim3(1), dim3(256), 0, static_cast<hipStream_t>(stream)>>>(A, Bm, C);
  PRNN_HIP(hipGetLastError());
  return PRNN_OK;
}
