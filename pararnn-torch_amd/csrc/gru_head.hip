// ParaGRU mix='head' Newton + scan kernels for gfx950 (CDNA4).
//
// Each (batch b, head) pair is an independent 64-dimensional recurrence
// ("sequence").  One Newton iteration solves delta_t = J_t delta_{t-1} + F_t
// over T steps with J_t the dense 64x64 head Jacobian
//     J = diag(1-z) + diag((n-h) z(1-z)) A_z^T
//         + diag(z (1-n^2)) A_n^T (diag(r) + diag(h r(1-r)) A_r^T)
// (reference cells/para_gru.py:385-412, solvers/scan.py:103-123).  Time is cut
// into chunks of kChunk steps; per Newton iteration:
//
//  gru_phi_kernel     per chunk: the chunk transfer Phi = J_last ... J_first
//                     (gates of all steps by fp32 MFMA GEMMs, kept in HBM for
//                     the replays, then per step three bf16 MFMA products of
//                     the factorised J with Phi held in registers, fp32
//                     accumulation);
//  gru_replay_kernel  LOCAL: per chunk, the exact fp32 recurrence from a zero
//                     carry, giving the chunk's local solution e;
//  carry scan         carry_{c+1} = Phi_c carry_c + e_c over the chunks, fp32:
//                     group transfers (gru_group_kernel, fp32 MFMA) in
//                     parallel, a serial walk over the groups, then every
//                     group re-walked from its carry (gru_carry_kernel);
//  gru_replay_kernel  per chunk: the exact fp32 recurrence from the chunk's
//                     carry with the factorised J v (three 64-wide mat-vecs),
//                     then H += omega delta.
//
// Phi is composed from bf16-rounded operands and only multiplies the carry
// entering a chunk; e and every delta_t are fp32, so the bf16 rounding reaches
// the result only through Phi times the carry.
#include "prnn_common.h"
#include "pararnn_amd.h"
#include "prnn_host.h"

#include <algorithm>
#include <type_traits>

namespace prnn {
namespace gru {

constexpr int DH = 64;      // head width handled by these kernels
constexpr int kChunk = 32;  // time steps per chunk
constexpr int kPad = 72;    // bf16 row stride of the LDS operand tiles (16-byte aligned rows)

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

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

// Packed streams (cu_seqlens): one batch row (B = 1) of T steps holding n_seq
// sequences, sequence q on steps [cu[q], cu[q+1]); hq[t] = q at a sequence's
// first step (a head), -1 elsewhere.  A head's previous state is row tbl[q]
// of h0 (row q without a table) or zero without h0, and the Jacobian there is
// zero: no carry crosses a head (reference solvers/scan.py:206-216,
// layout.py:115-138).  The PK = false instantiations ignore it: each batch
// row is one sequence starting at t = 0 from h0 row b.
struct GPk {
  const int* cu;
  const int* hq;
  const int* tbl;
  int n_seq;
};

// Row of h0 that step t starts from, or -1 when its previous state is step
// t - 1's.
template <bool PK>
__device__ __forceinline__ int start_row(const GPk& pk, int b, int t) {
  if constexpr (PK) {
    const int q = pk.hq[t];
    return q < 0 ? -1 : (pk.tbl != nullptr ? pk.tbl[q] : q);
  } else {
    return t == 0 ? b : -1;
  }
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

// 4 consecutive values of storage type T as floats / from floats (16-bit: RNE).
template <typename T>
__device__ __forceinline__ void st4(T* p, floatx4 v) {
  if constexpr (sizeof(T) == 4) {
    *reinterpret_cast<floatx4*>(p) = v;
  } else {
    uint2 w;
    w.x = Narrow<T>::pack(v[0], v[1]);
    w.y = Narrow<T>::pack(v[2], v[3]);
    *reinterpret_cast<uint2*>(p) = w;
  }
}

template <typename T>
__device__ __forceinline__ floatx4 ld4(const T* p) {
  if constexpr (sizeof(T) == 4) {
    return *reinterpret_cast<const floatx4*>(p);
  } else {
    const uint2 w = *reinterpret_cast<const uint2*>(p);
    return floatx4{Narrow<T>::lo(w.x), Narrow<T>::hi(w.x), Narrow<T>::lo(w.y),
                   Narrow<T>::hi(w.y)};
  }
}

// Four values as loaded (fp32, or 16-bit storage packed two to a register),
// for loads issued ahead of their use: unpacking right after the load would
// wait for it there.
template <typename T>
using Raw4 = typename std::conditional<sizeof(T) == 4, floatx4, uint2>::type;
template <typename T>
__device__ __forceinline__ Raw4<T> ldr4(const T* p) {
  return *reinterpret_cast<const Raw4<T>*>(p);
}
template <typename T>
__device__ __forceinline__ floatx4 unpack4(const Raw4<T>& w) {
  if constexpr (sizeof(T) == 4) {
    return w;
  } else {
    return floatx4{Narrow<T>::lo(w.x), Narrow<T>::hi(w.x), Narrow<T>::lo(w.y),
                   Narrow<T>::hi(w.y)};
  }
}

// ---------------------------------------------------------------------------
// Initial guess: H_t = f(h_prev0_t, x_t), h_prev0 = 0 except h0 at t = 0
// (reference solvers/newton/__init__.py:925-940).  With h_prev = 0 the step is
// elementwise: gru_init_elem_kernel, 4 channels per thread; only t = 0 with
// h0 needs the mat-vecs (gru_init_kernel, one wave per sequence and block of
// `steps` steps).
// ---------------------------------------------------------------------------
template <typename TX, typename TOUT, bool PK>
__global__ __launch_bounds__(256) void gru_init_elem_kernel(const TX* __restrict__ wx,
                                                            const TX* __restrict__ h0,
                                                            TOUT* __restrict__ out, int B, int T,
                                                            int d, GPk pk) {
  const int q4 = d / 4;
  const size_t n = static_cast<size_t>(B) * T * q4;
  const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
  for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) {
    const size_t bt = i / q4;
    const int c = static_cast<int>(i % q4) * 4;
    // a first step with h0: gru_init_kernel
    if (h0 != nullptr &&
        start_row<PK>(pk, static_cast<int>(bt / T), static_cast<int>(bt % T)) >= 0)
      continue;
    const TX* row = wx + bt * 3 * d + c;
    const floatx4 zx = ld4(row), nx = ld4(row + 2 * static_cast<size_t>(d));
    floatx4 h;
#pragma unroll
    for (int v = 0; v < 4; ++v) h[v] = lerp_t(0.f, ftanh(nx[v]), fsigmoid(zx[v]));
    st4(out + bt * d + c, h);
  }
}


// PK: one block per (packed sequence q, head): the sequence's first step.
template <typename TX, typename TOUT, bool PK>
__global__ __launch_bounds__(64) void gru_init_kernel(const TX* __restrict__ wx,
                                                     const TX* __restrict__ a_z,
                                                     const TX* __restrict__ a_r,
                                                     const TX* __restrict__ a_n,
                                                     const TX* __restrict__ h0,
                                                     TOUT* __restrict__ out, int B, int T, int H,
                                                     int steps, int n_blk, GPk pk) {
  __shared__ float s_h[DH], s_u[DH];
  const int j = threadIdx.x;
  const int d = H * DH;
  const int seq = blockIdx.x / n_blk, blk = blockIdx.x % n_blk;
  const int b = PK ? 0 : seq / H, head = seq % H;
  const int t0 = PK ? pk.cu[seq / H] : blk * steps, t1 = min(T, t0 + steps);
  for (int t = t0; t < t1; ++t) {
    const float zx = ld(wx + wx_at(b, t, T, d, 0, head, j));
    const float rx = ld(wx + wx_at(b, t, T, d, 1, head, j));
    const float nx = ld(wx + wx_at(b, t, T, d, 2, head, j));
    Gates g;
    const int hr = start_row<PK>(pk, b, t);
    if (hr >= 0 && h0 != nullptr) {
      float az[DH], ar[DH], an[DH];
      load_col(a_z, head, j, az);
      load_col(a_r, head, j, ar);
      load_col(a_n, head, j, an);
      const float hp = ld(h0 + static_cast<size_t>(hr) * d + head * DH + j);
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
// Chunk transfer Phi = J_last ... J_first.  256 threads = 4 waves; wave w owns
// columns 16w..16w+15 of Phi and keeps them in registers for the whole chunk.
//
// Phase A (gates of every step of the chunk) runs as fp32 MFMA GEMMs over the
// chunk's steps: [steps x 64] h_prev times A_z, A_r, then (h_prev r) times
// A_n, each wave producing its 16 output channels; the per-step row scalars
// of J (d1 = 1-z, d2 = (n-h) z(1-z), d3 = z(1-n^2), r, d5 = h r(1-r)) go to
// LDS.
//
// Phase B: J Phi = d1 Phi + d2 (A_z^T Phi) + d3 A_n^T (r Phi + d5 (A_r^T Phi))
// (rows scaled by the d's), three bf16 MFMA products per step with fp32
// accumulation and no J formed.  The contraction index of every product is
// permuted so that the accumulator layout of Phi (lane holds rows
// 16 rt + 4 g + v of its column, g = lane / 16) is exactly the next B
// operand: Phi never leaves the wave's registers and the step loop has no
// barrier.
// ---------------------------------------------------------------------------
constexpr int kRowPad = DH + 4;  // fp32 LDS row stride of the A-operand tiles (bank spread)

// D(16x16) += A(16x4) B(4x16) in fp32: lane l holds A[l%16][l/16], B[l/16][l%16],
// D[4(l/16)+v][l%16].
__device__ __forceinline__ floatx4 mfma_f32(float a, float b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

struct PhiInputs {
  float hp[kChunk][kRowPad];  // h_prev per step
  float r[kChunk][kRowPad];   // r per step
  float x[3][kChunk][DH];     // zx, rx, nx
};
// Phase A reads the inputs; phase B reads the row scalars of J per step,
// [step][d1, d2, d3, r, d5][row], one base address per step for all of them.
union __attribute__((aligned(16))) PhiShared {
  PhiInputs in;
  float rs[kChunk][5][DH];
};
static_assert(sizeof(float) * kChunk * 5 * DH <= sizeof(PhiInputs), "row scalars alias the inputs");

// The fp32 gates z, r, n of every step go to gates_out, laid out
// [task][step][gate][64] with task = seq * n_chunks + c (the replays read
// them instead of recomputing three mat-vecs per step).  TRANS (eq. 2.6
// backward at H* = hin): Phi is stored transposed, Phi^T being the reverse
// chunk transfer.
// The bf16 A^T operands of the chunk kernel's products, in its permuted
// contraction order, packed once per call (they are the same for every chunk
// of a head): out[head][matrix z, r, n][rt][ks][lane] = the 8 values lane
// (li, g) supplies, A[k][16 rt + li] for k = 16 (2 ks + q / 4) + 4 g + q % 4.
// Also the fp32 B operands of its gate GEMMs: out_b[head][wave][matrix][kk / 4]
// [lane] = A[16 g + kk][16 wave + li] for kk = 4 (kk / 4) .. + 3.
template <typename TX>
__global__ __launch_bounds__(64) void gru_pack_at_kernel(const TX* __restrict__ a_z,
                                                         const TX* __restrict__ a_r,
                                                         const TX* __restrict__ a_n,
                                                         u32x4* __restrict__ out,
                                                         floatx4* __restrict__ out_b) {
  const int head = blockIdx.x, lane = threadIdx.x;
  const int li = lane & 15, g = lane >> 4;
  const size_t hoff = static_cast<size_t>(head) * DH * DH;
  for (int w = 0; w < 4; ++w)
#pragma unroll
    for (int m = 0; m < 3; ++m) {
      const TX* A = (m == 0 ? a_z : m == 1 ? a_r : a_n) + hoff;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        floatx4 v;
#pragma unroll
        for (int u = 0; u < 4; ++u)
          v[u] = ld(A + static_cast<size_t>(16 * g + 4 * q + u) * DH + 16 * w + li);
        out_b[((static_cast<size_t>(head) * 4 + w) * 3 + m) * 4 * 64 + q * 64 + lane] = v;
      }
    }
#pragma unroll
  for (int m = 0; m < 3; ++m) {
    const TX* A = (m == 0 ? a_z : m == 1 ? a_r : a_n) + hoff;
#pragma unroll
    for (int rt = 0; rt < 4; ++rt)
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        bf16x8 v;
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          const int k = 16 * (2 * ks + (q >> 2)) + 4 * g + (q & 3);
          v[q] = static_cast<__bf16>(ld(A + static_cast<size_t>(k) * DH + 16 * rt + li));
        }
        out[((static_cast<size_t>(head) * 3 + m) * 4 + rt) * 2 * 64 + ks * 64 + lane] =
            __builtin_bit_cast(u32x4, v);
      }
  }
}

template <typename TX, typename TH, bool TRANS, bool PK>
__global__ __launch_bounds__(256) void gru_phi_kernel(
    const TX* __restrict__ wx, const TX* __restrict__ a_z, const TX* __restrict__ a_r,
    const TX* __restrict__ a_n, const TX* __restrict__ h0, const TH* __restrict__ hin, int B,
    int T, int H, int n_chunks, float* __restrict__ phi_out, float* __restrict__ gates_out,
    const u32x4* __restrict__ at_packed, const floatx4* __restrict__ b_packed, GPk pk) {
  __shared__ PhiShared sh;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int li = lane & 15, g = lane >> 4;
  const int d = H * DH;
  const int seq = blockIdx.x / n_chunks, c = blockIdx.x % n_chunks;
  const int b = seq / H, head = seq % H;
  const int t0 = c * kChunk;
  const int len = min(kChunk, T - t0);
  const size_t hoff = static_cast<size_t>(head) * DH * DH;

  // ---- inputs of the chunk into LDS (zero rows past the end); unrolled so
  // every load of the chunk is in flight at once ----
  bool head_here = false;  // PK: a head among this thread's steps
#pragma unroll
  for (int idx = threadIdx.x; idx < kChunk * DH / 4; idx += 256) {
    const int s = idx / (DH / 4), j = 4 * (idx % (DH / 4));
    const int t = t0 + s;
    floatx4 hp = {0.f, 0.f, 0.f, 0.f}, zx = hp, rx = hp, nx = hp;
    if (s < len) {
      const int hr = start_row<PK>(pk, b, t);
      if (PK) head_here |= hr >= 0;
      if (hr < 0)
        hp = ld4(hin + h_at(b, t - 1, T, d, head, j));
      else if (h0 != nullptr)
        hp = ld4(h0 + static_cast<size_t>(hr) * d + head * DH + j);
      zx = ld4(wx + wx_at(b, t, T, d, 0, head, j));
      rx = ld4(wx + wx_at(b, t, T, d, 1, head, j));
      nx = ld4(wx + wx_at(b, t, T, d, 2, head, j));
    }
    *reinterpret_cast<floatx4*>(&sh.in.hp[s][j]) = hp;
    *reinterpret_cast<floatx4*>(&sh.in.x[0][s][j]) = zx;
    *reinterpret_cast<floatx4*>(&sh.in.x[1][s][j]) = rx;
    *reinterpret_cast<floatx4*>(&sh.in.x[2][s][j]) = nx;
  }

  // ---- phase A: gates by fp32 MFMA (wave w: output channels 16w + li) ----
  const int col = 16 * wave + li;
  floatx4 gz[2], gr[2], gn[2];
  {
    // B operands: A[k][col] for k = 16 g + kk (the contraction order every
    // lane uses for its A operand below).
    // Packed once per call by gru_pack_at_kernel: [head][wave][matrix][kk / 4][lane].
    float bz[16], br[16], bn[16];
    {
      const floatx4* pb = b_packed + (static_cast<size_t>(head) * 4 + wave) * 3 * 4 * 64 + lane;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const floatx4 z4 = pb[(0 * 4 + q) * 64], r4 = pb[(1 * 4 + q) * 64], n4 = pb[(2 * 4 + q) * 64];
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          bz[4 * q + v] = z4[v];
          br[4 * q + v] = r4[v];
          bn[4 * q + v] = n4[v];
        }
      }
    }
    __syncthreads();
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
      gz[rt] = floatx4{0.f, 0.f, 0.f, 0.f};
      gr[rt] = floatx4{0.f, 0.f, 0.f, 0.f};
      const float* hrow = &sh.in.hp[16 * rt + li][16 * g];
#pragma unroll
      for (int kk = 0; kk < 16; kk += 4) {
        const float4 a4 = *reinterpret_cast<const float4*>(hrow + kk);
        const float av[4] = {a4.x, a4.y, a4.z, a4.w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          gz[rt] = mfma_f32(av[q], bz[kk + q], gz[rt]);
          gr[rt] = mfma_f32(av[q], br[kk + q], gr[rt]);
        }
      }
    }
    // r at the D positions (step 16 rt + 4 g + v, channel col) -> LDS
#pragma unroll
    for (int rt = 0; rt < 2; ++rt)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int s = 16 * rt + 4 * g + v;
        gr[rt][v] = fsigmoid(gr[rt][v] + sh.in.x[1][s][col]);
        gz[rt][v] = fsigmoid(gz[rt][v] + sh.in.x[0][s][col]);
        sh.in.r[s][col] = gr[rt][v];
      }
    __syncthreads();
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
      gn[rt] = floatx4{0.f, 0.f, 0.f, 0.f};
      const float* hrow = &sh.in.hp[16 * rt + li][16 * g];
      const float* rrow = &sh.in.r[16 * rt + li][16 * g];
#pragma unroll
      for (int kk = 0; kk < 16; kk += 4) {
        const float4 h4 = *reinterpret_cast<const float4*>(hrow + kk);
        const float4 r4 = *reinterpret_cast<const float4*>(rrow + kk);
        const float av[4] = {h4.x * r4.x, h4.y * r4.y, h4.z * r4.z, h4.w * r4.w};
#pragma unroll
        for (int q = 0; q < 4; ++q) gn[rt] = mfma_f32(av[q], bn[kk + q], gn[rt]);
      }
    }
  }
  // Row scalars of J per step at (step, channel col).
  float rs[2][4][5];
#pragma unroll
  for (int rt = 0; rt < 2; ++rt)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int s = 16 * rt + 4 * g + v;
      const float z = gz[rt][v], r = gr[rt][v];
      const float n = ftanh(gn[rt][v] + sh.in.x[2][s][col]);
      const float hp = sh.in.hp[s][col];
      rs[rt][v][0] = 1.f - z;
      rs[rt][v][1] = (n - hp) * z * (1.f - z);
      rs[rt][v][2] = z * (1.f - n * n);
      rs[rt][v][3] = r;
      rs[rt][v][4] = hp * r * (1.f - r);
      if (s < len) {
        float* gp = gates_out + ((static_cast<size_t>(blockIdx.x) * kChunk + s) * 3) * DH + col;
        gp[0] = z;
        gp[DH] = r;
        gp[2 * DH] = n;
      }
    }
  __syncthreads();  // every read of hp / x / r above is done
#pragma unroll
  for (int rt = 0; rt < 2; ++rt)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int s = 16 * rt + 4 * g + v;
#pragma unroll
      for (int q = 0; q < 5; ++q) sh.rs[s][q][col] = rs[rt][v][q];
    }

  // ---- phase B constants: A^T operands in bf16, contraction permuted ----
  // Product X = A^T P for output row tile rt, step ks: lane (li, g) supplies
  // A^T[16 rt + li][k] = A[k][16 rt + li] for the 8 k of its slots
  // k = 16 (2 ks + q / 4) + 4 g + q % 4, q = 0..7.
  bf16x8 atz[4][2], atr[4][2], atn[4][2];
  {
    // Packed once per call by gru_pack_at_kernel: [head][matrix][rt][ks][lane].
    const u32x4* pk = at_packed + static_cast<size_t>(head) * 3 * 4 * 2 * 64 + lane;
#pragma unroll
    for (int rt = 0; rt < 4; ++rt)
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        atz[rt][ks] = __builtin_bit_cast(bf16x8, pk[((0 * 4 + rt) * 2 + ks) * 64]);
        atr[rt][ks] = __builtin_bit_cast(bf16x8, pk[((1 * 4 + rt) * 2 + ks) * 64]);
        atn[rt][ks] = __builtin_bit_cast(bf16x8, pk[((2 * 4 + rt) * 2 + ks) * 64]);
      }
  }
  __syncthreads();

  // Phi = I on this wave's columns: lane holds Phi[16 rt + 4 g + v][col].
  // PK: a chunk holding a head has Phi = 0 (the Jacobian at the head is zero).
  const bool cut = PK && __syncthreads_or(head_here);
  float P[4][4];
#pragma unroll
  for (int rt = 0; rt < 4; ++rt)
#pragma unroll
    for (int v = 0; v < 4; ++v) P[rt][v] = (!cut && 16 * rt + 4 * g + v == col) ? 1.f : 0.f;

  // B operand of a product from D-layout values: slots of step ks are rows
  // 16 (2 ks) + 4 g + (0..3) then 16 (2 ks + 1) + 4 g + (0..3).
  auto to_b = [](const float X[4][4], bf16x8 out[2]) {
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const u32x4 w = {pack_bf16x2(X[2 * ks][0], X[2 * ks][1]),
                       pack_bf16x2(X[2 * ks][2], X[2 * ks][3]),
                       pack_bf16x2(X[2 * ks + 1][0], X[2 * ks + 1][1]),
                       pack_bf16x2(X[2 * ks + 1][2], X[2 * ks + 1][3])};
      out[ks] = __builtin_bit_cast(bf16x8, w);
    }
  };
  auto product = [](const bf16x8 at[4][2], const bf16x8 bop[2], float X[4][4]) {
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) {
      floatx4 acc = {0.f, 0.f, 0.f, 0.f};
      acc = mfma(at[rt][0], bop[0], acc);
      acc = mfma(at[rt][1], bop[1], acc);
#pragma unroll
      for (int v = 0; v < 4; ++v) X[rt][v] = acc[v];
    }
  };

  // One step, in three MFMA groups of 8, each interleaved with VALU work
  // that does not wait on it (one MFMA, then the VALU that fits in its
  // execution), so the matrix pipe and the vector ALU overlap inside the wave:
  //   A_r^T P  with  Y = r P,  P <- d1 P
  //   A_z^T P  with  Y += d5 (A_r^T P), Y -> bf16
  //   A_n^T Y  with  P += d2 (A_z^T P)
  // then P += d3 (A_n^T Y) and P -> bf16 for the next step.  The sums are the
  // same fused multiply-adds in the same order as J Phi written out.
  bf16x8 bp[2];
  to_b(P, bp);
  for (int s = 0; s < (cut ? 0 : len); ++s) {
    const float* rsc = &sh.rs[s][0][4 * g];
    float rv[4][4], d1v[4][4], d2v[4][4], d3v[4][4], d5v[4][4];
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) {
      const float4 q0 = *reinterpret_cast<const float4*>(rsc + 0 * DH + 16 * rt);
      const float4 q1 = *reinterpret_cast<const float4*>(rsc + 1 * DH + 16 * rt);
      const float4 q2 = *reinterpret_cast<const float4*>(rsc + 2 * DH + 16 * rt);
      const float4 q3 = *reinterpret_cast<const float4*>(rsc + 3 * DH + 16 * rt);
      const float4 q4 = *reinterpret_cast<const float4*>(rsc + 4 * DH + 16 * rt);
      d1v[rt][0] = q0.x; d1v[rt][1] = q0.y; d1v[rt][2] = q0.z; d1v[rt][3] = q0.w;
      d2v[rt][0] = q1.x; d2v[rt][1] = q1.y; d2v[rt][2] = q1.z; d2v[rt][3] = q1.w;
      d3v[rt][0] = q2.x; d3v[rt][1] = q2.y; d3v[rt][2] = q2.z; d3v[rt][3] = q2.w;
      rv[rt][0] = q3.x; rv[rt][1] = q3.y; rv[rt][2] = q3.z; rv[rt][3] = q3.w;
      d5v[rt][0] = q4.x; d5v[rt][1] = q4.y; d5v[rt][2] = q4.z; d5v[rt][3] = q4.w;
    }
    float X[4][4], X1[4][4], X3[4][4], Y[4][4];
    product(atr, bp, X);
#pragma unroll
    for (int rt = 0; rt < 4; ++rt)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        Y[rt][v] = rv[rt][v] * P[rt][v];
        P[rt][v] = d1v[rt][v] * P[rt][v];
      }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
      __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);  // four VALU
    }
    __builtin_amdgcn_sched_barrier(0);
    product(atz, bp, X1);
#pragma unroll
    for (int rt = 0; rt < 4; ++rt)
#pragma unroll
      for (int v = 0; v < 4; ++v) Y[rt][v] = __builtin_fmaf(d5v[rt][v], X[rt][v], Y[rt][v]);
    bf16x8 by[2];
    to_b(Y, by);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);
      __builtin_amdgcn_sched_group_barrier(0x002, 3, 1);
    }
    __builtin_amdgcn_sched_barrier(0);
    product(atn, by, X3);
#pragma unroll
    for (int rt = 0; rt < 4; ++rt)
#pragma unroll
      for (int v = 0; v < 4; ++v) P[rt][v] = __builtin_fmaf(d2v[rt][v], X1[rt][v], P[rt][v]);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 2);
      __builtin_amdgcn_sched_group_barrier(0x002, 2, 2);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int rt = 0; rt < 4; ++rt)
#pragma unroll
      for (int v = 0; v < 4; ++v) P[rt][v] = __builtin_fmaf(d3v[rt][v], X3[rt][v], P[rt][v]);
    to_b(P, bp);
  }
  float* po = phi_out + static_cast<size_t>(blockIdx.x) * DH * DH;
  if (TRANS) {
#pragma unroll
    for (int rt = 0; rt < 4; ++rt)
      *reinterpret_cast<float4*>(po + col * DH + 16 * rt + 4 * g) =
          float4{P[rt][0], P[rt][1], P[rt][2], P[rt][3]};
  } else {
#pragma unroll
    for (int rt = 0; rt < 4; ++rt)
#pragma unroll
      for (int v = 0; v < 4; ++v) po[(16 * rt + 4 * g + v) * DH + col] = P[rt][v];
  }
}

// Inclusive sum over each row of 16 lanes by DPP row shifts (VALU latency, no
// LDS round trips); lane 15 of the row ends with the row's total.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, true));
}
__device__ __forceinline__ float row_sum16(float v) {
  v += dpp_f<0x111>(v);  // row_shr:1
  v += dpp_f<0x112>(v);  // row_shr:2
  v += dpp_f<0x114>(v);  // row_shr:4
  v += dpp_f<0x118>(v);  // row_shr:8
  return v;
}

// ---------------------------------------------------------------------------
// Group transfers for the two-level carry scan.  Block (seq, g) composes the
// matrices of walk steps [g group, (g + 1) group) (chunks ascending, or
// descending for REV):  Psi = S_last ... S_first  (S the stored chunk matrix,
// Phi or Phi^T) as fp32 MFMA products, and the group's carry-out from a zero
// carry,  ell <- S ell + e  (from the same LDS tile, 4 lanes per row).
// 4 waves; wave w owns the output columns 16 w .. 16 w + 15 of each product.
// ---------------------------------------------------------------------------
constexpr int kGroup = 16;    // chunks per group of the two-level carry scan
constexpr int kSPad = DH + 4;  // LDS row stride of S (A operand, bank spread)
constexpr int kMPad = DH + 16;  // LDS row stride of M (B operand, bank spread)

template <bool REV>
__global__ __launch_bounds__(256) void gru_group_kernel(const float* __restrict__ phi,
                                                       const float* __restrict__ e, int n_chunks,
                                                       float* __restrict__ psi,
                                                       float* __restrict__ ell) {
  __shared__ float sS[DH][kSPad];
  __shared__ float sM[DH][kMPad];
  __shared__ float sL[2][DH];
  const int n_groups = (n_chunks + kGroup - 1) / kGroup;
  const int seq = blockIdx.x / n_groups, grp = blockIdx.x % n_groups;
  const int w_begin = grp * kGroup, w_end = min(n_chunks, w_begin + kGroup);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int li = lane & 15, g = lane >> 4;
  const float* P = phi + static_cast<size_t>(seq) * n_chunks * DH * DH;
  const float* E = e + static_cast<size_t>(seq) * n_chunks * DH;
  auto chunk_of = [&](int w) { return REV ? n_chunks - 1 - w : w; };
  // thread t stages elements 4 t .. 4 t + 3 of rows r = (t / 16) + 16 q
  const int r0 = threadIdx.x / 16, c4 = 4 * (threadIdx.x % 16);
  // Chunk matrices are fetched kAhead products ahead into a ring of register
  // slots (the loop is unrolled over the group, so every slot index is a
  // constant): the fetch latency is many products long under load, and one
  // matrix in flight per block left the kernel latency-bound.
  constexpr int kAhead = 3;
  float4 nxt[kAhead][4];
  auto fetch = [&](int slot, int w) {
    const float* src = P + static_cast<size_t>(chunk_of(min(w, w_end - 1))) * DH * DH;
#pragma unroll
    for (int q = 0; q < 4; ++q)
      nxt[slot][q] = *reinterpret_cast<const float4*>(src + (r0 + 16 * q) * DH + c4);
  };
  // M = S_first, ell = e_first
  {
    const float* src = P + static_cast<size_t>(chunk_of(w_begin)) * DH * DH;
#pragma unroll
    for (int q = 0; q < 4; ++q)
      *reinterpret_cast<float4*>(&sM[r0 + 16 * q][c4]) =
          *reinterpret_cast<const float4*>(src + (r0 + 16 * q) * DH + c4);
  }
  if (threadIdx.x < DH) sL[0][threadIdx.x] = E[static_cast<size_t>(chunk_of(w_begin)) * DH + threadIdx.x];
  int cur = 0;
  floatx4 acc[4];
  // This lane's row of e for every chunk of the group, loaded up front: a load
  // inside the loop would make its wait (memory counters retire in order)
  // also wait for the chunk matrices fetched ahead of it.
  const int erow = 16 * wave + (lane >> 2);
  float ev[kGroup];
#pragma unroll
  for (int i = 1; i < kGroup; ++i)
    ev[i] = E[static_cast<size_t>(chunk_of(min(w_begin + i, w_end - 1))) * DH + erow];
#pragma unroll
  for (int k = 0; k < kAhead; ++k) fetch(k, w_begin + 1 + k);  // clamped past the end
  // Branch-free over the whole group: past the group's end (a short last
  // group) the product runs with S = I and e = 0, which leaves M and ell as
  // they are.
#pragma unroll
  for (int i = 1; i < kGroup; ++i) {
    const int w = w_begin + i;
    const bool past = w >= w_end;
    const int slot = (i - 1) % kAhead;
    __syncthreads();  // the previous product's reads of sS / sM are done
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int row = r0 + 16 * q;
      float4 v = nxt[slot][q];
      if (past) {
        v.x = row == c4 ? 1.f : 0.f;
        v.y = row == c4 + 1 ? 1.f : 0.f;
        v.z = row == c4 + 2 ? 1.f : 0.f;
        v.w = row == c4 + 3 ? 1.f : 0.f;
      }
      *reinterpret_cast<float4*>(&sS[row][c4]) = v;
    }
    __syncthreads();
    fetch(slot, w + kAhead);  // clamped to the group's last chunk past the end
    // keep the fetch here: it is consumed kAhead products later
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) acc[rt] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < DH / 4; ++ks) {
      const float bb = sM[4 * ks + g][16 * wave + li];
#pragma unroll
      for (int rt = 0; rt < 4; ++rt) acc[rt] = mfma_f32(sS[16 * rt + li][4 * ks + g], bb, acc[rt]);
    }
    {
      // ell <- S ell + e: row 16 wave + lane / 4, quarter lane % 4 of its terms
      const int row = 16 * wave + (lane >> 2), q0 = 16 * (lane & 3);
      float v = 0.f;
#pragma unroll
      for (int k = 0; k < 16; k += 4) {
        const float4 s4 = *reinterpret_cast<const float4*>(&sS[row][q0 + k]);
        const float4 l4 = *reinterpret_cast<const float4*>(&sL[cur][q0 + k]);
        v += s4.x * l4.x + s4.y * l4.y + s4.z * l4.z + s4.w * l4.w;
      }
      v += dpp_f<0xB1>(v);  // quad_perm [1,0,3,2]
      v += dpp_f<0x4E>(v);  // quad_perm [2,3,0,1]
      if ((lane & 3) == 0) sL[cur ^ 1][row] = v + (past ? 0.f : ev[i]);
    }
    cur ^= 1;
    __syncthreads();  // every read of sM is done
#pragma unroll
    for (int rt = 0; rt < 4; ++rt)
#pragma unroll
      for (int v = 0; v < 4; ++v) sM[16 * rt + 4 * g + v][16 * wave + li] = acc[rt][v];
  }
  __syncthreads();
  float* out = psi + static_cast<size_t>(blockIdx.x) * DH * DH;
#pragma unroll
  for (int q = 0; q < 4; ++q)
    *reinterpret_cast<float4*>(out + (r0 + 16 * q) * DH + c4) =
        *reinterpret_cast<const float4*>(&sM[r0 + 16 * q][c4]);
  if (threadIdx.x < DH) ell[static_cast<size_t>(blockIdx.x) * DH + threadIdx.x] = sL[cur][threadIdx.x];
}

// ---------------------------------------------------------------------------
// Carries over chunks: carry_0 = 0, carry_{c+1} = Phi_c carry_c + e_c.
// REV (eq. 2.6 backward, phi holding Phi^T): chunks from the last one down,
// carry_{n-1} = 0, carry_{c-1} = Phi_c^T carry_c + e_c.
// 64 PARTS threads: thread (i, part) sums 64 / PARTS of row i's products
// (PARTS = 16 for a single long chain per block, more loads in flight;
// PARTS = 4 for many short chains, a 4-wave barrier per step).
// ---------------------------------------------------------------------------
template <int PARTS>
__device__ __forceinline__ float parts_sum(float v) {
  if constexpr (PARTS == 16) {
    return row_sum16(v);  // the 16 threads of a row are one DPP row; lane 15 holds the sum
  } else {
    static_assert(PARTS == 4, "4 or 16 threads per row");
    v += dpp_f<0xB1>(v);  // quad_perm [1,0,3,2]
    v += dpp_f<0x4E>(v);  // quad_perm [2,3,0,1]: every lane of the quad holds the sum
    return v;
  }
}

template <bool REV, int PARTS>
__global__ __launch_bounds__(64 * PARTS) void gru_carry_kernel(
    const float* __restrict__ phi, const float* __restrict__ e, int n_chunks, int group,
    const float* __restrict__ init, float* __restrict__ carry_in) {
  // The chain is serial over chunks, so each step costs the latency of its
  // 16 KB of Phi and its e.  Thread (i, part) holds NQ float4 of row i; the
  // chunks are fetched a block of kB ahead into one of two register blocks
  // (written out by hand, no dynamic register indexing) while the other block
  // is walked, and a block's carries are stored after its kB steps.
  // Block (seq, g) walks steps [g group, (g + 1) group) of the walk order
  // (chunks ascending, or descending for REV) from init[seq, g] (zeros when
  // init is NULL).
  constexpr int NQ = DH / PARTS / 4;  // float4 per thread and row
  constexpr int kB = PARTS == 16 ? 8 : 4;
  __shared__ float s_c[2][DH];
  const int n_groups = (n_chunks + group - 1) / group;
  const int seq = blockIdx.x / n_groups, grp = blockIdx.x % n_groups;
  const int w_begin = grp * group, w_end = min(n_chunks, w_begin + group);
  const int i = threadIdx.x / PARTS, part = threadIdx.x % PARTS;
  if (threadIdx.x < DH)
    s_c[0][threadIdx.x] = init != nullptr ? init[static_cast<size_t>(blockIdx.x) * DH + threadIdx.x] : 0.f;
  __syncthreads();
  const float* P = phi + static_cast<size_t>(seq) * n_chunks * DH * DH;
  const float* E = e + static_cast<size_t>(seq) * n_chunks * DH;
  // Steps past the group's end re-read its last chunk (no branch around the
  // loads) and write nothing.
  auto chunk_of = [&](int step) {
    const int k = min(step, w_end - 1);
    return REV ? n_chunks - 1 - k : k;
  };
  auto fetch = [&](int step0, float4 rows[kB][NQ], float ev[kB]) {
#pragma unroll
    for (int k = 0; k < kB; ++k) {
      const int c = chunk_of(step0 + k);
      const float* row = P + (static_cast<size_t>(c) * DH + i) * DH + 4 * NQ * part;
#pragma unroll
      for (int q = 0; q < NQ; ++q) rows[k][q] = *reinterpret_cast<const float4*>(row + 4 * q);
      ev[k] = E[static_cast<size_t>(c) * DH + i];
    }
  };
  int cur = 0;
  auto walk = [&](int step0, const float4 rows[kB][NQ], const float ev[kB]) {
    float out[kB];
#pragma unroll
    for (int k = 0; k < kB; ++k) {
      float acc = 0.f;
#pragma unroll
      for (int q = 0; q < NQ; ++q) {
        const float4 v = *reinterpret_cast<const float4*>(s_c[cur] + 4 * NQ * part + 4 * q);
        acc += rows[k][q].x * v.x + rows[k][q].y * v.y + rows[k][q].z * v.z + rows[k][q].w * v.w;
      }
      acc = parts_sum<PARTS>(acc);
      out[k] = s_c[cur][i];
      if (part == PARTS - 1) s_c[cur ^ 1][i] = acc + ev[k];
      __syncthreads();
      cur ^= 1;
    }
    if (part == PARTS - 1) {
#pragma unroll
      for (int k = 0; k < kB; ++k)
        if (step0 + k < w_end)
          carry_in[(static_cast<size_t>(seq) * n_chunks + chunk_of(step0 + k)) * DH + i] = out[k];
    }
  };
  float4 ra[kB][NQ], rb[kB][NQ];
  float ea[kB], eb[kB];
  fetch(w_begin, ra, ea);
  for (int step0 = w_begin; step0 < w_end; step0 += 2 * kB) {
    fetch(step0 + kB, rb, eb);
    walk(step0, ra, ea);
    fetch(step0 + 2 * kB, ra, ea);
    walk(step0 + kB, rb, eb);
  }
}

// ---------------------------------------------------------------------------
// Replay: the exact fp32 recurrence of a chunk from its carry.  Each wave
// walks kPair consecutive chunks of one sequence side by side (the two serial
// chains hide each other's latency); lane j keeps column j of A_z, A_r, A_n
// in registers, shared by the chunks, and reads the step's gates (written by
// the chunk kernel from the same guess).  LOCAL: from a zero carry, writing
// only each chunk's final delta (the local solution e of the carry scan);
// otherwise from the chunk's carry, writing H + omega delta.
// ---------------------------------------------------------------------------
constexpr int kPair = 2;
constexpr int kSimds = 1024;  // 256 CUs x 4 SIMDs

template <typename TX, typename TOUT, bool LOCAL, bool PK, int NP>
__global__ __launch_bounds__(256) void gru_replay_kernel(
    const TX* __restrict__ a_z, const TX* __restrict__ a_r, const TX* __restrict__ a_n,
    const TX* __restrict__ h0, const float* __restrict__ hin, const float* __restrict__ gates,
    const float* __restrict__ carry_in, TOUT* __restrict__ hout, float* __restrict__ e_out,
    int B, int T, int H, int n_chunks, float omega, GPk pk) {
  __shared__ float s_v[4][NP][2][DH];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n_pairs = (n_chunks + NP - 1) / NP;
  const int task = blockIdx.x * 4 + wave;
  const int n_seq = B * H;
  if (task >= n_seq * n_pairs) return;  // whole wave exits together
  const int d = H * DH;
  const int seq = task / n_pairs, c0 = (task % n_pairs) * NP;
  const int b = seq / H, head = seq % H;
  float az[DH], ar[DH], an[DH];
  load_col(a_z, head, lane, az);
  load_col(a_r, head, lane, ar);
  load_col(a_n, head, lane, an);

  struct In {
    float hp, z, r, n, ht;
    bool head;  // PK: a sequence's first step (no carry reaches it)
  };
  int t0[NP], len[NP];
  float dl[NP];
  const float* gt[NP];
#pragma unroll
  for (int k = 0; k < NP; ++k) {
    const int c = c0 + k;
    const bool valid = c < n_chunks;
    t0[k] = c * kChunk;
    len[k] = valid ? min(kChunk, T - t0[k]) : 0;
    const size_t id = static_cast<size_t>(seq) * n_chunks + (valid ? c : c0);
    dl[k] = (LOCAL || !valid) ? 0.f : carry_in[id * DH + lane];
    gt[k] = gates + id * kChunk * 3 * DH + lane;
  }
  auto load_in = [&](int k, int s) {
    In v{0.f, 0.f, 0.f, 0.f, 0.f, false};
    if (s < len[k]) {
      const int t = t0[k] + s;
      const int hr = start_row<PK>(pk, b, t);
      v.head = PK && hr >= 0;
      if (hr < 0)
        v.hp = hin[h_at(b, t - 1, T, d, head, lane)];
      else if (h0 != nullptr)
        v.hp = ld(h0 + static_cast<size_t>(hr) * d + head * DH + lane);
      v.z = gt[k][(s * 3) * DH];
      v.r = gt[k][(s * 3 + 1) * DH];
      v.n = gt[k][(s * 3 + 2) * DH];
      v.ht = hin[h_at(b, t, T, d, head, lane)];
    }
    return v;
  };
  // Chunk 0 of the pair is the longest (only a sequence's last chunk is short).
  for (int s = 0; s < len[0]; ++s) {
    In cur[NP];
#pragma unroll
    for (int k = 0; k < NP; ++k) cur[k] = load_in(k, s);
    // J delta = (1-z) delta + d2 (delta @ A_z) + d3 ((r delta + d5 (delta @ A_r)) @ A_n)
    if constexpr (PK) {
#pragma unroll
      for (int k = 0; k < NP; ++k)
        if (cur[k].head) dl[k] = 0.f;  // no carry crosses a head
    }
#pragma unroll
    for (int k = 0; k < NP; ++k) s_v[wave][k][0][lane] = dl[k];
    __builtin_amdgcn_wave_barrier();
    float yz[NP], yr[NP], yn[NP];
#pragma unroll
    for (int k = 0; k < NP; ++k) {
      yz[k] = vec_col(s_v[wave][k][0], az);
      yr[k] = vec_col(s_v[wave][k][0], ar);
    }
#pragma unroll
    for (int k = 0; k < NP; ++k) {
      const float d5 = cur[k].hp * cur[k].r * (1.f - cur[k].r);
      s_v[wave][k][1][lane] = cur[k].r * dl[k] + d5 * yr[k];
    }
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int k = 0; k < NP; ++k) yn[k] = vec_col(s_v[wave][k][1], an);
#pragma unroll
    for (int k = 0; k < NP; ++k) {
      const In& v = cur[k];
      const float d2 = (v.n - v.hp) * v.z * (1.f - v.z);
      const float d3 = v.z * (1.f - v.n * v.n);
      const float h_new = lerp_t(v.hp, v.n, v.z);
      dl[k] = (1.f - v.z) * dl[k] + d2 * yz[k] + d3 * yn[k] + (h_new - v.ht);
      if (!LOCAL && s < len[k])
        st(hout + h_at(b, t0[k] + s, T, d, head, lane), v.ht + omega * dl[k]);
    }
    __builtin_amdgcn_wave_barrier();
  }
  if (LOCAL) {
#pragma unroll
    for (int k = 0; k < NP; ++k)
      if (len[k] > 0) e_out[(static_cast<size_t>(seq) * n_chunks + c0 + k) * DH + lane] = dl[k];
  }
}

// ---------------------------------------------------------------------------
// Replay on the matrix cores.  The chunks of one sequence share A_z, A_r,
// A_n, so a step of 16 chunks side by side is three 64x64 by 64x16 fp32
// products: wave w of a block takes chunks c = 16 (4 grp + w) + n, lane
// (n, g) = (l % 16, l / 16) holding rows 16 T + 4 g + v (T, v = 0..3) of
// chunk n's delta, which is the fp32 MFMA accumulator layout.  With the
// contraction index permuted (MFMA (Tc, v) contracts over rows
// 16 Tc + 4 g + v), that accumulator is directly the B operand of the next
// product, so delta never leaves the registers; the matching A operands,
// A[16 Tc + 4 (l / 16) + v][16 To + l % 16], are staged once per block in
// LDS.  Same recurrence, gates and outputs as gru_replay_kernel; the
// 64-term sums are accumulated in the MFMA's order (fp32 products and sums).
// A chunk past the end of the sequence is a zero column: columns of an
// MFMA product do not mix.
// ---------------------------------------------------------------------------
constexpr int kRCols = 16;  // chunks per wave (the MFMA N dimension)

template <typename TX, typename TOUT, bool LOCAL, bool PK>
__global__ __launch_bounds__(256) void gru_replay_mfma_kernel(
    const TX* __restrict__ a_z, const TX* __restrict__ a_r, const TX* __restrict__ a_n,
    const TX* __restrict__ h0, const float* __restrict__ hin, const float* __restrict__ gates,
    const float* __restrict__ carry_in, TOUT* __restrict__ hout, float* __restrict__ e_out,
    int B, int T, int H, int n_chunks, float omega, GPk pk) {
  // [matrix][output tile][contraction tile][lane] -> the 4 A operands v = 0..3
  __shared__ floatx4 sA[3][4][4][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n_grp = (n_chunks + 4 * kRCols - 1) / (4 * kRCols);
  const int seq = blockIdx.x / n_grp, grp = blockIdx.x % n_grp;
  const int b = seq / H, head = seq % H;
  const int d = H * DH;
  for (int e = threadIdx.x; e < 3 * 4 * 4 * 64; e += 256) {
    const int l = e & 63, tc = (e >> 6) & 3, to = (e >> 8) & 3, m = e >> 10;
    const TX* A = (m == 0 ? a_z : m == 1 ? a_r : a_n) + static_cast<size_t>(head) * DH * DH;
    floatx4 v;
#pragma unroll
    for (int q = 0; q < 4; ++q) v[q] = ld(A + (16 * tc + 4 * (l >> 4) + q) * DH + 16 * to + (l & 15));
    sA[m][to][tc][l] = v;
  }
  __syncthreads();
  const int c_first = (grp * 4 + wave) * kRCols;
  if (c_first >= n_chunks) return;  // whole wave exits together (no barrier follows)
  const int n = lane & 15, g = lane >> 4;
  const int c = c_first + n;
  const bool valid = c < n_chunks;
  const int t0 = c * kChunk;
  const int len = valid ? min(kChunk, T - t0) : 0;
  const size_t id = static_cast<size_t>(seq) * n_chunks + (valid ? c : c_first);
  const float* gt = gates + id * kChunk * 3 * DH + 4 * g;
  floatx4 dl[4];
#pragma unroll
  for (int to = 0; to < 4; ++to) {
    dl[to] = floatx4{0.f, 0.f, 0.f, 0.f};
    if (!LOCAL && valid) dl[to] = *reinterpret_cast<const floatx4*>(carry_in + id * DH + 16 * to + 4 * g);
  }
  const int steps = min(kChunk, T - c_first * kChunk);  // the wave's longest chunk
  struct In {
    floatx4 ht[4], gz[4], gr[4], gn[4];
    int hr;  // PK: the h0 row of the sequence this lane's chunk starts at this step, else -1
  };
  // Step s's inputs (zeros past the chunk's end); loaded one step ahead.
  auto load_in = [&](int s, In& v) {
    const bool act = s < len;
    const int t = t0 + s;
    v.hr = -1;
    if constexpr (PK) v.hr = act ? start_row<PK>(pk, b, t) : -1;
#pragma unroll
    for (int to = 0; to < 4; ++to) {
      const floatx4 zero{0.f, 0.f, 0.f, 0.f};
      v.ht[to] = v.gz[to] = v.gr[to] = v.gn[to] = zero;
      if (act) {
        v.ht[to] = *reinterpret_cast<const floatx4*>(hin + h_at(b, t, T, d, head, 16 * to + 4 * g));
        v.gz[to] = *reinterpret_cast<const floatx4*>(gt + (s * 3) * DH + 16 * to);
        v.gr[to] = *reinterpret_cast<const floatx4*>(gt + (s * 3 + 1) * DH + 16 * to);
        v.gn[to] = *reinterpret_cast<const floatx4*>(gt + (s * 3 + 2) * DH + 16 * to);
      }
    }
  };
  // h at t - 1 of the current step: the previous step's h at t, except at the
  // chunk's first step (below) and at a head (its sequence's h0 row, loaded
  // where it is used).  One copy of it rather than one per prefetched step
  // keeps the kernel at two waves per SIMD.
  floatx4 hprev[4];
#pragma unroll
  for (int to = 0; to < 4; ++to) {
    const int j = 16 * to + 4 * g;
    hprev[to] = floatx4{0.f, 0.f, 0.f, 0.f};
    if (len > 0) {
      if (t0 > 0)
        hprev[to] = *reinterpret_cast<const floatx4*>(hin + h_at(b, t0 - 1, T, d, head, j));
      else if (!PK && h0 != nullptr)
        hprev[to] = ld4(h0 + static_cast<size_t>(b) * d + head * DH + j);
    }
  }
  In nx;
  load_in(0, nx);
  for (int s = 0; s < steps; ++s) {
    const bool act = s < len;
    const int t = t0 + s;
    const In cur = nx;
    if (s + 1 < steps) load_in(s + 1, nx);
    floatx4 hpv[4];
#pragma unroll
    for (int to = 0; to < 4; ++to) hpv[to] = hprev[to];
    if constexpr (PK) {
      if (cur.hr >= 0) {
#pragma unroll
        for (int to = 0; to < 4; ++to) {
          hpv[to] = floatx4{0.f, 0.f, 0.f, 0.f};
          if (h0 != nullptr)
            hpv[to] = ld4(h0 + static_cast<size_t>(cur.hr) * d + head * DH + 16 * to + 4 * g);
        }
      }
    }
    const floatx4 *hp = hpv, *ht = cur.ht, *gz = cur.gz, *gr = cur.gr, *gn = cur.gn;
    if constexpr (PK) {
      // no carry crosses a head: this lane's column of delta restarts at zero
      if (cur.hr >= 0) {
#pragma unroll
        for (int to = 0; to < 4; ++to) dl[to] = floatx4{0.f, 0.f, 0.f, 0.f};
      }
    }
    // J delta = (1-z) delta + d2 (delta @ A_z) + d3 ((r delta + d5 (delta @ A_r)) @ A_n)
    floatx4 yz[4], yr[4], yn[4], vv[4];
#pragma unroll
    for (int to = 0; to < 4; ++to) yz[to] = yr[to] = yn[to] = floatx4{0.f, 0.f, 0.f, 0.f};
    // Eight independent accumulators between dependent MFMAs.
#pragma unroll
    for (int tc = 0; tc < 4; ++tc) {
      floatx4 az[4], ar[4];
#pragma unroll
      for (int to = 0; to < 4; ++to) {
        az[to] = sA[0][to][tc][lane];
        ar[to] = sA[1][to][tc][lane];
      }
#pragma unroll
      for (int v = 0; v < 4; ++v) {
#pragma unroll
        for (int to = 0; to < 4; ++to) {
          yz[to] = mfma_f32(az[to][v], dl[tc][v], yz[to]);
          yr[to] = mfma_f32(ar[to][v], dl[tc][v], yr[to]);
        }
        __builtin_amdgcn_sched_barrier(0);  // keep the rounds interleaved
      }
    }
#pragma unroll
    for (int to = 0; to < 4; ++to)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const float r = gr[to][v];
        const float d5 = hp[to][v] * r * (1.f - r);
        vv[to][v] = r * dl[to][v] + d5 * yr[to][v];
      }
#pragma unroll
    for (int tc = 0; tc < 4; ++tc) {
      floatx4 an[4];
#pragma unroll
      for (int to = 0; to < 4; ++to) an[to] = sA[2][to][tc][lane];
#pragma unroll
      for (int v = 0; v < 4; ++v) {
#pragma unroll
        for (int to = 0; to < 4; ++to) yn[to] = mfma_f32(an[to][v], vv[tc][v], yn[to]);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    if (act) {
#pragma unroll
      for (int to = 0; to < 4; ++to) {
        floatx4 o;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const float z = gz[to][v], nv = gn[to][v], h = hp[to][v];
          const float d2 = (nv - h) * z * (1.f - z);
          const float d3 = z * (1.f - nv * nv);
          const float h_new = lerp_t(h, nv, z);
          dl[to][v] = (1.f - z) * dl[to][v] + d2 * yz[to][v] + d3 * yn[to][v] + (h_new - ht[to][v]);
          o[v] = ht[to][v] + omega * dl[to][v];
        }
        if (!LOCAL) st4(hout + h_at(b, t, T, d, head, 16 * to + 4 * g), o);
      }
    }
#pragma unroll
    for (int to = 0; to < 4; ++to) hprev[to] = cur.ht[to];
  }
  if (LOCAL && valid) {
#pragma unroll
    for (int to = 0; to < 4; ++to)
      *reinterpret_cast<floatx4*>(e_out + id * DH + 16 * to + 4 * g) = dl[to];
  }
}

// ===========================================================================
// Eq. 2.6 backward at the solved trajectory H* (reference
// solvers/newton/__init__.py:765-866 with the head Jacobian, kernels/
// gru_head_factor.py:68-112 for J^T mu, kernels/vjp_gru.py:141-224 for the
// cell VJP).  With nu_t = J_t^T mu_t the adjoint recursion
//     mu_t = g_t + J_{t+1}^T mu_{t+1}   becomes   nu_t = J_t^T (g_t + nu_{t+1}),
// nu_T = 0, mu_t = g_t + nu_{t+1} and grad h0 = nu_0.  Over chunk c
// (steps t0..t1-1) nu_{t0} = Phi_c^T nu_{t1} + e_c, with Phi_c the forward
// chunk transfer J_{t1-1} ... J_{t0}: the same chunk kernel, stored
// transposed, and the carry kernel run from the last chunk down.
//
//  gru_phi_kernel<BWD>   Phi_c^T and the fp32 gates z, r, n of every step;
//  gru_rev_local_kernel  per chunk, nu from a zero carry -> e_c;
//  gru_carry_kernel<REV> nu entering each chunk from the right;
//  gru_rev_kernel        per chunk from its carry: mu_t, the pre-activation
//                        gradients (g_wx) and, for chunk 0, grad h0 = nu_0;
//  gru_ga_kernel         per (split of the B T rows, head): the partial sums
//                        of the outer products X^T D of all three gates by
//                        fp32 MFMA (X = h_prev for z, r; h_prev r for n);
//  gru_ga_reduce_kernel  fixed-order sum of the splits (deterministic).
// ===========================================================================

// Row i of a head's (in, out) matrix, i.e. A[i][o] for o = 0..63.
template <typename TX>
__device__ __forceinline__ void load_row(const TX* A, int head, int i, float row[DH]) {
  const TX* p = A + static_cast<size_t>(head) * DH * DH + static_cast<size_t>(i) * DH;
#pragma unroll
  for (int o = 0; o < DH; ++o) row[o] = ld(p + o);
}

// Reverse walk of one chunk per wave from its carry; lane i keeps row i of
// A_z, A_r, A_n.
// Per step: mu = g + nu;  d_zpre = mu (n - h) z(1-z);  d_npre = mu z (1-n^2);
// d_u = A_n d_npre;  d_rpre = d_u h r(1-r);
// nu <- (1-z) mu + A_z d_zpre + r d_u + A_r d_rpre.
// PK: at a head nu is that sequence's grad h0 (row q of g_h0), and nothing
// flows to the step before it.
template <typename TX, bool PK>
__global__ __launch_bounds__(256) void gru_rev_kernel(
    const TX* __restrict__ a_z, const TX* __restrict__ a_r, const TX* __restrict__ a_n,
    const TX* __restrict__ h0, const TX* __restrict__ states, const TX* __restrict__ grad,
    const float* __restrict__ gates, const float* __restrict__ carry_in, TX* __restrict__ g_wx,
    float* __restrict__ g_h0, int B, int T, int H, int n_chunks, GPk pk) {
  __shared__ float s_v[4][3][DH];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int task = blockIdx.x * 4 + wave;
  if (task >= B * H * n_chunks) return;  // whole wave exits together
  const int d = H * DH;
  const int seq = task / n_chunks, c = task % n_chunks;
  const int b = seq / H, head = seq % H;
  const int t0 = c * kChunk;
  const int len = min(kChunk, T - t0);
  float* s_a = s_v[wave][0];
  float* s_b = s_v[wave][1];
  float* s_c = s_v[wave][2];
  float az[DH], ar[DH], an[DH];
  load_row(a_z, head, lane, az);
  load_row(a_r, head, lane, ar);
  load_row(a_n, head, lane, an);
  float nu = carry_in[static_cast<size_t>(task) * DH + lane];

  struct In {
    float hp, g, z, r, n;
    int q;  // PK: the sequence this step starts, -1 elsewhere
  };
  const float* gt = gates + static_cast<size_t>(task) * kChunk * 3 * DH + lane;
  auto load_in = [&](int s) {
    In v{0.f, 0.f, 0.f, 0.f, 0.f, -1};
    if (s >= 0) {
      const int t = t0 + s;
      const int hr = start_row<PK>(pk, b, t);
      if (PK && hr >= 0) v.q = pk.hq[t];
      if (hr < 0)
        v.hp = ld(states + h_at(b, t - 1, T, d, head, lane));
      else if (h0 != nullptr)
        v.hp = ld(h0 + static_cast<size_t>(hr) * d + head * DH + lane);
      v.g = ld(grad + h_at(b, t, T, d, head, lane));
      v.z = gt[(s * 3) * DH];
      v.r = gt[(s * 3 + 1) * DH];
      v.n = gt[(s * 3 + 2) * DH];
    }
    return v;
  };
  In cur = load_in(len - 1), nx1 = load_in(len - 2);
  for (int s = len - 1; s >= 0; --s) {
    const In nx2 = load_in(s - 2);
    const float mu = cur.g + nu;
    const float zp = cur.z * (1.f - cur.z);
    const float d_zpre = mu * (cur.n - cur.hp) * zp;
    const float d_npre = mu * cur.z * (1.f - cur.n * cur.n);
    s_a[lane] = d_zpre;
    s_b[lane] = d_npre;
    __builtin_amdgcn_wave_barrier();
    const float t_z = vec_col(s_a, az);
    const float d_u = vec_col(s_b, an);
    const float d_rpre = d_u * cur.hp * cur.r * (1.f - cur.r);
    s_c[lane] = d_rpre;
    __builtin_amdgcn_wave_barrier();
    const float t_r = vec_col(s_c, ar);
    nu = (1.f - cur.z) * mu + t_z + cur.r * d_u + t_r;
    {
      const int t = t0 + s;
      st(g_wx + wx_at(b, t, T, d, 0, head, lane), d_zpre);
      st(g_wx + wx_at(b, t, T, d, 1, head, lane), d_rpre);
      st(g_wx + wx_at(b, t, T, d, 2, head, lane), d_npre);
    }
    if (PK && cur.q >= 0) {
      if (g_h0 != nullptr) g_h0[static_cast<size_t>(cur.q) * d + head * DH + lane] = nu;
      nu = 0.f;
    }
    __builtin_amdgcn_wave_barrier();
    cur = nx1;
    nx1 = nx2;
  }
  if (!PK && c == 0 && g_h0 != nullptr)
    g_h0[static_cast<size_t>(b) * d + head * DH + lane] = nu;
}

// Local reverse walk: nu from a zero carry over each chunk, NP consecutive
// chunks of a sequence per wave side by side (lane i keeps row i of A_z, A_r,
// A_n); the chunk's final nu is its local solution e.
template <typename TX, bool PK, int NP>
__global__ __launch_bounds__(256) void gru_rev_local_kernel(
    const TX* __restrict__ a_z, const TX* __restrict__ a_r, const TX* __restrict__ a_n,
    const TX* __restrict__ h0, const TX* __restrict__ states, const TX* __restrict__ grad,
    const float* __restrict__ gates, float* __restrict__ e_out, int B, int T, int H,
    int n_chunks, GPk pk) {
  __shared__ float s_v[4][NP][3][DH];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n_pairs = (n_chunks + NP - 1) / NP;
  const int task = blockIdx.x * 4 + wave;
  if (task >= B * H * n_pairs) return;  // whole wave exits together
  const int d = H * DH;
  const int seq = task / n_pairs, c0 = (task % n_pairs) * NP;
  const int b = seq / H, head = seq % H;
  float az[DH], ar[DH], an[DH];
  load_row(a_z, head, lane, az);
  load_row(a_r, head, lane, ar);
  load_row(a_n, head, lane, an);

  struct In {
    float hp, g, z, r, n;
    bool head;  // PK: a sequence's first step (nothing flows before it)
  };
  int t0[NP], len[NP];
  float nu[NP];
  const float* gt[NP];
#pragma unroll
  for (int k = 0; k < NP; ++k) {
    const int c = c0 + k;
    const bool valid = c < n_chunks;
    t0[k] = c * kChunk;
    len[k] = valid ? min(kChunk, T - t0[k]) : 0;
    const size_t id = static_cast<size_t>(seq) * n_chunks + (valid ? c : c0);
    nu[k] = 0.f;
    gt[k] = gates + id * kChunk * 3 * DH + lane;
  }
  // Steps past a chunk's end read zeros, and a zero step leaves nu unchanged.
  auto load_in = [&](int k, int s) {
    In v{0.f, 0.f, 0.f, 0.f, 0.f, false};
    if (s < len[k]) {
      const int t = t0[k] + s;
      const int hr = start_row<PK>(pk, b, t);
      v.head = PK && hr >= 0;
      if (hr < 0)
        v.hp = ld(states + h_at(b, t - 1, T, d, head, lane));
      else if (h0 != nullptr)
        v.hp = ld(h0 + static_cast<size_t>(hr) * d + head * DH + lane);
      v.g = ld(grad + h_at(b, t, T, d, head, lane));
      v.z = gt[k][(s * 3) * DH];
      v.r = gt[k][(s * 3 + 1) * DH];
      v.n = gt[k][(s * 3 + 2) * DH];
    }
    return v;
  };
  // Chunk 0 of the pair is the longest (only a sequence's last chunk is short).
  for (int s = len[0] - 1; s >= 0; --s) {
    In cur[NP];
#pragma unroll
    for (int k = 0; k < NP; ++k) cur[k] = load_in(k, s);
    float mu[NP], d_zpre[NP], d_npre[NP], d_u[NP], t_z[NP], d_rpre[NP];
#pragma unroll
    for (int k = 0; k < NP; ++k) {
      const In& v = cur[k];
      mu[k] = v.g + nu[k];
      d_zpre[k] = mu[k] * (v.n - v.hp) * (v.z * (1.f - v.z));
      d_npre[k] = mu[k] * v.z * (1.f - v.n * v.n);
      s_v[wave][k][0][lane] = d_zpre[k];
      s_v[wave][k][1][lane] = d_npre[k];
    }
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int k = 0; k < NP; ++k) {
      t_z[k] = vec_col(s_v[wave][k][0], az);
      d_u[k] = vec_col(s_v[wave][k][1], an);
      d_rpre[k] = d_u[k] * cur[k].hp * cur[k].r * (1.f - cur[k].r);
      s_v[wave][k][2][lane] = d_rpre[k];
    }
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int k = 0; k < NP; ++k) {
      const float t_r = vec_col(s_v[wave][k][2], ar);
      nu[k] = (1.f - cur[k].z) * mu[k] + t_z[k] + cur[k].r * d_u[k] + t_r;
      if (PK && cur[k].head) nu[k] = 0.f;  // nothing flows before a head
    }
    __builtin_amdgcn_wave_barrier();
  }
#pragma unroll
  for (int k = 0; k < NP; ++k)
    if (len[k] > 0) e_out[(static_cast<size_t>(seq) * n_chunks + c0 + k) * DH + lane] = nu[k];
}

// Reverse walks on the matrix cores: 16 chunks of a sequence per wave, as in
// gru_replay_mfma_kernel, with the products A_z D_z, A_n D_n and A_r D_r (rows
// of the untransposed matrices: A operand A[16 To + l % 16][16 Tc + 4 (l / 16)
// + v]).  Columns step from the chunk's end down; a chunk shorter than the
// wave's longest reads zeros on the steps past its end, which leave nu
// unchanged.  LOCAL: nu from zero, writing each chunk's final nu (e);
// otherwise from the chunk's carry, writing the pre-activation gradients
// g_wx and, for chunk 0, grad h0 = nu_0.
// PK: at a head (per column) nu is that sequence's grad h0 (written by the
// final walk) and restarts at zero for the steps before it.
template <typename TX, bool LOCAL, bool PK>
__global__ __launch_bounds__(256) void gru_rev_mfma_kernel(
    const TX* __restrict__ a_z, const TX* __restrict__ a_r, const TX* __restrict__ a_n,
    const TX* __restrict__ h0, const TX* __restrict__ states, const TX* __restrict__ grad,
    const float* __restrict__ gates, const float* __restrict__ carry_in, TX* __restrict__ g_wx,
    float* __restrict__ g_h0, float* __restrict__ e_out, int B, int T, int H, int n_chunks,
    GPk pk) {
  __shared__ floatx4 sA[3][4][4][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n_grp = (n_chunks + 4 * kRCols - 1) / (4 * kRCols);
  const int seq = blockIdx.x / n_grp, grp = blockIdx.x % n_grp;
  const int b = seq / H, head = seq % H;
  const int d = H * DH;
  for (int e = threadIdx.x; e < 3 * 4 * 4 * 64; e += 256) {
    const int l = e & 63, tc = (e >> 6) & 3, to = (e >> 8) & 3, m = e >> 10;
    const TX* A = (m == 0 ? a_z : m == 1 ? a_r : a_n) + static_cast<size_t>(head) * DH * DH;
    floatx4 v;
#pragma unroll
    for (int q = 0; q < 4; ++q) v[q] = ld(A + (16 * to + (l & 15)) * DH + 16 * tc + 4 * (l >> 4) + q);
    sA[m][to][tc][l] = v;
  }
  __syncthreads();
  const int c_first = (grp * 4 + wave) * kRCols;
  if (c_first >= n_chunks) return;  // whole wave exits together (no barrier follows)
  const int n = lane & 15, g = lane >> 4;
  const int c = c_first + n;
  const bool valid = c < n_chunks;
  const int t0 = c * kChunk;
  const int len = valid ? min(kChunk, T - t0) : 0;
  const size_t id = static_cast<size_t>(seq) * n_chunks + (valid ? c : c_first);
  const float* gt = gates + id * kChunk * 3 * DH + 4 * g;
  floatx4 nu[4];
#pragma unroll
  for (int to = 0; to < 4; ++to) {
    nu[to] = floatx4{0.f, 0.f, 0.f, 0.f};
    if (!LOCAL && valid) nu[to] = *reinterpret_cast<const floatx4*>(carry_in + id * DH + 16 * to + 4 * g);
  }
  const int steps = min(kChunk, T - c_first * kChunk);  // the wave's longest chunk
  struct In {
    Raw4<TX> hp[4], gr_[4];  // as loaded (unpacked where the step uses them)
    floatx4 z[4], r[4], nn[4];
    int q;  // PK: the sequence this lane's step starts, -1 elsewhere
  };
  auto load_in = [&](int s, In& v) {
    const bool act = s >= 0 && s < len;
    const int t = t0 + s;
    const int hr = act ? start_row<PK>(pk, b, t) : -1;
    v.q = (PK && hr >= 0) ? pk.hq[t] : -1;
#pragma unroll
    for (int to = 0; to < 4; ++to) {
      const floatx4 zero{0.f, 0.f, 0.f, 0.f};
      v.hp[to] = v.gr_[to] = Raw4<TX>{};
      v.z[to] = v.r[to] = v.nn[to] = zero;
      if (act) {
        const int j = 16 * to + 4 * g;
        if (hr < 0)
          v.hp[to] = ldr4(states + h_at(b, t - 1, T, d, head, j));
        else if (h0 != nullptr)
          v.hp[to] = ldr4(h0 + static_cast<size_t>(hr) * d + head * DH + j);
        v.gr_[to] = ldr4(grad + h_at(b, t, T, d, head, j));
        v.z[to] = *reinterpret_cast<const floatx4*>(gt + (s * 3) * DH + 16 * to);
        v.r[to] = *reinterpret_cast<const floatx4*>(gt + (s * 3 + 1) * DH + 16 * to);
        v.nn[to] = *reinterpret_cast<const floatx4*>(gt + (s * 3 + 2) * DH + 16 * to);
      }
    }
  };
  In nx;
  load_in(steps - 1, nx);
  for (int s = steps - 1; s >= 0; --s) {
    const bool act = s < len;
    const int t = t0 + s;
    const In cur = nx;
    if (s > 0) load_in(s - 1, nx);
    floatx4 hpv[4], grv[4];
#pragma unroll
    for (int to = 0; to < 4; ++to) {
      hpv[to] = unpack4<TX>(cur.hp[to]);
      grv[to] = unpack4<TX>(cur.gr_[to]);
    }
    // mu = g + nu;  d_zpre = mu (n - h) z(1-z);  d_npre = mu z (1-n^2)
    floatx4 mu[4], dz[4], dn[4], dr[4], tz[4], du[4], tr[4];
#pragma unroll
    for (int to = 0; to < 4; ++to)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const float z = cur.z[to][v], nv = cur.nn[to][v];
        mu[to][v] = grv[to][v] + nu[to][v];
        dz[to][v] = mu[to][v] * (nv - hpv[to][v]) * (z * (1.f - z));
        dn[to][v] = mu[to][v] * z * (1.f - nv * nv);
      }
#pragma unroll
    for (int to = 0; to < 4; ++to) tz[to] = du[to] = tr[to] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int tc = 0; tc < 4; ++tc) {
      floatx4 az[4], an[4];
#pragma unroll
      for (int to = 0; to < 4; ++to) {
        az[to] = sA[0][to][tc][lane];
        an[to] = sA[2][to][tc][lane];
      }
#pragma unroll
      for (int v = 0; v < 4; ++v) {
#pragma unroll
        for (int to = 0; to < 4; ++to) {
          tz[to] = mfma_f32(az[to][v], dz[tc][v], tz[to]);
          du[to] = mfma_f32(an[to][v], dn[tc][v], du[to]);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    // d_rpre = d_u h r(1-r)
#pragma unroll
    for (int to = 0; to < 4; ++to)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const float r = cur.r[to][v];
        dr[to][v] = du[to][v] * hpv[to][v] * r * (1.f - r);
      }
#pragma unroll
    for (int tc = 0; tc < 4; ++tc) {
      floatx4 ar[4];
#pragma unroll
      for (int to = 0; to < 4; ++to) ar[to] = sA[1][to][tc][lane];
#pragma unroll
      for (int v = 0; v < 4; ++v) {
#pragma unroll
        for (int to = 0; to < 4; ++to) tr[to] = mfma_f32(ar[to][v], dr[tc][v], tr[to]);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    // nu <- (1-z) mu + A_z d_zpre + r d_u + A_r d_rpre
#pragma unroll
    for (int to = 0; to < 4; ++to)
#pragma unroll
      for (int v = 0; v < 4; ++v)
        nu[to][v] = (1.f - cur.z[to][v]) * mu[to][v] + tz[to][v] + cur.r[to][v] * du[to][v] +
                    tr[to][v];
    if (!LOCAL && act) {
#pragma unroll
      for (int to = 0; to < 4; ++to) {
        const int j = 16 * to + 4 * g;
        st4(g_wx + wx_at(b, t, T, d, 0, head, j), dz[to]);
        st4(g_wx + wx_at(b, t, T, d, 1, head, j), dr[to]);
        st4(g_wx + wx_at(b, t, T, d, 2, head, j), dn[to]);
      }
    }
    if constexpr (PK) {
      if (cur.q >= 0) {
#pragma unroll
        for (int to = 0; to < 4; ++to) {
          if (!LOCAL && g_h0 != nullptr)
            *reinterpret_cast<floatx4*>(g_h0 + static_cast<size_t>(cur.q) * d + head * DH +
                                        16 * to + 4 * g) = nu[to];
          nu[to] = floatx4{0.f, 0.f, 0.f, 0.f};
        }
      }
    }
  }
  if (valid) {
#pragma unroll
    for (int to = 0; to < 4; ++to) {
      const int j = 16 * to + 4 * g;
      if (LOCAL)
        *reinterpret_cast<floatx4*>(e_out + id * DH + j) = nu[to];
      else if (!PK && c == 0 && g_h0 != nullptr)
        *reinterpret_cast<floatx4*>(g_h0 + static_cast<size_t>(b) * d + head * DH + j) = nu[to];
    }
  }
}

// Partial sums of g_A[gate][head][i][o] = sum over rows k = (b, t) of
// X_g[k][i] D_g[k][o] over one split of the B T rows, all three gates in one
// block (X = h_prev for z and r, h_prev r for n; D the gate's pre-activation
// gradients), so h_prev and r are read once.  4 waves; wave w owns the output
// columns 16 w .. 16 w + 15 of each gate (four 16x16 tiles down the rows i).
// Rows are staged through LDS 16 at a time.
constexpr int kGaRows = 16;
constexpr int kGaPad = 80;  // fp32 LDS row stride (the 4 lane groups land on distinct banks)

template <typename TX, bool PK>
__global__ __launch_bounds__(256) void gru_ga_kernel(
    const TX* __restrict__ h0, const TX* __restrict__ states, const float* __restrict__ gates,
    const TX* __restrict__ g_wx, int B, int T, int H, int n_chunks, int n_split, int rows_per,
    float* __restrict__ part, GPk pk) {
  __shared__ float sx[2][kGaRows][kGaPad], sy[3][kGaRows][kGaPad];
  const int split = blockIdx.x % n_split;
  const int head = blockIdx.x / n_split;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int li = lane & 15, g = lane >> 4;
  const int d = H * DH;
  const long long n_rows = static_cast<long long>(B) * T;
  const long long r0 = static_cast<long long>(split) * rows_per;
  const long long r1 = min(n_rows, r0 + rows_per);
  floatx4 acc[3][4];
#pragma unroll
  for (int q = 0; q < 3; ++q)
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) acc[q][rt] = floatx4{0.f, 0.f, 0.f, 0.f};
  // Thread t stages channels 4 (t % 16) .. + 3 of row t / 16 of each block
  // of 16 rows, one 128-bit load per array; the next block is loaded while
  // the current one's products run.
  static_assert(kGaRows * DH == 4 * 256, "one float4 per thread and array");
  const int sr = threadIdx.x / 16, sj = 4 * (threadIdx.x % 16);
  struct Stage {
    Raw4<TX> hv, y0, y1, y2;  // h_{t-1} and dL/dwx as loaded (unpacked when staged)
    floatx4 rv;               // r_t (h r is formed when staged)
  };
  auto load_rows = [&](long long k0, Stage& st) {
    const floatx4 zero{0.f, 0.f, 0.f, 0.f};
    st.hv = st.y0 = st.y1 = st.y2 = Raw4<TX>{};
    st.rv = zero;
    const long long k = k0 + sr;
    if (k < r1) {
      const int b = static_cast<int>(k / T), t = static_cast<int>(k % T);
      const int hr = start_row<PK>(pk, b, t);
      if (hr < 0)
        st.hv = ldr4(states + h_at(b, t - 1, T, d, head, sj));
      else if (h0 != nullptr)
        st.hv = ldr4(h0 + static_cast<size_t>(hr) * d + head * DH + sj);
      const size_t task = static_cast<size_t>(b * H + head) * n_chunks + t / kChunk;
      // r stays as loaded: multiplying here would wait for these loads at
      // once instead of while the current block's products run
      st.rv =
          *reinterpret_cast<const floatx4*>(gates + ((task * kChunk + t % kChunk) * 3 + 1) * DH + sj);
      st.y0 = ldr4(g_wx + wx_at(b, t, T, d, 0, head, sj));
      st.y1 = ldr4(g_wx + wx_at(b, t, T, d, 1, head, sj));
      st.y2 = ldr4(g_wx + wx_at(b, t, T, d, 2, head, sj));
    }
  };
  Stage nx;
  load_rows(r0, nx);
  for (long long k0 = r0; k0 < r1; k0 += kGaRows) {
    __syncthreads();  // the previous block's products are done with sx / sy
    const floatx4 hv = unpack4<TX>(nx.hv);
    *reinterpret_cast<floatx4*>(&sx[0][sr][sj]) = hv;
    *reinterpret_cast<floatx4*>(&sx[1][sr][sj]) = hv * nx.rv;
    *reinterpret_cast<floatx4*>(&sy[0][sr][sj]) = unpack4<TX>(nx.y0);
    *reinterpret_cast<floatx4*>(&sy[1][sr][sj]) = unpack4<TX>(nx.y1);
    *reinterpret_cast<floatx4*>(&sy[2][sr][sj]) = unpack4<TX>(nx.y2);
    __syncthreads();
    if (k0 + kGaRows < r1) load_rows(k0 + kGaRows, nx);
#pragma unroll
    for (int kk = 0; kk < kGaRows / 4; ++kk) {
      const float* xh = &sx[0][4 * kk + g][li];
      const float* xu = &sx[1][4 * kk + g][li];
#pragma unroll
      for (int q = 0; q < 3; ++q) {
        const float bv = sy[q][4 * kk + g][16 * wave + li];
        const float* xa = q == 2 ? xu : xh;
#pragma unroll
        for (int rt = 0; rt < 4; ++rt) acc[q][rt] = mfma_f32(xa[16 * rt], bv, acc[q][rt]);
      }
    }
  }
#pragma unroll
  for (int q = 0; q < 3; ++q) {
    float* po = part + (static_cast<size_t>(head * 3 + q) * n_split + split) * DH * DH;
#pragma unroll
    for (int rt = 0; rt < 4; ++rt)
#pragma unroll
      for (int v = 0; v < 4; ++v) po[(16 * rt + 4 * g + v) * DH + 16 * wave + li] = acc[q][rt][v];
  }
}

// g_a[gate][head] = sum over the splits.  Each block takes 64 elements; its
// four waves sum every fourth split (wave q: splits q, q + 4, ...) and the four
// partial sums are added in wave order, so the order is fixed (deterministic)
// and four times as many loads are in flight as with one thread per element.
__global__ __launch_bounds__(256) void gru_ga_reduce_kernel(const float* __restrict__ part,
                                                           int H, int n_split,
                                                           float* __restrict__ g_a) {
  __shared__ float s_part[4][64];
  const int lane = threadIdx.x & 63, q = threadIdx.x >> 6;
  const int e = blockIdx.x * 64 + lane;  // over 3 H 64 64
  float acc = 0.f;
  if (e < 3 * H * DH * DH) {
    const int mat = e / (DH * DH), ij = e % (DH * DH);
    const int gate = mat / H, head = mat % H;
    const float* p = part + (static_cast<size_t>(head * 3 + gate) * n_split) * DH * DH + ij;
    for (int sp = q; sp < n_split; sp += 4) acc += p[static_cast<size_t>(sp) * DH * DH];
  }
  s_part[q][lane] = acc;
  __syncthreads();
  if (q == 0 && e < 3 * H * DH * DH)
    g_a[e] = ((s_part[0][lane] + s_part[1][lane]) + s_part[2][lane]) + s_part[3][lane];
}


// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
// Two-level carry scan: group transfers Psi, group carry-outs ell and the
// carries entering each group.
struct CarryWs {
  float* psi;
  float* ell;
  float* cg;
};

static CarryWs carve_carry(Carver& cv, int n_seq, int n_chunks) {
  const size_t ng = static_cast<size_t>(n_seq) * ((n_chunks + kGroup - 1) / kGroup);
  CarryWs c;
  c.psi = static_cast<float*>(cv.take(sizeof(float) * ng * DH * DH));
  c.ell = static_cast<float*>(cv.take(sizeof(float) * ng * DH));
  c.cg = static_cast<float*>(cv.take(sizeof(float) * ng * DH));
  return c;
}

// carry[c] = the carry entering chunk c of every sequence, from the stored
// chunk matrices (Phi, or Phi^T walked from the last chunk down for REV) and
// the local solutions e.  More than one group: group transfers in parallel,
// a serial walk over the groups, then every group re-walked from its carry.
template <bool REV>
static void carry_scan(const float* phi, const float* e, float* carry, int n_seq, int n_chunks,
                       const CarryWs& c, hipStream_t stream) {
  const int n_groups = (n_chunks + kGroup - 1) / kGroup;
  const dim3 walk_block(64 * 16), rewalk_block(64 * 4);
  static const bool single = [] {
    const char* e = getenv("PRNN_GRU_CARRY_SINGLE");
    return e && atoi(e) != 0;
  }();
  if (n_groups <= 1 || single) {
    gru_carry_kernel<REV, 16><<<dim3(n_seq), walk_block, 0, stream>>>(phi, e, n_chunks, n_chunks,
                                                                  nullptr, carry);
    return;
  }
  gru_group_kernel<REV><<<dim3(n_seq * n_groups), dim3(256), 0, stream>>>(phi, e, n_chunks, c.psi,
                                                                         c.ell);
  gru_carry_kernel<false, 16><<<dim3(n_seq), walk_block, 0, stream>>>(c.psi, c.ell, n_groups,
                                                                  n_groups, nullptr, c.cg);
  gru_carry_kernel<REV, 4><<<dim3(n_seq * n_groups), rewalk_block, 0, stream>>>(phi, e, n_chunks,
                                                                           kGroup, c.cg, carry);
}

struct Ws {
  float* phi;
  float* e;
  float* carry;
  float* gates;
  float* work[2];
  u32x4* at;     // packed bf16 A^T operands of the chunk kernel
  floatx4* atb;  // packed fp32 B operands of its gate GEMMs
  CarryWs cs;
  int* hq;  // packed streams: the head table (see GPk)
};

static u32x4* carve_at(Carver& cv, int H) {
  return static_cast<u32x4*>(cv.take(sizeof(u32x4) * static_cast<size_t>(H) * 3 * 4 * 2 * 64));
}
static floatx4* carve_atb(Carver& cv, int H) {
  return static_cast<floatx4*>(cv.take(sizeof(floatx4) * static_cast<size_t>(H) * 4 * 3 * 4 * 64));
}

static Ws carve(void* base, int B, int T, int H, int K, size_t* total, bool packed = false) {
  const int n_seq = B * H, n_chunks = (T + kChunk - 1) / kChunk;
  Carver cv(base);
  Ws w;
  w.hq = packed ? static_cast<int*>(cv.take(sizeof(int) * static_cast<size_t>(T))) : nullptr;
  w.phi = static_cast<float*>(cv.take(sizeof(float) * static_cast<size_t>(n_seq) * n_chunks * DH * DH));
  w.e = static_cast<float*>(cv.take(sizeof(float) * static_cast<size_t>(n_seq) * n_chunks * DH));
  w.carry = static_cast<float*>(cv.take(sizeof(float) * static_cast<size_t>(n_seq) * n_chunks * DH));
  w.gates = static_cast<float*>(
      cv.take(sizeof(float) * static_cast<size_t>(n_seq) * n_chunks * kChunk * 3 * DH));
  w.cs = carve_carry(cv, n_seq, n_chunks);
  w.at = carve_at(cv, H);
  w.atb = carve_atb(cv, H);
  const size_t hb = sizeof(float) * static_cast<size_t>(B) * T * H * DH;
  w.work[0] = K >= 1 ? static_cast<float*>(cv.take(hb)) : nullptr;
  w.work[1] = K >= 2 ? static_cast<float*>(cv.take(hb)) : nullptr;
  *total = cv.used;
  return w;
}

// Forward replays on the matrix cores (gru_replay_mfma_kernel) when there are
// enough 16-chunk groups to give every SIMD work; otherwise (short or few
// sequences) the per-lane mat-vec kernel, whose waves take 2 chunks each.
// PRNN_GRU_REPLAY_MFMA=1 / 0 forces one or the other (read per call); the
// backward's reverse walks choose the same way (PRNN_GRU_REV_MFMA).
constexpr int kReplayMfmaMinWaves = 512;

static bool walks_mfma(const char* env, int n_seq, int n_chunks) {
  if (const char* e = getenv(env)) return atoi(e) != 0;
  return n_seq * ((n_chunks + kRCols - 1) / kRCols) >= kReplayMfmaMinWaves;
}

template <typename TX, typename TOUT, bool LOCAL, bool PK>
static void launch_replay(const TX* az, const TX* ar, const TX* an, const TX* h0,
                          const float* hin, const float* gates, const float* carry, TOUT* out,
                          float* e, int B, int T, int H, int n_chunks, float omega,
                          hipStream_t stream, const GPk& pk) {
  const int n_seq = B * H;
  if (walks_mfma("PRNN_GRU_REPLAY_MFMA", n_seq, n_chunks)) {
    const int n_grp = (n_chunks + 4 * kRCols - 1) / (4 * kRCols);
    gru_replay_mfma_kernel<TX, TOUT, LOCAL, PK><<<dim3(n_seq * n_grp), dim3(256), 0, stream>>>(
        az, ar, an, h0, hin, gates, carry, out, e, B, T, H, n_chunks, omega, pk);
  } else {
    // kPair chunks per wave give each wave two independent serial walks, but
    // when that leaves SIMDs without a wave (short or few sequences: the
    // reference's B=1, T=4096 shape) one chunk per wave fills them instead
    if (n_seq * ((n_chunks + kPair - 1) / kPair) < kSimds) {
      const int blocks = (n_seq * n_chunks + 3) / 4;
      gru_replay_kernel<TX, TOUT, LOCAL, PK, 1><<<dim3(blocks), dim3(256), 0, stream>>>(
          az, ar, an, h0, hin, gates, carry, out, e, B, T, H, n_chunks, omega, pk);
    } else {
      const int blocks = (n_seq * ((n_chunks + kPair - 1) / kPair) + 3) / 4;
      gru_replay_kernel<TX, TOUT, LOCAL, PK, kPair><<<dim3(blocks), dim3(256), 0, stream>>>(
          az, ar, an, h0, hin, gates, carry, out, e, B, T, H, n_chunks, omega, pk);
    }
  }
}

// The head table of a packed stream: hq[t] = q where t = cu[q], -1 elsewhere.
__global__ __launch_bounds__(256) void gru_heads_kernel(const int* __restrict__ cu, int n_seq,
                                                        int T, int* __restrict__ hq) {
  const int t = blockIdx.x * 256 + threadIdx.x;
  if (t >= T) return;
  int lo = 0, hi = n_seq;  // largest q in [0, n_seq) with cu[q] <= t
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (cu[mid] <= t)
      lo = mid;
    else
      hi = mid;
  }
  hq[t] = cu[lo] == t ? lo : -1;
}

// The initial guess into `out`: every step elementwise, then the t = 0 rows
// from h0 (one step per sequence) when h0 is given.
template <typename TX, typename TOUT, bool PK>
static void launch_init(const TX* wx, const TX* az, const TX* ar, const TX* an, const TX* h0,
                        TOUT* out, int B, int T, int H, hipStream_t stream, const GPk& pk) {
  const int d = H * DH;
  const size_t n = static_cast<size_t>(B) * T * (d / 4);
  const unsigned blocks = static_cast<unsigned>(std::min<size_t>((n + 255) / 256, 8192));
  gru_init_elem_kernel<TX, TOUT, PK><<<dim3(blocks), dim3(256), 0, stream>>>(wx, h0, out, B, T,
                                                                           d, pk);
  if (h0 != nullptr)  // one block of one step per sequence and head: its first step
    gru_init_kernel<TX, TOUT, PK><<<dim3((PK ? pk.n_seq : B) * H), dim3(64), 0, stream>>>(
        wx, az, ar, an, h0, out, B, T, H, 1, 1, pk);
}

template <typename TX, bool PK>
static int run(const TX* wx, const TX* az, const TX* ar, const TX* an, const TX* h0, TX* out,
               int B, int T, int H, int K, float omega, const Ws& w, hipStream_t stream,
               const GPk& pk) {
  const int n_seq = B * H, n_chunks = (T + kChunk - 1) / kChunk;
  if (K == 0) {
    launch_init<TX, TX, PK>(wx, az, ar, an, h0, out, B, T, H, stream, pk);
    PRNN_HIP(hipGetLastError());
    return PRNN_OK;
  }
  launch_init<TX, float, PK>(wx, az, ar, an, h0, w.work[0], B, T, H, stream, pk);
  gru_pack_at_kernel<TX><<<dim3(H), dim3(64), 0, stream>>>(az, ar, an, w.at, w.atb);
  PRNN_HIP(hipGetLastError());
  for (int k = 1; k <= K; ++k) {
    const float* hin = w.work[(k - 1) & 1];
    gru_phi_kernel<TX, float, false, PK><<<dim3(n_seq * n_chunks), dim3(256), 0, stream>>>(
        wx, az, ar, an, h0, hin, B, T, H, n_chunks, w.phi, w.gates, w.at, w.atb, pk);
    PRNN_HIP(hipGetLastError());
    launch_replay<TX, float, true, PK>(az, ar, an, h0, hin, w.gates, nullptr,
                                       static_cast<float*>(nullptr), w.e, B, T, H, n_chunks,
                                       omega, stream, pk);
    PRNN_HIP(hipGetLastError());
    carry_scan<false>(w.phi, w.e, w.carry, n_seq, n_chunks, w.cs, stream);
    PRNN_HIP(hipGetLastError());
    if (k == K)
      launch_replay<TX, TX, false, PK>(az, ar, an, h0, hin, w.gates, w.carry, out, nullptr, B,
                                       T, H, n_chunks, omega, stream, pk);
    else
      launch_replay<TX, float, false, PK>(az, ar, an, h0, hin, w.gates, w.carry, w.work[k & 1],
                                          nullptr, B, T, H, n_chunks, omega, stream, pk);
    PRNN_HIP(hipGetLastError());
  }
  return PRNN_OK;
}

// ---- backward host side ----
struct BwdWs {
  float* phi;
  float* e;
  float* carry;
  float* gates;
  float* part;
  int n_split, rows_per;
  u32x4* at;
  floatx4* atb;
  CarryWs cs;
  int* hq;  // packed streams: the head table (see GPk)
};

static void ga_split(int B, int T, int H, int* n_split, int* rows_per) {
  const long long n_rows = static_cast<long long>(B) * T;
  const long long want = (2048 + H - 1) / H;  // ~2048 blocks in flight
  long long ns = std::min<long long>(want, (n_rows + 63) / 64);
  if (ns < 1) ns = 1;
  long long rp = (n_rows + ns - 1) / ns;
  rp = (rp + kGaRows - 1) / kGaRows * kGaRows;
  *rows_per = static_cast<int>(rp);
  *n_split = static_cast<int>((n_rows + rp - 1) / rp);
}

static BwdWs carve_bwd(void* base, int B, int T, int H, size_t* total, bool packed = false) {
  const int n_seq = B * H, n_chunks = (T + kChunk - 1) / kChunk;
  Carver cv(base);
  BwdWs w;
  const size_t tasks = static_cast<size_t>(n_seq) * n_chunks;
  w.phi = static_cast<float*>(cv.take(sizeof(float) * tasks * DH * DH));
  w.e = static_cast<float*>(cv.take(sizeof(float) * tasks * DH));
  w.carry = static_cast<float*>(cv.take(sizeof(float) * tasks * DH));
  w.gates = static_cast<float*>(cv.take(sizeof(float) * tasks * kChunk * 3 * DH));
  ga_split(B, T, H, &w.n_split, &w.rows_per);
  w.part = static_cast<float*>(cv.take(sizeof(float) * static_cast<size_t>(w.n_split) * 3 * H * DH * DH));
  w.cs = carve_carry(cv, n_seq, n_chunks);
  w.at = carve_at(cv, H);
  w.atb = carve_atb(cv, H);
  w.hq = packed ? static_cast<int*>(cv.take(sizeof(int) * static_cast<size_t>(T))) : nullptr;
  *total = cv.used;
  return w;
}

template <typename TX, bool PK>
static int run_bwd(const TX* wx, const TX* az, const TX* ar, const TX* an, const TX* h0,
                   const TX* states, const TX* grad, TX* g_wx, float* g_a, float* g_h0, int B,
                   int T, int H, const BwdWs& w, hipStream_t stream, const GPk& pk) {
  const int n_seq = B * H, n_chunks = (T + kChunk - 1) / kChunk;
  const int rev_blocks_local = (n_seq * ((n_chunks + kPair - 1) / kPair) + 3) / 4;
  const int rev_blocks = (n_seq * n_chunks + 3) / 4;
  const bool mfma_walks = walks_mfma("PRNN_GRU_REV_MFMA", n_seq, n_chunks);
  const int mfma_blocks = n_seq * ((n_chunks + 4 * kRCols - 1) / (4 * kRCols));
  gru_pack_at_kernel<TX><<<dim3(H), dim3(64), 0, stream>>>(az, ar, an, w.at, w.atb);
  gru_phi_kernel<TX, TX, true, PK><<<dim3(n_seq * n_chunks), dim3(256), 0, stream>>>(
      wx, az, ar, an, h0, states, B, T, H, n_chunks, w.phi, w.gates, w.at, w.atb, pk);
  PRNN_HIP(hipGetLastError());
  if (mfma_walks)
    gru_rev_mfma_kernel<TX, true, PK><<<dim3(mfma_blocks), dim3(256), 0, stream>>>(
        az, ar, an, h0, states, grad, w.gates, nullptr, nullptr, nullptr, w.e, B, T, H,
        n_chunks, pk);
  else if (n_seq * ((n_chunks + kPair - 1) / kPair) < kSimds)  // as in launch_replay
    gru_rev_local_kernel<TX, PK, 1><<<dim3(rev_blocks), dim3(256), 0, stream>>>(
        az, ar, an, h0, states, grad, w.gates, w.e, B, T, H, n_chunks, pk);
  else
    gru_rev_local_kernel<TX, PK, kPair><<<dim3(rev_blocks_local), dim3(256), 0, stream>>>(
        az, ar, an, h0, states, grad, w.gates, w.e, B, T, H, n_chunks, pk);
  PRNN_HIP(hipGetLastError());
  carry_scan<true>(w.phi, w.e, w.carry, n_seq, n_chunks, w.cs, stream);
  PRNN_HIP(hipGetLastError());
  if (mfma_walks)
    gru_rev_mfma_kernel<TX, false, PK><<<dim3(mfma_blocks), dim3(256), 0, stream>>>(
        az, ar, an, h0, states, grad, w.gates, w.carry, g_wx, h0 != nullptr ? g_h0 : nullptr,
        nullptr, B, T, H, n_chunks, pk);
  else
    gru_rev_kernel<TX, PK><<<dim3(rev_blocks), dim3(256), 0, stream>>>(
        az, ar, an, h0, states, grad, w.gates, w.carry, g_wx, h0 != nullptr ? g_h0 : nullptr,
        B, T, H, n_chunks, pk);
  PRNN_HIP(hipGetLastError());
  gru_ga_kernel<TX, PK><<<dim3(w.n_split * H), dim3(256), 0, stream>>>(
      h0, states, w.gates, g_wx, B, T, H, n_chunks, w.n_split, w.rows_per, w.part, pk);
  PRNN_HIP(hipGetLastError());
  gru_ga_reduce_kernel<<<dim3((3 * H * DH * DH + 63) / 64), dim3(256), 0, stream>>>(
      w.part, H, w.n_split, g_a);
  PRNN_HIP(hipGetLastError());
  return PRNN_OK;
}

static int check(int B, int T, int H, int dh, int K, int dtype) {
  if (B < 1 || T < 1 || H < 1)
    return fail(PRNN_ERR_VALUE, "B, T, n_heads must be >= 1, got B=%d T=%d n_heads=%d", B, T, H);
  if (dh != DH) return fail(PRNN_ERR_TYPE, "d_head must be %d, got %d", DH, dh);
  if (K < 0) return fail(PRNN_ERR_VALUE, "max_iters must be >= 0, got %d", K);
  if (check_dtype(dtype) != PRNN_OK) return PRNN_ERR_TYPE;
  if (static_cast<long long>(B) * H * ((T + kChunk - 1) / kChunk) > (1ll << 30))
    return fail(PRNN_ERR_VALUE, "problem too large");
  return PRNN_OK;
}

}  // namespace gru
}  // namespace prnn

using namespace prnn;

namespace {

int head_newton_call(const void* wx, const void* a_z, const void* a_r, const void* a_n,
                     const void* h0, void* out, int B, int T, int n_heads, int d_head,
                     int max_iters, float omega, int dtype, void* workspace,
                     size_t workspace_bytes, void* stream, const int* cu, int n_seq,
                     const int* tbl) {
  int rc = gru::check(B, T, n_heads, d_head, max_iters, dtype);
  if (rc != PRNN_OK) return rc;
  const bool packed = cu != nullptr;
  if (packed && (n_seq < 1 || n_seq > T))
    return fail(PRNN_ERR_VALUE, "n_seq must be in [1, T], got %d", n_seq);
  if (!wx || !a_z || !a_r || !a_n || !out || !workspace)
    return fail(PRNN_ERR_VALUE, "wx, a_z, a_r, a_n, out and workspace must be non-null");
  size_t need = 0;
  const gru::Ws w = gru::carve(workspace, B, T, n_heads, max_iters, &need, packed);
  if (workspace_bytes < need)
    return fail(PRNN_ERR_VALUE, "workspace too small: %zu < %zu bytes", workspace_bytes, need);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const gru::GPk pk{cu, w.hq, tbl, n_seq};
  if (packed) {
    gru::gru_heads_kernel<<<dim3((T + 255) / 256), dim3(256), 0, s>>>(cu, n_seq, T, w.hq);
    PRNN_HIP(hipGetLastError());
  }
  return with_storage(dtype, [&](auto tag) {
    using TX = decltype(tag);
    const TX* wx_ = static_cast<const TX*>(wx);
    const TX* az = static_cast<const TX*>(a_z);
    const TX* ar = static_cast<const TX*>(a_r);
    const TX* an = static_cast<const TX*>(a_n);
    const TX* h0_ = static_cast<const TX*>(h0);
    TX* out_ = static_cast<TX*>(out);
    if (packed)
      return gru::run<TX, true>(wx_, az, ar, an, h0_, out_, B, T, n_heads, max_iters, omega, w,
                                s, pk);
    return gru::run<TX, false>(wx_, az, ar, an, h0_, out_, B, T, n_heads, max_iters, omega, w,
                               s, pk);
  });
}

int head_backward_call(const void* wx, const void* a_z, const void* a_r, const void* a_n,
                       const void* h0, const void* states, const void* grad, void* g_wx,
                       float* g_a, float* g_h0, int B, int T, int n_heads, int d_head, int dtype,
                       void* workspace, size_t workspace_bytes, void* stream, const int* cu,
                       int n_seq) {
  int rc = gru::check(B, T, n_heads, d_head, 0, dtype);
  if (rc != PRNN_OK) return rc;
  const bool packed = cu != nullptr;
  if (packed && (n_seq < 1 || n_seq > T))
    return fail(PRNN_ERR_VALUE, "n_seq must be in [1, T], got %d", n_seq);
  if (!wx || !a_z || !a_r || !a_n || !states || !grad || !g_wx || !g_a || !workspace)
    return fail(PRNN_ERR_VALUE,
                "wx, a_z, a_r, a_n, states, grad, g_wx, g_a and workspace must be non-null");
  size_t need = 0;
  const gru::BwdWs w = gru::carve_bwd(workspace, B, T, n_heads, &need, packed);
  if (workspace_bytes < need)
    return fail(PRNN_ERR_VALUE, "workspace too small: %zu < %zu bytes", workspace_bytes, need);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const gru::GPk pk{cu, w.hq, nullptr, n_seq};
  if (packed) {
    gru::gru_heads_kernel<<<dim3((T + 255) / 256), dim3(256), 0, s>>>(cu, n_seq, T, w.hq);
    PRNN_HIP(hipGetLastError());
  }
  return with_storage(dtype, [&](auto tag) {
    using TX = decltype(tag);
    const TX* wx_ = static_cast<const TX*>(wx);
    const TX* az = static_cast<const TX*>(a_z);
    const TX* ar = static_cast<const TX*>(a_r);
    const TX* an = static_cast<const TX*>(a_n);
    const TX* h0_ = static_cast<const TX*>(h0);
    const TX* st_ = static_cast<const TX*>(states);
    const TX* gr_ = static_cast<const TX*>(grad);
    TX* gwx = static_cast<TX*>(g_wx);
    if (packed)
      return gru::run_bwd<TX, true>(wx_, az, ar, an, h0_, st_, gr_, gwx, g_a, g_h0, B, T,
                                    n_heads, w, s, pk);
    return gru::run_bwd<TX, false>(wx_, az, ar, an, h0_, st_, gr_, gwx, g_a, g_h0, B, T, n_heads,
                                   w, s, pk);
  });
}

}  // namespace

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
  return head_newton_call(wx, a_z, a_r, a_n, h0, out, B, T, n_heads, d_head, max_iters, omega,
                          dtype, workspace, workspace_bytes, stream, nullptr, 0, nullptr);
}

extern "C" PRNN_API size_t prnn_gru_head_newton_packed_workspace_size(int T, int n_heads,
                                                                      int d_head, int max_iters,
                                                                      int dtype) {
  if (gru::check(1, T, n_heads, d_head, max_iters, dtype) != PRNN_OK) return 0;
  size_t total = 0;
  gru::carve(nullptr, 1, T, n_heads, max_iters, &total, true);
  return total;
}

extern "C" PRNN_API int prnn_gru_head_newton_packed(const void* wx, const void* a_z,
                                                    const void* a_r, const void* a_n,
                                                    const void* h0, void* out, int T,
                                                    int n_heads, int d_head, int max_iters,
                                                    float omega, int dtype,
                                                    const int* cu_seqlens, int n_seq,
                                                    const int* block_table, void* workspace,
                                                    size_t workspace_bytes, void* stream) {
  if (!cu_seqlens) return fail(PRNN_ERR_VALUE, "cu_seqlens must be non-null");
  return head_newton_call(wx, a_z, a_r, a_n, h0, out, 1, T, n_heads, d_head, max_iters, omega,
                          dtype, workspace, workspace_bytes, stream, cu_seqlens, n_seq,
                          block_table);
}

extern "C" PRNN_API size_t prnn_gru_head_backward_workspace_size(int B, int T, int n_heads,
                                                                 int d_head, int dtype) {
  if (gru::check(B, T, n_heads, d_head, 0, dtype) != PRNN_OK) return 0;
  size_t total = 0;
  gru::carve_bwd(nullptr, B, T, n_heads, &total);
  return total;
}

extern "C" PRNN_API int prnn_gru_head_backward(const void* wx, const void* a_z, const void* a_r,
                                               const void* a_n, const void* h0,
                                               const void* states, const void* grad, void* g_wx,
                                               float* g_a, float* g_h0, int B, int T,
                                               int n_heads, int d_head, int dtype,
                                               void* workspace, size_t workspace_bytes,
                                               void* stream) {
  return head_backward_call(wx, a_z, a_r, a_n, h0, states, grad, g_wx, g_a, g_h0, B, T, n_heads,
                            d_head, dtype, workspace, workspace_bytes, stream, nullptr, 0);
}

extern "C" PRNN_API size_t prnn_gru_head_backward_packed_workspace_size(int T, int n_heads,
                                                                        int d_head, int dtype) {
  if (gru::check(1, T, n_heads, d_head, 0, dtype) != PRNN_OK) return 0;
  size_t total = 0;
  gru::carve_bwd(nullptr, 1, T, n_heads, &total, true);
  return total;
}

extern "C" PRNN_API int prnn_gru_head_backward_packed(const void* wx, const void* a_z,
                                                      const void* a_r, const void* a_n,
                                                      const void* h0, const void* states,
                                                      const void* grad, void* g_wx, float* g_a,
                                                      float* g_h0, int T, int n_heads,
                                                      int d_head, int dtype,
                                                      const int* cu_seqlens, int n_seq,
                                                      void* workspace, size_t workspace_bytes,
                                                      void* stream) {
  if (!cu_seqlens) return fail(PRNN_ERR_VALUE, "cu_seqlens must be non-null");
  return head_backward_call(wx, a_z, a_r, a_n, h0, states, grad, g_wx, g_a, g_h0, 1, T, n_heads,
                            d_head, dtype, workspace, workspace_bytes, stream, cu_seqlens, n_seq);
}
