// ParaGRU mix='head' with wide heads (64 < d_head <= 128): the Newton
// iteration's linear solve and the eq. 2.6 adjoint as walks over time, one
// workgroup per (sequence, head) -- and, for K >= 2 iterations, one launch
// whose K walks per (sequence, head) run a few blocks of steps apart, each
// fed by a workgroup evaluating its gates (gruw_newton_kernel, further down).
//
// This is the tier of the reference's streamed head kernel
// (kernels/newton_gru_head.py:765-960, _newton_head_stream_a_kernel: one
// program per (b, head), a serial walk over T per Newton iteration, A_* read
// in fp32).  Here the parts of an iteration that do not depend on the walk
// run beforehand as wide parallel work (the gates z, r, n at the iterate for
// all B*T rows, gruw_gates_kernel), so a walk step is only the Jacobian
// applied to the previous delta,
//     J delta = (1-z) delta + d2 (A_z^T delta) + d3 A_n^T (r delta + d5 (A_r^T delta))
// with d2 = (n-h) z(1-z), d3 = z(1-n^2), d5 = h r(1-r) (reference
// cells/para_gru.py:385-412), three 128-wide mat-vecs.
//
// Workgroup: 512 lanes = 64 channel pairs x 8 parts of the contraction index
// (see Role): a lane keeps 16 entries of each A for both channels of its pair
// in registers -- columns (forward: A^T products) or rows (adjoint: A
// products) -- and the eight parts of a pair are eight neighbouring lanes, so
// their partial sums meet through three DPP moves.  A step then needs LDS
// and a barrier only to broadcast the two vectors the next products read:
// two barriers per step.  fp32 throughout; channels >= d_head and entries
// k >= d_head hold zeros.
#include "gru_wide.h"

namespace prnn {
namespace gruw {

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
  __shared__ __attribute__((aligned(16))) float s_d[kVec];
  __shared__ __attribute__((aligned(16))) float s_w[kVec];
  __shared__ float s_in[2][kIn][kS][DW];
  const Role rl = role();
  const int c = rl.c;
  const int sc = slot(c);
  const int head = blockIdx.x % H;
  const Span sp = span_of(blockIdx.x / H, T, cu);
  const size_t hoff = static_cast<size_t>(head) * dh * dh;
  float az[kK], ar[kK], an[kK];
  load_pair<TX, true>(a_z + hoff, dh, rl, az);
  load_pair<TX, true>(a_r + hoff, dh, rl, ar);
  load_pair<TX, true>(a_n + hoff, dh, rl, an);
  const int d = H * dh;
  const bool live = c < dh;
  const size_t col = static_cast<size_t>(head) * dh + c;
  if (rl.wr) s_d[sc] = 0.f;
  float delta = 0.f;
  if (sp.t0 >= sp.t1) return;
  const size_t row_base = static_cast<size_t>(sp.row) * T * d;
  const rsrc_t ro = make_rsrc(out + row_base,
                              static_cast<uint32_t>(static_cast<size_t>(T) * d * sizeof(TOUT)));
  const uint32_t vo = (live && rl.wr) ? static_cast<uint32_t>(col * sizeof(TOUT)) : kOOB;
  store_block(s_in[0], load_block(z, r, n, hp, hin, row_base, d, head, dh, sp.t0, 1, sp.t0,
                                  sp.t1 - 1), dh);
  __syncthreads();
  int buf = 0;
  for (int tb = sp.t0; tb < sp.t1; tb += kS) {
    const bool more = tb + kS < sp.t1;
    Staged next;
    if (more)
      next = load_block(z, r, n, hp, hin, row_base, d, head, dh, tb + kS, 1, sp.t0, sp.t1 - 1);
    const int ns = min(kS, sp.t1 - tb);
    for (int s = 0; s < ns; ++s) {
      const int t = tb + s;
      const float zt = s_in[buf][0][s][c], rt = s_in[buf][1][s][c], nt = s_in[buf][2][s][c];
      const float ht = s_in[buf][3][s][c], hv = s_in[buf][4][s][c];
      // A_r^T delta and A_z^T delta (delta_{t-1} broadcast in s_d)
      const float sr = dot_pair(ar, s_d, rl);
      const float sz = dot_pair(az, s_d, rl);
      const float d5 = ht * rt * (1.f - rt);
      if (rl.wr) s_w[sc] = rt * delta + d5 * sr;
      __syncthreads();
      // A_n^T (r delta + d5 A_r^T delta)
      const float sn = dot_pair(an, s_w, rl);
      const float d2 = (nt - ht) * zt * (1.f - zt);
      const float d3 = zt * (1.f - nt * nt);
      const float f = lerp_t(ht, nt, zt) - hv;
      delta = (1.f - zt) * delta + d2 * sz + d3 * sn + f;
      if (rl.wr) s_d[sc] = delta;
      // a buffer store, dropped for lanes with the out-of-range offset
      stb<TOUT>(ro, vo, static_cast<uint32_t>(t) * (d * sizeof(TOUT)), hv + omega * delta);
      __syncthreads();
    }
    if (more) {
      store_block(s_in[buf ^ 1], next, dh);
      __syncthreads();
    }
    buf ^= 1;
  }
}

// Gates z, r, n of every row (b, t) at its previous state hp: z =
// sigmoid(wx_z + hp A_z), r = sigmoid(wx_r + hp A_r), n = tanh(wx_n + (hp r)
// A_n), per head (reference cells/para_gru.py:443-467).  Rows are independent
// (no walk), so the products are fp32 GEMMs on the matrix cores
// (v_mfma_f32_16x16x4f32): workgroup (head, block of rows) takes 16 rows at
// a time, wave w the 16 output channels 16 w .. 16 w + 15.  The contraction
// index is permuted so that lane (n, g) = (l % 16, l / 16) supplies entries k
// = 32 g + j (j = 0 .. 31) of row n of hp (eight 16-byte LDS reads) and holds
// column 16 w + n of each A at the same k in registers.  h A_z and h A_r for
// the 16 rows, then, after one barrier for the (hp r) rows, (hp r) A_n.  z, r,
// n fp32 (rows, d).
constexpr int kGRows = 16;          // rows per MFMA tile
constexpr int kGPad = DW + 4;       // LDS row stride of the staged rows
__device__ __forceinline__ floatx4 mfma_f32(float a, float b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

template <typename TX>
__global__ __launch_bounds__(kThreads) void gruw_gates_kernel(
    const TX* __restrict__ wx, const float* __restrict__ hp, const TX* __restrict__ a_z,
    const TX* __restrict__ a_r, const TX* __restrict__ a_n, float* __restrict__ z,
    float* __restrict__ r, float* __restrict__ n, int rows, int rows_per_block, int H, int dh) {
  __shared__ __attribute__((aligned(16))) float s_h[kGRows][kGPad];
  __shared__ __attribute__((aligned(16))) float s_hr[kGRows][kGPad];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int li = lane & 15, g = lane >> 4;
  const int head = blockIdx.x % H;
  const int r0 = (blockIdx.x / H) * rows_per_block;
  const int r1 = min(rows, r0 + rows_per_block);
  if (r0 >= r1) return;
  const int d = H * dh;
  const int col = 16 * wave + li;  // this lane's output channel within the head
  const bool live = col < dh;
  // B operands: A[32 g + j][col] (zero outside the head)
  float bz[32], br[32], bn[32];
  {
    const size_t hoff = static_cast<size_t>(head) * dh * dh;
#pragma unroll
    for (int j = 0; j < 32; ++j) {
      const int k = 32 * g + j;
      const bool in = live && k < dh;
      const size_t at = hoff + static_cast<size_t>(k) * dh + col;
      bz[j] = in ? ld(a_z + at) : 0.f;
      br[j] = in ? ld(a_r + at) : 0.f;
      bn[j] = in ? ld(a_n + at) : 0.f;
    }
  }
  const size_t ccol = static_cast<size_t>(head) * dh + min(col, dh - 1);
  // Staging of hp rows: thread tid holds channel tid % DW of rows tid / DW + 4 q.
  const int sc = static_cast<int>(threadIdx.x) & (DW - 1);
  const bool live_sc = sc < dh;
  const size_t scol = static_cast<size_t>(head) * dh + min(sc, dh - 1);
  constexpr int kQ = kGRows * DW / kThreads;  // 4
  float nh[kQ], nx[3][4];
  auto fetch = [&](int rb) {
#pragma unroll
    for (int q = 0; q < kQ; ++q) {
      const int row = min(rb + static_cast<int>(threadIdx.x) / DW + 4 * q, r1 - 1);
      nh[q] = hp[static_cast<size_t>(row) * d + scol];
    }
    // wx at this lane's output positions: rows 4 g + v, channel col
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const size_t row = static_cast<size_t>(min(rb + 4 * g + v, r1 - 1));
#pragma unroll
      for (int gt = 0; gt < 3; ++gt) nx[gt][v] = ld(wx + row * 3 * d + gt * d + ccol);
    }
  };
  fetch(r0);
  for (int rb = r0; rb < r1; rb += kGRows) {
    float cx[3][4];
#pragma unroll
    for (int q = 0; q < kQ; ++q)
      s_h[static_cast<int>(threadIdx.x) / DW + 4 * q][sc] = live_sc ? nh[q] : 0.f;
#pragma unroll
    for (int gt = 0; gt < 3; ++gt)
#pragma unroll
      for (int v = 0; v < 4; ++v) cx[gt][v] = nx[gt][v];
    __syncthreads();
    if (rb + kGRows < r1) fetch(rb + kGRows);
    // A operands: entries 32 g .. 32 g + 31 of row li
    float av[32];
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const float4 f = *reinterpret_cast<const float4*>(&s_h[li][32 * g + 4 * q]);
      av[4 * q] = f.x;
      av[4 * q + 1] = f.y;
      av[4 * q + 2] = f.z;
      av[4 * q + 3] = f.w;
    }
    floatx4 accz = {0.f, 0.f, 0.f, 0.f}, accr = accz;
#pragma unroll
    for (int j = 0; j < 32; ++j) {
      accz = mfma_f32(av[j], bz[j], accz);
      accr = mfma_f32(av[j], br[j], accr);
    }
    // D layout: rows 4 g + v, channel col
    float zv[4];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      zv[v] = fsigmoid(cx[0][v] + accz[v]);
      const float rv = fsigmoid(cx[1][v] + accr[v]);
      s_hr[4 * g + v][col] = s_h[4 * g + v][col] * rv;
      const int row = rb + 4 * g + v;
      if (live && row < r1) {
        const size_t at = static_cast<size_t>(row) * d + ccol;
        z[at] = zv[v];
        r[at] = rv;
      }
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const float4 f = *reinterpret_cast<const float4*>(&s_hr[li][32 * g + 4 * q]);
      av[4 * q] = f.x;
      av[4 * q + 1] = f.y;
      av[4 * q + 2] = f.z;
      av[4 * q + 3] = f.w;
    }
    floatx4 accn = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 32; ++j) accn = mfma_f32(av[j], bn[j], accn);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int row = rb + 4 * g + v;
      if (live && row < r1) n[static_cast<size_t>(row) * d + ccol] = ftanh(cx[2][v] + accn[v]);
    }
    // s_h and s_hr are rewritten for the next rows after this
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// All K Newton iterations in one launch.  Iteration k needs only the previous
// iterate H_{k-1} (at steps t-1 and t), so the iterations of a (sequence,
// head) run together, iteration k a few blocks of steps behind iteration
// k - 1, with kGateWGs + 1 workgroups per (iteration, sequence, head):
//  * gate workgroups evaluate the gates z, r, n of iteration k at H_{k-1}
//    (h A_z, h A_r, then (h r) A_n, a block of steps per barrier; every
//    kGateWGs-th block each) as soon as H_{k-1} reaches them;
//  * a walk workgroup runs the linear solve of iteration k on those gates
//    (the three Jacobian products per step, as in gruw_walk_kernel).
// The gate products do not depend on the walk, so they run on other CUs and
// leave the walk's per-step critical path with the Jacobian alone.
//   H_{k-1} (k >= 1) and the gates pass through the workspace as tagged
// words {value, tag}, written step by step and read with a tag check, so no
// flag or fence orders them (the device-coherent words of the sLSTM
// look-back); iteration 0 reads the initial guess, the last iteration writes
// `out`.  Workgroups take their (k, role, sequence, head) from a ticket in
// start order -- iteration-major, gates before walks -- so whatever a
// workgroup waits on belongs to a running or finished workgroup.  A wait that
// outlasts the spin limit gives up -- the value reads as NaN and the call's
// status word is set -- so every workgroup ends.

// Bounded waits: `limit` polling rounds, then the wait gives up and ORs 1
// into *status (the word after PRNN_TAG_SPAN ticket counters, where
// prnn_slstm_lookback_status reads it).
struct WaitLimit {
  int* status;
  int limit;
};

// Steps per staged block of the one-launch solve (the raw tagged words a
// lane prefetches for the next block, three gates and the iterate per step,
// sit beside the three A's in registers: 8-step blocks ran 6.67 ms at the
// bench's wide shape, 16-step blocks 6.40 ms).
constexpr int kSN = 16;
constexpr int kRows = kThreads / DW;          // steps one load pass covers (4)
constexpr int kXP = 3 * kSN * DW / kThreads;  // staged gate or wx values per lane (12)
constexpr int kSP = kSN * DW / kThreads;      // staged iterate values per lane (4)

// A staged value: plain fp32 (wx converted, the initial guess) or a raw
// tagged word.  Tagged words are kept as loaded and tested only when the
// block is consumed: testing them at the load would make every load of the
// block wait for its round trip in turn.
template <bool TAGGED>
using Raw = typename std::conditional<TAGGED, unsigned long long, float>::type;

// Staged inputs of one block: x (wx for the gate workgroups, the gates z, r,
// n for the walks; gate j / kSP, step tid / DW + kRows (j % kSP)) and the
// iterate H_{k-1} (step tid / DW + kRows j, shifted by vshift).
template <bool XT, bool VT>
struct StagedN {
  Raw<XT> x[kXP];
  Raw<VT> v[kSP];
};

// Sources: the gate words of this iteration (gate g at g * plane) or wx;
// the previous iteration's words or the initial guess.
template <typename TX>
struct NewtonSrc {
  const TX* wx;
  const unsigned long long* gwords;
  size_t plane;
  int gtag;
  const float* guess;
  const unsigned long long* hwords;
  int htag;
};

__device__ __forceinline__ size_t wide_at(size_t row_base, int t, int d, size_t col) {
  return row_base + static_cast<size_t>(t) * d + col;
}

__device__ __forceinline__ unsigned long long ld_word(const unsigned long long* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Where lane tid's staged values of the block at t_first live (steps clamped
// into [t_lo, t_hi]; clamped values are never used).
struct BlockAt {
  size_t row_base;
  int d;
  size_t col;
  int t_first, vshift, t_lo, t_hi;
  __device__ __forceinline__ int x_step(int j) const {
    const int s = static_cast<int>(threadIdx.x) / DW + kRows * (j % kSP);
    return min(max(t_first + s, t_lo), t_hi);
  }
  __device__ __forceinline__ size_t x_at(int j) const {
    return wide_at(row_base, x_step(j), d, col);
  }
  __device__ __forceinline__ size_t v_at(int j) const {
    const int s = static_cast<int>(threadIdx.x) / DW + kRows * j;
    return wide_at(row_base, min(max(t_first + s + vshift, t_lo), t_hi), d, col);
  }
};

template <bool XT, bool VT, typename TX>
__device__ __forceinline__ void load_block_n(StagedN<XT, VT>& st, const NewtonSrc<TX>& src,
                                             const BlockAt& at, int d) {
#pragma unroll
  for (int j = 0; j < kXP; ++j) {
    if constexpr (XT) {
      st.x[j] = ld_word(src.gwords + (j / kSP) * src.plane + at.x_at(j));
    } else {
      // wx rows hold the three gates' blocks of d one after the other
      st.x[j] = ld(src.wx + 3 * wide_at(at.row_base, at.x_step(j), d, 0) +
                   static_cast<size_t>(j / kSP) * d + at.col);
    }
  }
#pragma unroll
  for (int j = 0; j < kSP; ++j) {
    if constexpr (VT)
      st.v[j] = ld_word(src.hwords + at.v_at(j));
    else
      st.v[j] = src.guess[at.v_at(j)];
  }
}

__device__ __forceinline__ bool word_ok(unsigned long long w, int tag) {
  return static_cast<int>(w >> 32) == tag;
}
__device__ __forceinline__ float word_val(unsigned long long w) {
  return __uint_as_float(static_cast<uint32_t>(w));
}

// Waits until every staged tagged word carries this call's tag, reloading
// the ones that do not.  Bounded: after `limit` rounds the lane gives up
// (NaN for what is missing, status word set) and, through `gave_up`, waits
// no more for the rest of its walk.
template <bool XT, bool VT, typename TX>
__device__ __forceinline__ void await_block_n(StagedN<XT, VT>& st, const NewtonSrc<TX>& src,
                                              const BlockAt& at_in, const WaitLimit& spin,
                                              bool& gave_up) {
  if constexpr (XT || VT) {
    // The reload addresses are recomputed from an opaque copy of the block's
    // first step: otherwise the compiler keeps the load's 16 addresses live
    // through the whole block (and spills).
    BlockAt at = at_in;
    asm volatile("" : "+s"(at.t_first));
    auto missing = [&]() {
      bool m = false;
      if constexpr (XT) {
#pragma unroll
        for (int j = 0; j < kXP; ++j) m |= !word_ok(st.x[j], src.gtag);
      }
      if constexpr (VT) {
#pragma unroll
        for (int j = 0; j < kSP; ++j) m |= !word_ok(st.v[j], src.htag);
      }
      return m;
    };
    int rounds = 0;
    while (missing()) {
      if (gave_up || ++rounds > spin.limit) {
        const unsigned long long nan_w = 0x7fc00000ull;
        if constexpr (XT) {
#pragma unroll
          for (int j = 0; j < kXP; ++j)
            if (!word_ok(st.x[j], src.gtag))
              st.x[j] = (static_cast<unsigned long long>(static_cast<uint32_t>(src.gtag)) << 32) |
                        nan_w;
        }
        if constexpr (VT) {
#pragma unroll
          for (int j = 0; j < kSP; ++j)
            if (!word_ok(st.v[j], src.htag))
              st.v[j] = (static_cast<unsigned long long>(static_cast<uint32_t>(src.htag)) << 32) |
                        nan_w;
        }
        if (!gave_up)
          __hip_atomic_fetch_or(spin.status, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        gave_up = true;
        break;
      }
      __builtin_amdgcn_s_sleep(2);
      // reload the whole block (the words already there read the same)
      if constexpr (XT) {
#pragma unroll
        for (int j = 0; j < kXP; ++j)
          st.x[j] = ld_word(src.gwords + (j / kSP) * src.plane + at.x_at(j));
      }
      if constexpr (VT) {
#pragma unroll
        for (int j = 0; j < kSP; ++j) st.v[j] = ld_word(src.hwords + at.v_at(j));
      }
    }
  }
}

template <bool XT, bool VT>
__device__ __forceinline__ void store_block_n(float (*x)[kSN][DW], float (*v)[kVec],
                                              const StagedN<XT, VT>& st, int dh) {
  const int cc = static_cast<int>(threadIdx.x) & (DW - 1);
  const bool live = cc < dh;
#pragma unroll
  for (int j = 0; j < kXP; ++j) {
    float val;
    if constexpr (XT)
      val = word_val(st.x[j]);
    else
      val = st.x[j];
    x[j / kSP][static_cast<int>(threadIdx.x) / DW + kRows * (j % kSP)][cc] = live ? val : 0.f;
  }
#pragma unroll
  for (int j = 0; j < kSP; ++j) {
    float val;
    if constexpr (VT)
      val = word_val(st.v[j]);
    else
      val = st.v[j];
    v[static_cast<int>(threadIdx.x) / DW + kRows * j][slot(cc)] = live ? val : 0.f;
  }
}

// Gate workgroups per walk (each takes every kGateWGs-th block).  One keeps
// up with its walk: with two or three the solve ran 1-2% slower.
constexpr int kGateWGs = 1;

struct NewtonShared {
  float x[2][3][kSN][DW];                               // wx (gates) or z, r, n (walks)
  __attribute__((aligned(16))) float v[2][kSN][kVec];   // H_{k-1}
  __attribute__((aligned(16))) float first[kVec];      // the sequence's initial state
  __attribute__((aligned(16))) float d[kVec];          // walks: delta_{t-1}
  __attribute__((aligned(16))) float w[kVec];          // walks: r delta + d5 A_r^T delta
  __attribute__((aligned(16))) float hr[kSN][kVec];     // gates: (h r) rows of a block
};

// What both roles of a workgroup share.
struct NewtonCtx {
  Role rl;
  int c, sc, head, d, dh, k, K, T;
  bool live;
  size_t col, btd, row_base;
  Span sp;
};

// Gate workgroup `part` of iteration k: blocks part, part + kGateWGs, ... of
// the span.  Step t of a block needs H_{k-1} at t - 1 (the sequence's
// initial state at its first step), staged as the block's rows (vshift -1).
//   z = sigmoid(wx_z + h A_z), r = sigmoid(wx_r + h A_r) for the block's
// steps, then n = tanh(wx_n + (h r) A_n) after one barrier (reference
// cells/para_gru.py:443-467), each written as a tagged word.
template <bool VT, typename TX>
__device__ __forceinline__ void newton_gates(NewtonShared& sh, const NewtonCtx& cx,
                                             const NewtonSrc<TX>& src, int part,
                                             const float az[kK], const float ar[kK],
                                             const float an[kK],
                                             unsigned long long* __restrict__ gk, int gtag,
                                             const WaitLimit& spin) {
  const Span& sp = cx.sp;
  const Role& rl = cx.rl;
  const int c = cx.c, sc = cx.sc;
  int tb = sp.t0 + part * kSN;
  if (tb >= sp.t1) return;
  const int cc = min(static_cast<int>(threadIdx.x) & (DW - 1), cx.dh - 1);
  const size_t ccol = static_cast<size_t>(cx.head) * cx.dh + cc;
  auto at_of = [&](int t_first) {
    return BlockAt{cx.row_base, cx.d, ccol, t_first, -1, sp.t0, sp.t1 - 1};
  };
  bool gave_up = false;
  {
    StagedN<false, VT> st;
    load_block_n(st, src, at_of(tb), cx.d);
    await_block_n(st, src, at_of(tb), spin, gave_up);
    store_block_n(sh.x[0], sh.v[0], st, cx.dh);
  }
  __syncthreads();
  int buf = 0;
  for (; tb < sp.t1; tb += kGateWGs * kSN) {
    const int tn = tb + kGateWGs * kSN;
    const bool more = tn < sp.t1;
    StagedN<false, VT> next;
    if (more) load_block_n(next, src, at_of(tn), cx.d);
    const int ns = min(kSN, sp.t1 - tb);
    auto gates_zr = [&](int s) {
      const float* hrow = tb + s == sp.t0 ? sh.first : sh.v[buf][s];
      const float hz = dot_pair(az, hrow, rl);
      const float hr = dot_pair(ar, hrow, rl);
      const float z = fsigmoid(sh.x[buf][0][s][c] + hz);
      const float r = fsigmoid(sh.x[buf][1][s][c] + hr);
      if (rl.wr) {
        sh.hr[s][sc] = hrow[sc] * r;
        if (cx.live) {
          const size_t a = wide_at(cx.row_base, tb + s, cx.d, cx.col);
          st_tagged(gk + a, z, gtag);
          st_tagged(gk + cx.btd + a, r, gtag);
        }
      }
    };
    auto gate_n = [&](int s) {
      const float un = dot_pair(an, sh.hr[s], rl);
      const float n = ftanh(sh.x[buf][2][s][c] + un);
      if (rl.wr && cx.live)
        st_tagged(gk + 2 * cx.btd + wide_at(cx.row_base, tb + s, cx.d, cx.col), n, gtag);
    };
    if (ns == kSN) {
#pragma unroll
      for (int s = 0; s < kSN; ++s) gates_zr(s);
    } else {
      for (int s = 0; s < ns; ++s) gates_zr(s);
    }
    __syncthreads();
    if (ns == kSN) {
#pragma unroll
      for (int s = 0; s < kSN; ++s) gate_n(s);
    } else {
      for (int s = 0; s < ns; ++s) gate_n(s);
    }
    if (more) {
      await_block_n(next, src, at_of(tn), spin, gave_up);
      store_block_n(sh.x[buf ^ 1], sh.v[buf ^ 1], next, cx.dh);
    }
    // (h r) rows and the staging buffers are rewritten after this
    __syncthreads();
    buf ^= 1;
  }
}

// Walk of iteration k: delta_t = J_t delta_{t-1} + F_t, F_t = lerp(h, n, z) -
// H_t, then H_t + omega delta_t (the gates and H_{k-1} from the staged
// blocks); iterations before the last write tagged words, the last `out`.
template <bool VT, typename TX>
__device__ __forceinline__ void newton_walk(NewtonShared& sh, const NewtonCtx& cx,
                                            const NewtonSrc<TX>& src, const float az[kK],
                                            const float ar[kK], const float an[kK],
                                            unsigned long long* __restrict__ iters,
                                            TX* __restrict__ out, float omega, int tag_base,
                                            const WaitLimit& spin) {
  const Span& sp = cx.sp;
  const Role& rl = cx.rl;
  const int c = cx.c, sc = cx.sc;
  const int cc = min(static_cast<int>(threadIdx.x) & (DW - 1), cx.dh - 1);
  const size_t ccol = static_cast<size_t>(cx.head) * cx.dh + cc;
  auto at_of = [&](int t_first) {
    return BlockAt{cx.row_base, cx.d, ccol, t_first, 0, sp.t0, sp.t1 - 1};
  };
  bool gave_up = false;
  {
    StagedN<true, VT> st;
    load_block_n(st, src, at_of(sp.t0), cx.d);
    await_block_n(st, src, at_of(sp.t0), spin, gave_up);
    store_block_n(sh.x[0], sh.v[0], st, cx.dh);
  }
  __syncthreads();
  const bool last = cx.k == cx.K - 1;
  unsigned long long* dst = last ? nullptr : iters + cx.k * cx.btd;
  const int dst_tag = tag_base + 1 + cx.k;
  const rsrc_t ro = make_rsrc(out + cx.row_base,
                              static_cast<uint32_t>(static_cast<size_t>(cx.T) * cx.d * sizeof(TX)));
  const uint32_t vo =
      (last && cx.live && rl.wr) ? static_cast<uint32_t>(cx.col * sizeof(TX)) : kOOB;
  float delta = 0.f;
  // this lane's word of the iterate at the current step (iterations before the last)
  unsigned long long* dst_t =
      dst == nullptr ? nullptr : dst + wide_at(cx.row_base, sp.t0, cx.d, cx.col);
  int buf = 0;
  for (int tb = sp.t0; tb < sp.t1; tb += kSN) {
    const bool more = tb + kSN < sp.t1;
    StagedN<true, VT> next;
    if (more) load_block_n(next, src, at_of(tb + kSN), cx.d);
    const int ns = min(kSN, sp.t1 - tb);
    for (int s = 0; s < ns; ++s) {
      const int t = tb + s;
      // previous state (the sequence's initial state, the other buffer's
      // last row, or this block's previous row) and the iterate at t
      const float* hrow =
          s > 0 ? sh.v[buf][s - 1] : tb == sp.t0 ? sh.first : sh.v[buf ^ 1][kSN - 1];
      const float hp = hrow[sc];
      const float hin = sh.v[buf][s][sc];
      const float z = sh.x[buf][0][s][c], r = sh.x[buf][1][s][c], n = sh.x[buf][2][s][c];
      // A_r^T delta and A_z^T delta (delta_{t-1} broadcast in sh.d)
      const float sr = dot_pair(ar, sh.d, rl);
      const float sz = dot_pair(az, sh.d, rl);
      const float d5 = hp * r * (1.f - r);
      if (rl.wr) sh.w[sc] = r * delta + d5 * sr;
      __syncthreads();
      // A_n^T (r delta + d5 A_r^T delta)
      const float sn = dot_pair(an, sh.w, rl);
      const float d2 = (n - hp) * z * (1.f - z);
      const float d3 = z * (1.f - n * n);
      const float f = lerp_t(hp, n, z) - hin;
      delta = (1.f - z) * delta + d2 * sz + d3 * sn + f;
      const float h_new = hin + omega * delta;
      if (rl.wr) sh.d[sc] = delta;
      if (dst != nullptr) {
        if (cx.live && rl.wr) st_tagged(dst_t, h_new, dst_tag);
        dst_t += cx.d;
      } else {
        stb<TX>(ro, vo, static_cast<uint32_t>(t) * (cx.d * sizeof(TX)), h_new);
      }
      __syncthreads();
    }
    if (more) {
      await_block_n(next, src, at_of(tb + kSN), spin, gave_up);
      store_block_n(sh.x[buf ^ 1], sh.v[buf ^ 1], next, cx.dh);
      __syncthreads();
    }
    buf ^= 1;
  }
}

template <typename TX>
__global__ __launch_bounds__(kThreads) void gruw_newton_kernel(
    const TX* __restrict__ wx, const TX* __restrict__ a_z, const TX* __restrict__ a_r,
    const TX* __restrict__ a_n, const float* __restrict__ h0, const float* __restrict__ guess,
    unsigned long long* __restrict__ iters, unsigned long long* __restrict__ gates,
    TX* __restrict__ out, int B, int T, int H, int dh, int n_rows, int K, float omega,
    const int* __restrict__ cu, int* __restrict__ ticket, int tag_base, WaitLimit spin) {
  __shared__ NewtonShared sh;
  __shared__ int s_ticket;
  if (threadIdx.x == 0)
    s_ticket = __hip_atomic_fetch_add(ticket, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  // per iteration: kGateWGs gate workgroups per (sequence, head), then the walks
  const int units = n_rows * H;
  const int per_iter = (kGateWGs + 1) * units;
  const int k = s_ticket / per_iter, q = s_ticket % per_iter;
  const bool gate_role = q < kGateWGs * units;
  const int part = q / units;
  const int unit = q % units;
  NewtonCtx cx;
  cx.rl = role();
  cx.c = cx.rl.c;
  cx.sc = slot(cx.c);
  cx.head = unit % H;
  cx.sp = span_of(unit / H, T, cu);
  cx.d = H * dh;
  cx.dh = dh;
  cx.k = k;
  cx.K = K;
  cx.T = T;
  cx.live = cx.c < dh;
  cx.col = static_cast<size_t>(cx.head) * dh + cx.c;
  cx.btd = static_cast<size_t>(B) * T * cx.d;
  cx.row_base = static_cast<size_t>(cx.sp.row) * T * cx.d;
  const size_t hoff = static_cast<size_t>(cx.head) * dh * dh;
  float az[kK], ar[kK], an[kK];
  load_pair<TX, true>(a_z + hoff, dh, cx.rl, az);
  load_pair<TX, true>(a_r + hoff, dh, cx.rl, ar);
  load_pair<TX, true>(a_n + hoff, dh, cx.rl, an);
  // the sequence's initial state (h0 row or zeros) and delta_{t0-1} = 0
  if (cx.rl.wr) {
    sh.first[cx.sc] =
        (cx.live && h0 != nullptr) ? h0[static_cast<size_t>(cx.sp.seq) * cx.d + cx.col] : 0.f;
    sh.d[cx.sc] = 0.f;
  }
  if (cx.sp.t0 >= cx.sp.t1) return;
  // Iterations k and k + 2 share gate words: the gate workgroups of k + 2
  // reach block b only after the iterate of k + 1 covers it, i.e. after the
  // walk of k has finished block b and so read its gates for the last time
  // (distinct tags keep the two iterations' words apart).
  unsigned long long* gk = gates + static_cast<size_t>(k % 2) * 3 * cx.btd;
  const NewtonSrc<TX> src{wx,    gk,    cx.btd, tag_base + 1 + k, guess,
                          k == 0 ? nullptr : iters + (k - 1) * cx.btd, tag_base + k};
  // iteration 0 reads the plain initial guess, later ones the tagged iterate
  if (gate_role) {
    if (k == 0)
      newton_gates<false>(sh, cx, src, part, az, ar, an, gk, tag_base + 1 + k, spin);
    else
      newton_gates<true>(sh, cx, src, part, az, ar, an, gk, tag_base + 1 + k, spin);
  } else {
    if (k == 0)
      newton_walk<false>(sh, cx, src, az, ar, an, iters, out, omega, tag_base, spin);
    else
      newton_walk<true>(sh, cx, src, az, ar, an, iters, out, omega, tag_base, spin);
  }
}

// Workspace of the one-launch Newton solve: PRNN_TAG_SPAN ticket counters
// (the first is used) and the status word, then the tagged iterates
// H_0 .. H_{K-2} and the tagged gates z, r, n of two iterations (even and
// odd k), (B, T, d) 64-bit words each.
struct NewtonWs {
  int* counters;
  unsigned long long* iters;
  unsigned long long* gates;
  size_t clear_words;  // 32-bit words from `counters` to the end
};

static NewtonWs carve_newton(void* base, int B, int T, int d, int K, size_t* total) {
  Carver cv(base);
  NewtonWs w;
  const size_t plane = static_cast<size_t>(B) * T * d;
  w.counters = static_cast<int*>(cv.take(sizeof(int) * (PRNN_TAG_SPAN + 1)));
  w.iters = static_cast<unsigned long long*>(
      cv.take(sizeof(unsigned long long) * static_cast<size_t>(K > 1 ? K - 1 : 0) * plane));
  w.gates = static_cast<unsigned long long*>(
      cv.take(sizeof(unsigned long long) * 3 * static_cast<size_t>(K > 1 ? 2 : 1) * plane));
  w.clear_words = cv.used / sizeof(int);
  *total = cv.used;
  return w;
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

extern "C" PRNN_API size_t prnn_gru_wide_newton_workspace_size(int B, int T, int n_heads,
                                                              int d_head, int max_iters) {
  if (B < 1 || T < 1 || n_heads < 1 || d_head < 1 || max_iters < 1) return 0;
  size_t total = 0;
  gruw::carve_newton(nullptr, B, T, n_heads * d_head, max_iters, &total);
  return total;
}

extern "C" PRNN_API int prnn_gru_wide_newton(const void* wx, const void* a_z, const void* a_r,
                                             const void* a_n, const float* h0,
                                             const float* guess, void* out, int B, int T,
                                             int n_heads, int d_head, int max_iters, float omega,
                                             int dtype, const int* cu_seqlens, int n_seq,
                                             void* workspace, size_t workspace_bytes,
                                             int tag_base, void* stream) {
  int rc = gruw::check(B, T, n_heads, d_head, dtype, cu_seqlens, n_seq);
  if (rc != PRNN_OK) return rc;
  if (max_iters < 1 || max_iters > PRNN_TAG_SPAN)
    return fail(PRNN_ERR_VALUE, "max_iters must be in [1, %d], got %d", PRNN_TAG_SPAN, max_iters);
  if (tag_base < 0 || tag_base > PRNN_TAG_BASE_MAX)
    return fail(PRNN_ERR_VALUE, "tag_base must be in [0, %d], got %d", PRNN_TAG_BASE_MAX,
                tag_base);
  if (!wx || !a_z || !a_r || !a_n || !guess || !out || !workspace)
    return fail(PRNN_ERR_VALUE, "wx, a_z, a_r, a_n, guess, out and workspace must be non-null");
  if (static_cast<const void*>(guess) == out)
    return fail(PRNN_ERR_VALUE, "out must not alias guess");
  const int d = n_heads * d_head;
  size_t need = 0;
  const gruw::NewtonWs w = gruw::carve_newton(workspace, B, T, d, max_iters, &need);
  if (workspace_bytes < need)
    return fail(PRNN_ERR_VALUE, "workspace too small: %zu < %zu bytes", workspace_bytes, need);
  hipStream_t s = static_cast<hipStream_t>(stream);
  // tag_base > 0: every word holds a tag below tag_base + 1, only the
  // counters need zeroing (as for the sLSTM workspaces)
  rc = clear_words(w.counters, tag_base > 0 ? PRNN_TAG_SPAN + 1 : w.clear_words, s);
  if (rc != PRNN_OK) return rc;
  const int rows = cu_seqlens ? n_seq : B;
  const gruw::WaitLimit lim{w.counters + PRNN_TAG_SPAN, spin_limit()};
  // per iteration and (sequence, head): kGateWGs gate workgroups and a walk
  const int grid = (gruw::kGateWGs + 1) * max_iters * rows * n_heads;
  timing_begin(s);
  with_storage(dtype, [&](auto tag) {
    using TX = decltype(tag);
    gruw::gruw_newton_kernel<TX>
        <<<dim3(grid), dim3(gruw::kThreads), 0, s>>>(
            static_cast<const TX*>(wx), static_cast<const TX*>(a_z),
            static_cast<const TX*>(a_r), static_cast<const TX*>(a_n), h0, guess, w.iters,
            w.gates, static_cast<TX*>(out), B, T, n_heads, d_head, rows, max_iters, omega,
            cu_seqlens, w.counters, tag_base, lim);
    return PRNN_OK;
  });
  timing_end(s);
  PRNN_HIP(hipGetLastError());
  return PRNN_OK;
}

extern "C" PRNN_API int prnn_gru_wide_gates(const void* wx, const float* hp, const void* a_z,
                                            const void* a_r, const void* a_n, float* z, float* r,
                                            float* n, int rows, int n_heads, int d_head,
                                            int dtype, void* stream) {
  if (rows < 1 || n_heads < 1)
    return fail(PRNN_ERR_VALUE, "rows and n_heads must be >= 1, got rows=%d n_heads=%d", rows,
                n_heads);
  if (d_head < 1 || d_head > gruw::DW)
    return fail(PRNN_ERR_TYPE, "d_head must be in [1, %d], got %d", gruw::DW, d_head);
  if (check_dtype(dtype) != PRNN_OK) return PRNN_ERR_TYPE;
  if (!wx || !hp || !a_z || !a_r || !a_n || !z || !r || !n)
    return fail(PRNN_ERR_VALUE, "wx, hp, a_z, a_r, a_n, z, r and n must be non-null");
  // about four workgroups per CU over all heads, whole staging blocks each
  const int target = (1024 + n_heads - 1) / n_heads;
  int per = (rows + target - 1) / target;
  per = ((per + gruw::kS - 1) / gruw::kS) * gruw::kS;
  const int blocks = (rows + per - 1) / per;
  hipStream_t s = static_cast<hipStream_t>(stream);
  with_storage(dtype, [&](auto tag) {
    using TX = decltype(tag);
    gruw::gruw_gates_kernel<TX><<<dim3(blocks * n_heads), dim3(gruw::kThreads), 0, s>>>(
        static_cast<const TX*>(wx), hp, static_cast<const TX*>(a_z), static_cast<const TX*>(a_r),
        static_cast<const TX*>(a_n), z, r, n, rows, per, n_heads, d_head);
    return PRNN_OK;
  });
  PRNN_HIP(hipGetLastError());
  return PRNN_OK;
}
