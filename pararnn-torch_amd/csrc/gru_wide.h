// Device code shared by the wide-head kernels (gru_wide.hip: the walks, the
// gates and the one-launch Newton solve; gru_wide_rev.hip: the adjoint walk):
// lane roles, the A entries a lane keeps, the pair products, the staging of
// a block's per-step inputs and the argument checks.
#pragma once

#include <type_traits>

#include "prnn_common.h"
#include "pararnn_amd.h"
#include "prnn_host.h"

namespace prnn {
namespace gruw {

typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int DW = 128;       // widest head
constexpr int kParts = 8;     // parts of the contraction index
constexpr int kKP = DW / kParts;  // contraction entries per lane (16)
constexpr int kK = 2 * kKP;   // entries per lane and matrix: two channels (32)
constexpr int kThreads = DW / 2 * kParts;
// A broadcast vector sits in LDS in two halves of 64 entries, the second
// shifted by four words (bank spread of the segments one wave reads).
constexpr int kVec = DW + 4;
__device__ __forceinline__ int slot(int c) { return c + (c >> 6) * 4; }

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

// Lane roles.  Lane l of wave w holds the channel pair 2 p, 2 p + 1 with
// p = 8 w + l / 8, and the contraction entries k in [16 j, 16 j + 16) with
// j = l % 8: its products read 16 entries of the broadcast vector and feed
// two channels (half the LDS reads per multiply-add of one channel per
// lane: the walks are bound by the LDS read rate).  After the reduction the
// lanes j < 4 hold channel 2 p and the lanes j >= 4 channel 2 p + 1; j = 0
// and j = 4 write it.
struct Role {
  int pair, part, c;
  bool wr;
};
__device__ __forceinline__ Role role() {
  const int lane = threadIdx.x & 63;
  Role o;
  o.part = lane & (kParts - 1);
  o.pair = (threadIdx.x >> 6) * 8 + (lane >> 3);
  o.c = 2 * o.pair + (o.part >> 2);
  o.wr = (o.part & 3) == 0;
  return o;
}

// Entries k in [16 j, 16 j + 16) of columns (COL) or rows 2 p, 2 p + 1 of a
// head's A ((in, out) layout, d_head x d_head), zero outside the head, the
// lane's own channel c first: a[2 kk + i] = A[k][ch_i] (COL) or A[ch_i][k]
// with ch_0 = c and ch_1 the other channel of the pair.
template <typename TX, bool COL>
__device__ __forceinline__ void load_pair(const TX* A, int dh, const Role& ro, float a[kK]) {
#pragma unroll
  for (int kk = 0; kk < kKP; ++kk)
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int k = ro.part * kKP + kk, ch = ro.c ^ i;
      const bool in = ch < dh && k < dh;
      a[2 * kk + i] =
          in ? ld(A + (COL ? static_cast<size_t>(k) * dh + ch : static_cast<size_t>(ch) * dh + k))
             : 0.f;
    }
}

// A step's per-channel inputs (z, r, n, the previous state, and the iterate
// or dL/dH) are staged through LDS kS steps at a time: while a block of kS
// steps is walked from LDS, every lane holds its share of the next block's
// loads in registers and writes them to the other LDS buffer at the end of
// the block.  A walk step is short, so loads issued per step would expose
// the memory latency every step; here it overlaps kS steps of work.
constexpr int kS = 16;                     // steps per staged block
constexpr int kIn = 5;                     // inputs per step and channel
constexpr int kPer = kIn * kS * DW / kThreads;  // staged values per lane (20)

struct Staged {
  float v[kPer];
};

// Lane `tid` loads values j = 0 .. kPer-1 of the block whose steps are
// t_first + dir * s (s < kS): input j / 4, step s = tid / DW + 4 (j % 4),
// channel tid % DW (clamped into the head and the sequence: the values
// outside are never used).
template <typename TG>
__device__ __forceinline__ Staged load_block(const float* __restrict__ z,
                                             const float* __restrict__ r,
                                             const float* __restrict__ n,
                                             const float* __restrict__ hp,
                                             const TG* __restrict__ x, size_t row_base, int d,
                                             int head, int dh, int t_first, int dir, int t_lo,
                                             int t_hi) {
  const int cc = min(static_cast<int>(threadIdx.x) & (DW - 1), dh - 1);
  const size_t colb = row_base + static_cast<size_t>(head) * dh + cc;
  Staged st;
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int s = static_cast<int>(threadIdx.x) / DW + 4 * (j % 4);
    const int t = min(max(t_first + dir * s, t_lo), t_hi);
    const size_t at = colb + static_cast<size_t>(t) * d;
    const int a = j / 4;
    st.v[j] = a == 0 ? z[at] : a == 1 ? r[at] : a == 2 ? n[at] : a == 3 ? hp[at] : ld(x + at);
  }
  return st;
}

__device__ __forceinline__ void store_block(float (*buf)[kS][DW], const Staged& st, int dh) {
  const int cc = static_cast<int>(threadIdx.x) & (DW - 1);
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int s = static_cast<int>(threadIdx.x) / DW + 4 * (j % 4);
    buf[j / 4][s][cc] = cc < dh ? st.v[j] : 0.f;  // dead channels read zeros
  }
}

// A lane's value from the lane the DPP control names (every lane has a
// source for the controls used here).  Written as an update with old = 0 and
// bound_ctrl so that the compiler folds the move into the add that consumes
// it (v_add_f32 with a DPP operand): one instruction per reduction step.
template <int CTRL>
__device__ __forceinline__ float dppf(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}

// sum_k A v for this lane's channel: the lane's 16 entries for both of its
// pair's channels (one chain each: two chains per channel and the adds that
// join them ran 2-3% slower), the sums over the eight parts of the
// pair (quad_perm [1,0,3,2] and [2,3,0,1] within each quad for both
// channels, then row_half_mirror between the two quads: each quad sends the
// sum of the channel it does not keep, which the other quad keeps).  Every
// lane of a channel ends with the same sum.
__device__ __forceinline__ float dot_pair(const float a[kK], const float* __restrict__ v,
                                          const Role& ro) {
  const float* seg = v + slot(ro.part * kKP);
  float s0 = 0.f, s1 = 0.f;
#pragma unroll
  for (int kk = 0; kk < kKP; kk += 4) {
    const float4 x = *reinterpret_cast<const float4*>(seg + kk);
    s0 = fmaf(a[2 * kk], x.x, s0);
    s1 = fmaf(a[2 * kk + 1], x.x, s1);
    s0 = fmaf(a[2 * kk + 2], x.y, s0);
    s1 = fmaf(a[2 * kk + 3], x.y, s1);
    s0 = fmaf(a[2 * kk + 4], x.z, s0);
    s1 = fmaf(a[2 * kk + 5], x.z, s1);
    s0 = fmaf(a[2 * kk + 6], x.w, s0);
    s1 = fmaf(a[2 * kk + 7], x.w, s1);
  }
  s0 += dppf<0xB1>(s0);
  s1 += dppf<0xB1>(s1);
  s0 += dppf<0x4E>(s0);
  s1 += dppf<0x4E>(s1);
  return s0 + dppf<0x141>(s1);
}

static int check(int B, int T, int H, int dh, int dtype, const int* cu, int n_seq) {
  if (B < 1 || T < 1 || H < 1)
    return fail(PRNN_ERR_VALUE, "B, T, n_heads must be >= 1, got B=%d T=%d n_heads=%d", B, T, H);
  if (dh < 1 || dh > DW) return fail(PRNN_ERR_TYPE, "d_head must be in [1, %d], got %d", DW, dh);
  if (check_dtype(dtype) != PRNN_OK) return PRNN_ERR_TYPE;
  // one batch row's outputs are addressed with 32-bit buffer offsets
  if (static_cast<long long>(T) * 3 * H * dh * sizeof(float) >= (1ll << 32))
    return fail(PRNN_ERR_VALUE, "a batch row of T * 3 * d fp32 values must stay below 4 GiB");
  if (cu != nullptr && (B != 1 || n_seq < 1 || n_seq > T))
    return fail(PRNN_ERR_VALUE, "a packed stream has B = 1 and n_seq in [1, T], got B=%d n_seq=%d",
                B, n_seq);
  return PRNN_OK;
}

}  // namespace gruw
}  // namespace prnn
