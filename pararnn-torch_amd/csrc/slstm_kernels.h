// ParaSLSTM mix='diag' Newton + scan device code for gfx950 (CDNA4): the
// kernels of slstm_diag.hip (rectangular batches) and slstm_packed.hip
// (packed streams), which instantiate them.
//
// Two single-pass chunked scans over time, both with the same tile schedule:
//
//   tile  = (batch b, channel block of 64, time chunk of W*L steps)
//   lane  = one channel; wave w = L consecutive steps of the chunk
//
// Pass 1 walks the lane's L steps serially from register-cached inputs and
// folds them into the lane's segment aggregate; the W wave aggregates are
// combined through LDS into the tile aggregate; wave 0 publishes it and runs a
// decoupled look-back over earlier chunks of the same (b, channel block) to
// get the carry into the tile; pass 2 replays the L steps from registers with
// the true carry and streams the outputs.  Inputs are read from HBM once and
// outputs written once per launch.
//
// (1) slstm_frozen_kernel: frozen-gate pass (zero-hidden or one Picard pass).
//     Per step  m' = max(z_f + m, z_i),  f = e^{z_f + m - m'},  i = e^{z_i - m'},
//     n' = f n + i,  c' = f c + i tanh z_z,  h = sigmoid(z_o) c' / (n' + eps)
//     with pre = wx (+ R * h_prev of the previous pass).  The carry (m, n, c)
//     composes through the stabilised monoid (F, M, N, C): F = sum z_f, M the
//     max-plus aggregate, N / C the sums scaled by e^{-M}.
//     Reference: solvers/slstm_picard.py:51-107, 143-181.
// (2) slstm_newton_kernel: one Newton iteration.  Per step the cell value
//     f(H_{t-1}, x_t), the 4x4 Jacobian J_t (12 structural non-zeros) and the
//     residual F_t = f - H_t; the scan solves delta_t = J_t delta_{t-1} + F_t
//     on the affine monoid (A, b) -> (J A, J b + F); H_t += omega delta_t.
//     Reference: cells/para_slstm.py:347-446, solvers/scan.py:82-100,
//     solvers/newton/__init__.py:516-543, kernels/newton_slstm.py:886-966.
#pragma once

#include "slstm_scan.h"

#include <stdio.h>
#include <stdlib.h>

#include <type_traits>

namespace prnn {
namespace slstm {

// ---------------------------------------------------------------------------
// (1) frozen-gate pass
// ---------------------------------------------------------------------------

struct FG {
  float F, M, N, C;
};

__device__ __forceinline__ FG fg_identity() { return FG{0.f, -INFINITY, 0.f, 0.f}; }

// Aggregate of segment x followed by segment y.
__device__ __forceinline__ FG fg_compose(FG x, FG y) {
  if (y.M == -INFINITY) return FG{x.F + y.F, x.M, x.N, x.C};
  if (x.M == -INFINITY) return FG{x.F + y.F, y.M, y.N, y.C};
  const float mx = y.F + x.M;
  const float m = fmaxf(mx, y.M);
  const float sx = fexp(mx - m), sy = fexp(y.M - m);
  return FG{x.F + y.F, m, x.N * sx + y.N * sy, x.C * sx + y.C * sy};
}

// Carry (m, n, c) after applying aggregate y to carry (m, n, c).
__device__ __forceinline__ void fg_apply(const FG& y, float& m, float& n, float& c) {
  if (y.M == -INFINITY) return;
  const float mc = y.F + m;
  const float mn = fmaxf(mc, y.M);
  const float sc = fexp(mc - mn), sy = fexp(y.M - mn);
  n = n * sc + y.N * sy;
  c = c * sc + y.C * sy;
  m = mn;
}

// One frozen-gate step in place on (m, n, c), given z = tanh(z_z).
// One of f, i is exactly e^0 = 1 (the larger exponent is the new stabiliser),
// so a single exp of -|left - z_i| gives both, bit-identical to two exps.
__device__ __forceinline__ void fg_step_z(float zi, float zf, float z, float& m, float& n,
                                          float& c) {
  const float left = zf + m;
  const float mn = fmaxf(left, zi);
  const float e = fexp(-fabsf(left - zi));
  const bool lf = left >= zi;
  const float f = lf ? 1.f : e;
  const float i = lf ? e : 1.f;
  n = f * n + i;
  c = f * c + i * z;
  m = mn;
}

__device__ __forceinline__ void fg_step(float zi, float zf, float zz, float& m, float& n, float& c) {
  fg_step_z(zi, zf, ftanh(zz), m, n, c);
}


struct FrozenMonoid {
  static constexpr int NI = 3;  // carry (m, n, c)
  static constexpr int NA = 4;  // aggregate (F, M, N, C)
  using Acc = FG;
  static __device__ __forceinline__ void identity(Acc& a) { a = fg_identity(); }
  static __device__ __forceinline__ void absorb(Acc& acc, const float a[NA]) {
    acc = fg_compose(FG{a[0], a[1], a[2], a[3]}, acc);
  }
  static __device__ __forceinline__ void finish(const Acc& acc, const float v[NI], float out[NI]) {
    float m = v[0], n = v[1], c = v[2];
    fg_apply(acc, m, n, c);
    out[0] = m;
    out[1] = n;
    out[2] = c;
  }
  static __device__ __forceinline__ void apply(const float a[NA], float v[NI]) {
    fg_apply(FG{a[0], a[1], a[2], a[3]}, v[0], v[1], v[2]);
  }
};

// Pre-activations of a tile's steps, held in registers between the two
// passes.  With 16-bit storage they are exact values of the storage type (wx,
// or wx + R h_prev rounded as the reference's two torch ops), packed two to a
// register.
template <typename TX>
struct PreStash {
  using NT = Narrow<TX>;
  static constexpr int N = 2;  // registers per step: (z_i, z_f), (z_z, z_o)
  template <bool HAS_H>
  static __device__ __forceinline__ void make(const uint32_t x[4], const float r[4], float hp,
                                              uint32_t w[N]) {
    if (!HAS_H) {
      w[0] = x[0] | (x[1] << 16);
      w[1] = x[2] | (x[3] << 16);
      return;
    }
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      // round(R h) and round(wx + round(R h)), two gates per conversion.
      const uint32_t q = NT::pack(r[2 * k] * hp, r[2 * k + 1] * hp);
      w[k] = NT::pack(NT::val(x[2 * k]) + NT::lo(q), NT::val(x[2 * k + 1]) + NT::hi(q));
    }
  }
  static __device__ __forceinline__ void get(const uint32_t w[N], float p[4]) {
    p[0] = NT::lo(w[0]);
    p[1] = NT::hi(w[0]);
    p[2] = NT::lo(w[1]);
    p[3] = NT::hi(w[1]);
  }
};

template <>
struct PreStash<float> {
  static constexpr int N = 4;
  template <bool HAS_H>
  static __device__ __forceinline__ void make(const uint32_t x[4], const float r[4], float hp,
                                              uint32_t w[N]) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const float xv = __uint_as_float(x[g]);
      w[g] = __float_as_uint(HAS_H ? add_rn(xv, mul_rn(r[g], hp)) : xv);
    }
  }
  static __device__ __forceinline__ void get(const uint32_t w[N], float p[4]) {
#pragma unroll
    for (int g = 0; g < 4; ++g) p[g] = __uint_as_float(w[g]);
  }
};

// One frozen-gate pass over a tile of W waves x L steps x 64 channels.  Each
// lane owns one channel; its L steps are read once (pass 1, which builds the
// lane aggregate), kept in registers through the look-back, and replayed from
// the true carry in pass 2, which writes the trajectory.
template <typename TX, int L, int W, bool HAS_H, bool FULL_OUT, bool DET, bool PK>
__global__ __launch_bounds__(64 * W) void slstm_frozen_kernel(
    const TX* __restrict__ wx, const TX* __restrict__ rmix, const TX* __restrict__ h0,
    const TX* __restrict__ hsrc, TX* __restrict__ out_full, TX* __restrict__ out_h, int B, int T,
    int d, int n_cb, float eps, int* __restrict__ counter, unsigned long long* __restrict__ agg,
    unsigned long long* __restrict__ incl, int epoch, Spin spin, Packed pk) {
  constexpr int KP = 2;  // predecessors per wave per look-back round
  using Stash = PreStash<TX>;
  constexpr uint32_t SZ = sizeof(TX);
  __shared__ float s_agg[W][4][kCB];
  __shared__ float s_carry[W][3][kCB];
  __shared__ LookbackShared<FrozenMonoid, W * KP> s_lb;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int tile = take_ticket(counter);
  const TileId id = decode_tile(tile, B, n_cb);
  const int c0 = id.cb * kCB;
  const bool live = c0 + lane < d;
  const int t0 = id.chunk * (W * L) + wave * L;
  const int n_steps = max(0, min(L, T - t0));
  const size_t row4 = static_cast<size_t>(4) * d;
  const size_t first = static_cast<size_t>(id.b) * T + t0;  // first (b, t) row of the wave
  const uint32_t voff = live ? lane * SZ : kOOB;
  const uint32_t slot = d * SZ;  // bytes between the slots of a (b, t, 4d) row
  // Bytes from the wave's base to the end of its last live element.
  const uint32_t span4 = n_steps > 0 ? ((n_steps - 1) * row4 + 3 * d + (d - c0)) * SZ : 0;
  const uint32_t span1 = n_steps > 0 ? ((n_steps - 1) * static_cast<size_t>(d) + (d - c0)) * SZ : 0;

  float r[4] = {0.f, 0.f, 0.f, 0.f};
  float hp0 = 0.f;  // h_prev of the wave's first step
  if (HAS_H && live) {
#pragma unroll
    for (int g = 0; g < 4; ++g) r[g] = ld(rmix + g * d + c0 + lane);
    if (t0 > 0 && n_steps > 0)
      hp0 = ld(hsrc + (first - 1) * d + c0 + lane);
    else if (t0 == 0 && h0 != nullptr)
      hp0 = ld(h0 + static_cast<size_t>(id.b) * row4 + 3 * d + c0 + lane);
  }

  // Packed sequences: heads among this wave's steps (see Packed); a head
  // restarts the state from its sequence's initial one.
  Heads hd{0ull, 0};
  if constexpr (PK) hd = find_heads(pk, t0, n_steps);
  auto head_of = [&](int s, float st[4]) { head_state(pk, h0, hd.seq(s), d, c0 + lane, live, st); };

  // Pass 1: read the steps, stash the pre-activations, and fold the segment
  // aggregate from the empty state (m = -inf, n = c = 0).
  uint32_t stash[L][Stash::N];
  FG a = fg_identity();
  {
    const rsrc_t rx = make_rsrc(wx + first * row4 + c0, span4);
    const rsrc_t rh = make_rsrc(HAS_H ? hsrc + first * d + c0 : nullptr, HAS_H ? span1 : 0);
    auto step = [&](int s, auto chk) {
      constexpr bool CHECK = decltype(chk)::value;
      const bool head = CHECK && hd.at(s);
      float hs[4];
      if (head) head_of(s, hs);
      uint32_t x[4];
#pragma unroll
      for (int g = 0; g < 4; ++g)
        x[g] = ldb_bits(static_cast<TX*>(nullptr), rx, voff, s * row4 * SZ + g * slot);
      float hp = hp0;
      if (HAS_H && s > 0) hp = ldb<TX>(rh, voff, (s - 1) * d * SZ);
      if (head) hp = hs[3];
      Stash::template make<HAS_H>(x, r, hp, stash[s]);
      float p[4];
      Stash::get(stash[s], p);
      if (head) a = FG{-INFINITY, hs[2], hs[1], hs[0]};
      a.F += p[1];
      fg_step(p[0], p[1], p[2], a.M, a.N, a.C);
    };
    // Whole segments run branch-free so the loads of many steps are in
    // flight together; only the last segment of a sequence is guarded.
    auto run = [&](auto chk) {
      if (n_steps == L) {
#pragma unroll
        for (int s = 0; s < L; ++s) step(s, chk);
      } else {
#pragma unroll
        for (int s = 0; s < L; ++s)
          if (s < n_steps) step(s, chk);
      }
    };
    if (PK && hd.mask)
      run(std::true_type{});
    else
      run(std::false_type{});
  }
  s_agg[wave][0][lane] = a.F;
  s_agg[wave][1][lane] = a.M;
  s_agg[wave][2][lane] = a.N;
  s_agg[wave][3][lane] = a.C;
  __syncthreads();

  float carry[3] = {0.f, 0.f, 0.f};  // (m, n, c) into the tile, wave 0
  FG tile_agg = fg_identity();
  if (wave == 0) {
#pragma unroll
    for (int w = 0; w < W; ++w)
      tile_agg = fg_compose(
          tile_agg, FG{s_agg[w][0][lane], s_agg[w][1][lane], s_agg[w][2][lane], s_agg[w][3][lane]});
    if (id.chunk == 0) {
      if (!PK && h0 != nullptr && live) {
        const TX* hb = h0 + static_cast<size_t>(id.b) * row4 + c0 + lane;
        carry[2] = ld(hb);
        carry[1] = ld(hb + d);
        carry[0] = ld(hb + 2 * d);
      }
    } else {
      unsigned long long* ap = agg + (static_cast<size_t>(tile) * 4) * kCB + lane;
      st_tagged(ap + 0 * kCB, tile_agg.F, epoch);
      st_tagged(ap + 1 * kCB, tile_agg.M, epoch);
      st_tagged(ap + 2 * kCB, tile_agg.N, epoch);
      st_tagged(ap + 3 * kCB, tile_agg.C, epoch);
    }
  }
  if (id.chunk > 0)
    windowed_lookback<FrozenMonoid, W, KP, DET>(
          id, B, n_cb, epoch, incl, agg, lane, wave, s_lb, carry, spin);
  if (wave == 0) {
    // Per-wave carries, then the tile's inclusive carry: the published
    // aggregate applied to the carry in (what a successor's walk computes).
    float m = carry[0], n = carry[1], c = carry[2];
#pragma unroll
    for (int w = 0; w < W; ++w) {
      s_carry[w][0][lane] = m;
      s_carry[w][1][lane] = n;
      s_carry[w][2][lane] = c;
      fg_apply(FG{s_agg[w][0][lane], s_agg[w][1][lane], s_agg[w][2][lane], s_agg[w][3][lane]}, m,
               n, c);
    }
    if (DET && id.chunk > 0) {
      m = carry[0];
      n = carry[1];
      c = carry[2];
      fg_apply(tile_agg, m, n, c);
    }
    unsigned long long* ip = incl + (static_cast<size_t>(tile) * 3) * kCB + lane;
    st_tagged(ip, m, epoch);
    st_tagged(ip + kCB, n, epoch);
    st_tagged(ip + 2 * kCB, c, epoch);
  }
  __syncthreads();

  // Pass 2: replay the stashed steps from the true carry and write the
  // trajectory (dead lanes' stores fall outside the resources).
  float m = s_carry[wave][0][lane], n = s_carry[wave][1][lane], c = s_carry[wave][2][lane];
  const rsrc_t ro = FULL_OUT ? make_rsrc(out_full + first * row4 + c0, span4)
                             : make_rsrc(out_h + first * d + c0, span1);
  auto replay = [&](int s, auto chk) {
    constexpr bool CHECK = decltype(chk)::value;
    if (CHECK && hd.at(s)) {
      float hs[4];
      head_of(s, hs);
      c = hs[0];
      n = hs[1];
      m = hs[2];
    }
    float p[4];
    Stash::get(stash[s], p);
    fg_step(p[0], p[1], p[2], m, n, c);
    // h = sigmoid(z_o) c / (n + eps) with one reciprocal.
    const float h = c * frcp((1.f + fexp(-p[3])) * (n + eps));
    if (FULL_OUT) {
      const uint32_t so = s * row4 * SZ;
      stb<TX>(ro, voff, so, c);
      stb<TX>(ro, voff, so + slot, n);
      stb<TX>(ro, voff, so + 2 * slot, m);
      stb<TX>(ro, voff, so + 3 * slot, h);
    } else {
      stb<TX>(ro, voff, s * d * SZ, h);
    }
  };
  auto run2 = [&](auto chk) {
    if (n_steps == L) {
#pragma unroll
      for (int s = 0; s < L; ++s) replay(s, chk);
    } else {
#pragma unroll
      for (int s = 0; s < L; ++s)
        if (s < n_steps) replay(s, chk);
    }
  };
  if (PK && hd.mask)
    run2(std::true_type{});
  else
    run2(std::false_type{});
}

// ---------------------------------------------------------------------------
// (1b) all frozen-gate passes in one launch (16-bit storage: bf16 or fp16)
// ---------------------------------------------------------------------------
//
// Pass p of the Picard warm start freezes the gates at wx + R * h_{p-1}[t-1]
// (h_{p-1} the readout of pass p - 1, rounded to the storage type as the reference keeps
// it in the tensor dtype).  Each tile runs stage p = 0 .. P over its own
// steps with wx, the stage's pre-activations and its h trajectory held in
// registers; only the last stage writes the state.  Stage p of a tile needs
//  * h_{p-1} at the step before the tile: the predecessor tile publishes the
//    h of its last step after each stage (tagged word, stage-indexed);
//  * the stage-p carry: a decoupled look-back on stage-indexed tagged words.
// Both only ever wait on tiles with earlier tickets (already resident or
// done), so every wave reaches the end.
template <typename TN, int L, int W, int WPE, bool DET, bool PK>
__global__ __launch_bounds__(64 * W) __attribute__((amdgpu_waves_per_eu(WPE))) void
slstm_picard_fused_kernel(
    const TN* __restrict__ wx, const TN* __restrict__ rmix, const TN* __restrict__ h0,
    TN* __restrict__ out, int B, int T, int d, int n_cb, int n_tiles, int P, float eps,
    int* __restrict__ counter, unsigned long long* __restrict__ agg,
    unsigned long long* __restrict__ incl, unsigned long long* __restrict__ hlast, int tag_base,
    Spin spin, Packed pk) {
  static_assert(L % 2 == 0, "h is packed two steps to a register");
  static_assert(sizeof(TN) == 2, "16-bit storage");
  using NT = Narrow<TN>;
  // one predecessor per wave and look-back round: measured 4% faster than
  // two at config 3, with a quarter less polled traffic (22 against 29 B of
  // reads per element).  The deterministic walk, which must find an
  // inclusive carry inside its window, keeps two.
  constexpr int KP = DET ? 2 : 1;
  constexpr uint32_t SZ = 2;
  __shared__ float s_agg[W][4][kCB];
  __shared__ float s_carry[W][3][kCB];
  __shared__ float s_hl[W][kCB];
  __shared__ float s_tagg[4][kCB];  // the published tile aggregate (wave 0's lanes)
  // tanh(z_z) of the stage's steps: pass 1 evaluates it, pass 2 reads it back
  // (it does not depend on the carry; a transcendental pair per step saved)
  __shared__ float s_z[W][L][kCB];
  __shared__ LookbackShared<FrozenMonoid, W * KP> s_lb;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int tile = take_ticket(counter);
  const TileId id = decode_tile(tile, B, n_cb);
  const int c0 = id.cb * kCB;
  const bool live = c0 + lane < d;
  const int t0 = id.chunk * (W * L) + wave * L;
  const int n_steps = max(0, min(L, T - t0));
  const size_t row4 = static_cast<size_t>(4) * d;
  const size_t first = static_cast<size_t>(id.b) * T + t0;
  const uint32_t voff = live ? lane * SZ : kOOB;
  const uint32_t slot = d * SZ;
  const uint32_t span4 = n_steps > 0 ? ((n_steps - 1) * row4 + 3 * d + (d - c0)) * SZ : 0;
  const size_t stage_incl = static_cast<size_t>(n_tiles) * 3 * kCB;
  const size_t stage_agg = static_cast<size_t>(n_tiles) * 4 * kCB;
  const size_t stage_h = static_cast<size_t>(n_tiles) * kCB;

  float r[4] = {0.f, 0.f, 0.f, 0.f};
  float h0h = 0.f;  // h_prev at t = 0 in every pass
  float c_init[3] = {0.f, 0.f, 0.f};  // (m, n, c) carry into time 0
  if (live) {
#pragma unroll
    for (int g = 0; g < 4; ++g) r[g] = ld(rmix + g * d + c0 + lane);
    if (h0 != nullptr) {
      const TN* hb = h0 + static_cast<size_t>(id.b) * row4 + c0 + lane;
      c_init[2] = ld(hb);
      c_init[1] = ld(hb + d);
      c_init[0] = ld(hb + 2 * d);
      h0h = ld(hb + 3 * d);
    }
  }

  // Packed sequences: heads among this wave's steps and the initial state
  // (c, n, m, h) of the first one's sequence (see Packed); a head restarts
  // the frozen-gate state from it in every stage.
  Heads hd_all{0ull, 0};
  if constexpr (PK) {
    c_init[0] = c_init[1] = c_init[2] = 0.f;
    h0h = 0.f;
    hd_all = find_heads(pk, t0, n_steps);
  }

  uint32_t xw[L][2], pre[L][2], hh[L / 2];
  {
    const rsrc_t rx = make_rsrc(wx + first * row4 + c0, span4);
    auto load = [&](int s) {
      uint32_t v[4];
#pragma unroll
      for (int g = 0; g < 4; ++g)
        v[g] = __builtin_amdgcn_raw_buffer_load_b16(rx, voff, s * row4 * SZ + g * slot, 0);
      xw[s][0] = v[0] | (v[1] << 16);
      xw[s][1] = v[2] | (v[3] << 16);
    };
    if (n_steps == L) {
#pragma unroll
      for (int s = 0; s < L; ++s) load(s);
    } else {
#pragma unroll
      for (int s = 0; s < L; ++s) {
        if (s < n_steps) {
          load(s);
        } else {
          // steps past the end run unguarded in packed streams: defined zeros
          xw[s][0] = xw[s][1] = 0u;
        }
      }
    }
  }
  const rsrc_t ro = make_rsrc(out + first * row4 + c0, span4);

  // Stage P, which writes the state, is compiled separately from the others
  // (no per-step branch between storing the state and keeping h).
  auto stage = [&](const int p, auto last_c) __attribute__((always_inline)) {
    constexpr bool last_stage = decltype(last_c)::value;
    const bool first_stage = p == 0;
    // Packed streams: the head flags re-enter each stage through an opaque
    // copy, so what the steps derive from them (flags, sequence numbers,
    // rows) is computed per stage where it is used instead of being hoisted
    // out of the stage loop into scalar registers for all L steps at once;
    // and the steps run one unguarded, head-checked loop (a single copy of
    // the unrolled stage body).  Only the stream's last tile has steps past
    // the end: they read zeros, their stores fall outside the output's
    // buffer range (dropped), and no tile follows the last one, so nothing
    // reads what they produce.
    Heads hd = hd_all;
    if constexpr (PK) {
      uint32_t lo = static_cast<uint32_t>(hd.mask), hi = static_cast<uint32_t>(hd.mask >> 32);
      int q0 = hd.seq0;
      asm volatile("" : "+v"(lo), "+v"(hi), "+v"(q0));
      lo = __builtin_amdgcn_readfirstlane(lo);
      hi = __builtin_amdgcn_readfirstlane(hi);
      hd.seq0 = __builtin_amdgcn_readfirstlane(q0);
      hd.mask = (static_cast<uint64_t>(hi) << 32) | lo;
    }
    int ns = n_steps;
    if constexpr (PK) {
      asm volatile("" : "+v"(ns));
      ns = __builtin_amdgcn_readfirstlane(ns);
    }
    auto head_of = [&](int s, float st[4]) {
      head_state(pk, h0, hd.seq(s), d, c0 + lane, live, st);
    };
    auto head_h = [&](int s) {
      float st[4];
      head_of(s, st);
      return st[3];
    };
    const int tag = tag_base + p + 1;
    // Keep wx packed across stages: without this the compiler hoists the
    // 16-bit unpacking out of the stage loop and holds 4 floats per step.
#pragma unroll
    for (int s = 0; s < L; ++s) asm volatile("" : "+v"(xw[s][0]), "+v"(xw[s][1]));
    // h_{p-1} at t0 - 1.
    float hp0 = 0.f;
    if (!first_stage) {
      if (PK && hd.at(0)) {
        float hs[4];
        head_of(0, hs);
        hp0 = hs[3];
      } else if (t0 == 0) {
        hp0 = h0h;
      } else if (wave > 0) {
        hp0 = s_hl[wave - 1][lane];
      } else {
        const unsigned long long* hw =
            hlast + (p - 1) * stage_h + (static_cast<size_t>(tile) - B * n_cb) * kCB + lane;
        int spins = 0;
        bool gave_up = false;
        while (true) {
          const bool ok = ld_tagged(hw, tag - 1, hp0);
          if (__ballot(!ok) == 0ull) break;
          if (++spins > 8) {
            if (spins > spin.limit) {  // give up (see Spin)
              spin_give_up(spin);
              gave_up = true;
              break;
            }
            __builtin_amdgcn_s_sleep(8);
          } else {
            __builtin_amdgcn_s_sleep(1);
          }
        }
        if (gave_up) hp0 = __builtin_nanf("");
      }
    }

    // Pass 1: this stage's pre-activations and the segment aggregate.
    FG a = fg_identity();
    auto step1 = [&](int s, auto chk) {
      constexpr bool CHECK = decltype(chk)::value;
      const bool head = CHECK && hd.at(s);
      if (first_stage) {
        pre[s][0] = xw[s][0];
        pre[s][1] = xw[s][1];
      } else {
        float hp =
            s == 0 ? hp0 : ((s - 1) & 1 ? NT::hi(hh[(s - 1) >> 1]) : NT::lo(hh[(s - 1) >> 1]));
        if (head) hp = head_h(s);
#pragma unroll
        for (int k = 0; k < 2; ++k) {
          // round(R h) and round(wx + round(R h)), two gates per conversion.
          const uint32_t q = NT::pack(r[2 * k] * hp, r[2 * k + 1] * hp);
          pre[s][k] = NT::pack(NT::lo(xw[s][k]) + NT::lo(q), NT::hi(xw[s][k]) + NT::hi(q));
        }
      }
      const float zi = NT::lo(pre[s][0]), zf = NT::hi(pre[s][0]), zz = NT::lo(pre[s][1]);
      // a head: the segment so far no longer matters (F = -inf), the state
      // restarts from the sequence's initial one
      if (head) {
        float hs[4];
        head_of(s, hs);
        a = FG{-INFINITY, hs[2], hs[1], hs[0]};
      }
      a.F += zf;
      const float z = ftanh(zz);
      s_z[wave][s][lane] = z;
      fg_step_z(zi, zf, z, a.M, a.N, a.C);
    };
    auto run1 = [&](auto chk) {
      if (PK || ns == L) {
#pragma unroll
        for (int s = 0; s < L; ++s) step1(s, chk);
      } else {
#pragma unroll
        for (int s = 0; s < L; ++s)
          if (s < ns) step1(s, chk);
      }
    };
    // Packed streams: a wave whose steps hold no sequence head runs pass 1
    // without the per-step head checks (1.90 -> 1.80 ms for a 130k-step
    // stream of 64 sequences at d = 1024).  Pass 2 keeps the one checked
    // copy: a second copy there spilled.
    if constexpr (PK) {
      if (hd.mask == 0ull)
        run1(std::false_type{});
      else
        run1(std::true_type{});
    } else {
      run1(std::false_type{});
    }
    s_agg[wave][0][lane] = a.F;
    s_agg[wave][1][lane] = a.M;
    s_agg[wave][2][lane] = a.N;
    s_agg[wave][3][lane] = a.C;
    // Hold pre packed through the look-back: pass 2 unpacks it again rather
    // than the compiler keeping four floats per step alive.
#pragma unroll
    for (int s = 0; s < L; ++s) asm volatile("" : "+v"(pre[s][0]), "+v"(pre[s][1]));
    __syncthreads();

    unsigned long long* incl_p = incl + p * stage_incl;
    unsigned long long* agg_p = agg + p * stage_agg;
    float carry[3] = {0.f, 0.f, 0.f};
    if (wave == 0) {
      FG tile_agg = fg_identity();
#pragma unroll
      for (int w = 0; w < W; ++w)
        tile_agg = fg_compose(tile_agg, FG{s_agg[w][0][lane], s_agg[w][1][lane],
                                           s_agg[w][2][lane], s_agg[w][3][lane]});
      if (id.chunk == 0) {
        carry[0] = c_init[0];
        carry[1] = c_init[1];
        carry[2] = c_init[2];
      } else {
        unsigned long long* ap = agg_p + (static_cast<size_t>(tile) * 4) * kCB + lane;
        st_tagged(ap + 0 * kCB, tile_agg.F, tag);
        st_tagged(ap + 1 * kCB, tile_agg.M, tag);
        st_tagged(ap + 2 * kCB, tile_agg.N, tag);
        st_tagged(ap + 3 * kCB, tile_agg.C, tag);
        if (DET) {
          s_tagg[0][lane] = tile_agg.F;
          s_tagg[1][lane] = tile_agg.M;
          s_tagg[2][lane] = tile_agg.N;
          s_tagg[3][lane] = tile_agg.C;
        }
      }
    }
    if (id.chunk > 0)
      windowed_lookback<FrozenMonoid, W, KP, DET>(
          id, B, n_cb, tag, incl_p, agg_p, lane, wave, s_lb, carry, spin);
    if (wave == 0) {
      float m = carry[0], n = carry[1], c = carry[2];
#pragma unroll
      for (int w = 0; w < W; ++w) {
        s_carry[w][0][lane] = m;
        s_carry[w][1][lane] = n;
        s_carry[w][2][lane] = c;
        fg_apply(FG{s_agg[w][0][lane], s_agg[w][1][lane], s_agg[w][2][lane], s_agg[w][3][lane]},
                 m, n, c);
      }
      if (DET && id.chunk > 0) {
        m = carry[0];
        n = carry[1];
        c = carry[2];
        fg_apply(FG{s_tagg[0][lane], s_tagg[1][lane], s_tagg[2][lane], s_tagg[3][lane]}, m, n, c);
      }
      unsigned long long* ip = incl_p + (static_cast<size_t>(tile) * 3) * kCB + lane;
      st_tagged(ip, m, tag);
      st_tagged(ip + kCB, n, tag);
      st_tagged(ip + 2 * kCB, c, tag);
    }
    __syncthreads();

    // Pass 2: replay from the true carry; h (storage type) stays in registers, the
    // last stage writes the state.
    float m = s_carry[wave][0][lane], n = s_carry[wave][1][lane], c = s_carry[wave][2][lane];
    float h_even = 0.f, h_last = 0.f;
    auto step2 = [&](int s, auto chk) {
      constexpr bool CHECK = decltype(chk)::value;
      if (CHECK && hd.at(s)) {
        float hs[4];
        head_of(s, hs);
        c = hs[0];
        n = hs[1];
        m = hs[2];
      }
      const float zi = NT::lo(pre[s][0]), zf = NT::hi(pre[s][0]);
      const float zo = NT::hi(pre[s][1]);
      fg_step_z(zi, zf, s_z[wave][s][lane], m, n, c);
      const float h = c * frcp((1.f + fexp(-zo)) * (n + eps));
      if constexpr (last_stage) {
        const uint32_t so = s * row4 * SZ;
        stb<TN>(ro, voff, so, c);
        stb<TN>(ro, voff, so + slot, n);
        stb<TN>(ro, voff, so + 2 * slot, m);
        stb<TN>(ro, voff, so + 3 * slot, h);
      } else if (s & 1) {
        hh[s >> 1] = NT::pack(h_even, h);
        h_last = NT::hi(hh[s >> 1]);
      } else {
        h_even = h;
        hh[s >> 1] = NT::pack(h, h);
        h_last = NT::lo(hh[s >> 1]);
      }
    };
    auto run2 = [&](auto chk) {
      if (PK || ns == L) {
#pragma unroll
        for (int s = 0; s < L; ++s) step2(s, chk);
      } else {
#pragma unroll
        for (int s = 0; s < L; ++s)
          if (s < ns) step2(s, chk);
      }
    };
    if constexpr (PK)
      run2(std::true_type{});
    else
      run2(std::false_type{});
    if constexpr (!last_stage) {
      s_hl[wave][lane] = h_last;
      if (wave == W - 1)
        st_tagged(hlast + p * stage_h + static_cast<size_t>(tile) * kCB + lane, h_last, tag);
    }
    __syncthreads();
  };
  for (int p = 0; p < P; ++p) stage(p, std::false_type{});
  stage(P, std::true_type{});
}

// ---------------------------------------------------------------------------
// (2) Newton iteration
// ---------------------------------------------------------------------------

// One Newton iteration over a tile of W waves x L steps x 64 channels.  Pass 1
// reads each step once (wx and the guess, kept in registers) and folds the
// lane's affine aggregate x -> J x + F; pass 2 replays the steps from the true
// carry, delta_t = J_t delta_{t-1} + F_t, and writes H + omega delta.
//
// EAGER (scan_backend='eager'): the step's cell and Jacobian round like the
// reference's eager tensor ops in the storage dtype TX (cell_jac_eager), the
// residual F = pred - H is rounded to TX, the scan runs in fp32 on those
// values, and the update rounds delta to TX before H + omega delta is rounded
// again (solvers/newton/__init__.py:516-543).  Pass 2 re-forms J instead of
// the forward-mode replay so that it applies exactly the rounded entries.
template <typename TX, typename TIN, typename TOUT, int L, int W, bool DET, bool PK,
          bool EAGER = false>
__global__ __launch_bounds__(64 * W) void slstm_newton_kernel(
    const TX* __restrict__ wx, const TX* __restrict__ rmix, const TX* __restrict__ h0,
    const TIN* __restrict__ hin, TOUT* __restrict__ hout, int B, int T, int d, int n_cb,
    float omega, float eps, int* __restrict__ counter, unsigned long long* __restrict__ agg,
    unsigned long long* __restrict__ incl, int epoch, Spin spin, Packed pk) {
  // predecessors per wave per look-back round (the deterministic walk, which
  // must find an inclusive carry inside its window, looks twice as far)
  constexpr int KP = DET ? 2 : 1;
  using XS = RowStash<TX>;
  using HS = RowStash<TIN>;
  __shared__ float s_agg[W][20][kCB];
  __shared__ float s_carry[W][4][kCB];
  __shared__ float s_tagg[20][kCB];  // the published tile aggregate (wave 0's lanes)
  __shared__ LookbackShared<NewtonMonoid, W * KP> s_lb;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int tile = take_ticket(counter);
  const TileId id = decode_tile(tile, B, n_cb);
  const int c0 = id.cb * kCB;
  const bool live = c0 + lane < d;
  const int t0 = id.chunk * (W * L) + wave * L;
  const int n_steps = max(0, min(L, T - t0));
  const size_t row4 = static_cast<size_t>(4) * d;
  const size_t first = static_cast<size_t>(id.b) * T + t0;
  // Per-slot byte offsets inside a (b, t, 4d) row for each storage type, and
  // the bytes from the wave's base to its last live element.
  const uint32_t vx = live ? lane * sizeof(TX) : kOOB;
  const uint32_t vi = live ? lane * sizeof(TIN) : kOOB;
  const uint32_t vo = live ? lane * sizeof(TOUT) : kOOB;
  const size_t span = n_steps > 0 ? (n_steps - 1) * row4 + 3 * d + (d - c0) : 0;

  float r[4] = {0.f, 0.f, 0.f, 0.f};
  // Linearisation point H_{t0-1}: previous guess, h0 at t = 0, else zeros.
  float prev0[4] = {0.f, 0.f, 0.f, 0.f};
  if (live) {
#pragma unroll
    for (int g = 0; g < 4; ++g) r[g] = ld(rmix + g * d + c0 + lane);
    if (t0 > 0 && n_steps > 0) {
      const TIN* p = hin + (first - 1) * row4 + c0 + lane;
#pragma unroll
      for (int k = 0; k < 4; ++k) prev0[k] = ld(p + k * d);
    } else if (t0 == 0 && h0 != nullptr) {
      const TX* p = h0 + static_cast<size_t>(id.b) * row4 + c0 + lane;
#pragma unroll
      for (int k = 0; k < 4; ++k) prev0[k] = ld(p + k * d);
    }
  }

  // Packed sequences: heads among this wave's steps (see Packed).
  Heads hd{0ull, 0};
  if constexpr (PK) {
    hd = find_heads(pk, t0, n_steps);
    if (hd.at(0)) head_state(pk, h0, hd.seq(0), d, c0 + lane, live, prev0);
  }
  auto head_prev = [&](int s, float p[4]) { head_state(pk, h0, hd.seq(s), d, c0 + lane, live, p); };

  uint32_t xs[L][XS::N], hs[L][HS::N];
  // Pass 1: lane segment aggregate (A, b) of the affine maps x -> J x + F.
  Aff a;
  aff_identity(a);
  {
    const rsrc_t rx = make_rsrc(wx + first * row4 + c0, span * sizeof(TX));
    const rsrc_t ri = make_rsrc(hin + first * row4 + c0, span * sizeof(TIN));
    float prev[4] = {prev0[0], prev0[1], prev0[2], prev0[3]};
    auto step = [&](int s, auto chk) {
      constexpr bool CHECK = decltype(chk)::value;
      const bool head = CHECK && hd.at(s);
      XS::load(rx, vx, s * row4 * sizeof(TX), d * sizeof(TX), xs[s]);
      HS::load(ri, vi, s * row4 * sizeof(TIN), d * sizeof(TIN), hs[s]);
      if (head && s > 0) head_prev(s, prev);
      float x[4], hv[4];
      XS::get(xs[s], x);
      HS::get(hs[s], hv);
      if constexpr (EAGER) {
        CellJE J = cell_jac_eager<TX>(prev, x, r, eps);
        if (head)
          J.f = J.cm = J.ch = J.nm = J.nh = J.al = J.mh = J.hc = J.hn = J.hm = J.hh = 0.f;
        const float F[4] = {round_to<TX>(J.pc - hv[0]), round_to<TX>(J.pn - hv[1]),
                            round_to<TX>(J.pm - hv[2]), round_to<TX>(J.ph - hv[3])};
        jmv_affine_e(J, F, a.b);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          float col[4] = {a.A[0][j], a.A[1][j], a.A[2][j], a.A[3][j]};
          jmv_e(J, col);
#pragma unroll
          for (int k = 0; k < 4; ++k) a.A[k][j] = col[k];
        }
      } else {
        CellJ J = cell_jac(prev, x, r, eps);
        if (head) J.f = J.cm = J.ch = J.nm = J.nh = J.al = J.mh = J.inv = J.dn = J.g = 0.f;
        const float F[4] = {J.pc - hv[0], J.pn - hv[1], J.pm - hv[2], J.ph - hv[3]};
        jmv_affine(J, F, a.b);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          float col[4] = {a.A[0][j], a.A[1][j], a.A[2][j], a.A[3][j]};
          jmv(J, col);
#pragma unroll
          for (int k = 0; k < 4; ++k) a.A[k][j] = col[k];
        }
      }
#pragma unroll
      for (int k = 0; k < 4; ++k) prev[k] = hv[k];
    };
    auto run = [&](auto chk) {
      if (n_steps == L) {
#pragma unroll
        for (int s = 0; s < L; ++s) step(s, chk);
      } else {
#pragma unroll
        for (int s = 0; s < L; ++s)
          if (s < n_steps) step(s, chk);
      }
    };
    if (PK && hd.mask)
      run(std::true_type{});
    else
      run(std::false_type{});
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    s_agg[wave][16 + i][lane] = a.b[i];
#pragma unroll
    for (int j = 0; j < 4; ++j) s_agg[wave][4 * i + j][lane] = a.A[i][j];
  }
  __syncthreads();

  float carry[4] = {0.f, 0.f, 0.f, 0.f};  // delta into the tile (delta_{-1} = 0), wave 0
  if (wave == 0 && id.chunk > 0) {
    Aff tile_agg;
    aff_identity(tile_agg);
#pragma unroll
    for (int w = 0; w < W; ++w) {
      Aff sw;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        sw.b[i] = s_agg[w][16 + i][lane];
#pragma unroll
        for (int j = 0; j < 4; ++j) sw.A[i][j] = s_agg[w][4 * i + j][lane];
      }
      tile_agg = w == 0 ? sw : aff_compose(tile_agg, sw);
    }
    unsigned long long* ap = agg + (static_cast<size_t>(tile) * 20) * kCB + lane;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (DET) s_tagg[16 + i][lane] = tile_agg.b[i];
      st_tagged(ap + (16 + i) * kCB, tile_agg.b[i], epoch);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (DET) s_tagg[4 * i + j][lane] = tile_agg.A[i][j];
        st_tagged(ap + (4 * i + j) * kCB, tile_agg.A[i][j], epoch);
      }
    }
  }
  if (id.chunk > 0)
    windowed_lookback<NewtonMonoid, W, KP, DET>(
          id, B, n_cb, epoch, incl, agg, lane, wave, s_lb, carry, spin);
  if (wave == 0) {
    // Carry into each wave's segment, then the tile's outgoing carry (the
    // published aggregate applied to the carry in, as a successor's walk
    // would compute it).
#pragma unroll
    for (int w = 0; w < W; ++w) {
#pragma unroll
      for (int k = 0; k < 4; ++k) s_carry[w][k][lane] = carry[k];
      Aff sw;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        sw.b[i] = s_agg[w][16 + i][lane];
#pragma unroll
        for (int j = 0; j < 4; ++j) sw.A[i][j] = s_agg[w][4 * i + j][lane];
      }
      aff_apply(sw, carry);
    }
    if (DET && id.chunk > 0) {
      float a[20];
#pragma unroll
      for (int k = 0; k < 20; ++k) a[k] = s_tagg[k][lane];
#pragma unroll
      for (int k = 0; k < 4; ++k) carry[k] = s_carry[0][k][lane];
      NewtonMonoid::apply(a, carry);
    }
    unsigned long long* ip = incl + (static_cast<size_t>(tile) * 4) * kCB + lane;
#pragma unroll
    for (int k = 0; k < 4; ++k) st_tagged(ip + k * kCB, carry[k], epoch);
  }
  __syncthreads();

  // Pass 2: delta_t = J_t delta_{t-1} + F_t from the true carry; H += omega delta.
  float dl[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) dl[k] = s_carry[wave][k][lane];
  {
    const rsrc_t ro = make_rsrc(hout + first * row4 + c0, span * sizeof(TOUT));
    float prev[4] = {prev0[0], prev0[1], prev0[2], prev0[3]};
    auto replay = [&](int s, auto chk) {
      constexpr bool CHECK = decltype(chk)::value;
      if (CHECK && hd.at(s)) {
        if (s > 0) head_prev(s, prev);
#pragma unroll
        for (int k = 0; k < 4; ++k) dl[k] = 0.f;
      }
      float x[4], hv[4];
      XS::get(xs[s], x);
      HS::get(hs[s], hv);
      const uint32_t so = s * row4 * sizeof(TOUT);
      if constexpr (EAGER) {
        CellJE J = cell_jac_eager<TX>(prev, x, r, eps);
        const float F[4] = {round_to<TX>(J.pc - hv[0]), round_to<TX>(J.pn - hv[1]),
                            round_to<TX>(J.pm - hv[2]), round_to<TX>(J.ph - hv[3])};
        jmv_affine_e(J, F, dl);
#pragma unroll
        for (int k = 0; k < 4; ++k)
          stb<TOUT>(ro, vo, so + k * d * sizeof(TOUT),
                    add_rn(hv[k], mul_rn(omega, round_to<TX>(dl[k]))));
      } else {
        float pv[4], jv[4];
        cell_jvp(prev, x, r, eps, dl, pv, jv);
#pragma unroll
        for (int k = 0; k < 4; ++k) dl[k] = jv[k] + (pv[k] - hv[k]);
#pragma unroll
        for (int k = 0; k < 4; ++k)
          stb<TOUT>(ro, vo, so + k * d * sizeof(TOUT), hv[k] + omega * dl[k]);
      }
#pragma unroll
      for (int k = 0; k < 4; ++k) prev[k] = hv[k];
    };
    auto run = [&](auto chk) {
      if (n_steps == L) {
#pragma unroll
        for (int s = 0; s < L; ++s) replay(s, chk);
      } else {
#pragma unroll
        for (int s = 0; s < L; ++s)
          if (s < n_steps) replay(s, chk);
      }
    };
    if (PK && hd.mask)
      run(std::true_type{});
    else
      run(std::false_type{});
  }
}


// ---------------------------------------------------------------------------
// (2b) all K Newton iterations in one launch
// ---------------------------------------------------------------------------
//
// Each tile runs iterations k = 1 .. K over its own steps with wx and the fp32
// iterate H^(k-1) held in registers; only the last iteration writes the state.
// Iteration k of a tile needs
//  * H^(k-1) at the step before the tile: the predecessor tile publishes the
//    4 slots of its last step after each iteration (tagged words,
//    iteration-indexed); waves of one tile hand it over through LDS;
//  * the iteration-k carry: a decoupled look-back on iteration-indexed words.
// Both only ever wait on tiles with earlier tickets, so every wave reaches the
// end.  The arithmetic is that of K separate launches exchanging the fp32
// iterate through memory.
template <typename TX, int L, int W, int WPE, bool DET, bool PK>
__global__ __launch_bounds__(64 * W) __attribute__((amdgpu_waves_per_eu(WPE))) void
slstm_newton_fused_kernel(
    const TX* __restrict__ wx, const TX* __restrict__ rmix, const TX* __restrict__ h0,
    const TX* __restrict__ guess, TX* __restrict__ out, int B, int T, int d, int n_cb,
    int n_tiles, int K, float omega, float eps, int* __restrict__ counter,
    unsigned long long* __restrict__ agg, unsigned long long* __restrict__ incl,
    unsigned long long* __restrict__ hlast, int tag_base, Spin spin, Packed pk) {
  // predecessors per wave per look-back round, in both modes: a window of 8
  // (20 KB more LDS) would leave one block per CU beside the tanh cache.  The
  // deterministic walk waits for an inclusive carry inside its window; its
  // result does not depend on the window.
  constexpr int KP = 1;
  using XS = RowStash<TX>;
  __shared__ float s_agg[W][20][kCB];
  __shared__ float s_carry[W][4][kCB];
  __shared__ float s_tagg[20][kCB];  // the published tile aggregate (wave 0's lanes)
  __shared__ float s_hl[W][4][kCB];
  // z = tanh(z_z) of the iteration's steps: pass 1 evaluates it at the
  // linearisation point, pass 2 (same point) reads it back
  __shared__ float s_z[W][L][kCB];
  __shared__ LookbackShared<NewtonMonoid, W * KP> s_lb;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int tile = take_ticket(counter);
  const TileId id = decode_tile(tile, B, n_cb);
  const int c0 = id.cb * kCB;
  const bool live = c0 + lane < d;
  const int t0 = id.chunk * (W * L) + wave * L;
  const int n_steps = max(0, min(L, T - t0));
  const size_t row4 = static_cast<size_t>(4) * d;
  const size_t first = static_cast<size_t>(id.b) * T + t0;
  const uint32_t vx = live ? lane * sizeof(TX) : kOOB;
  const size_t span = n_steps > 0 ? (n_steps - 1) * row4 + 3 * d + (d - c0) : 0;
  const size_t stage_incl = static_cast<size_t>(n_tiles) * 4 * kCB;
  const size_t stage_agg = static_cast<size_t>(n_tiles) * 20 * kCB;
  const size_t stage_h = static_cast<size_t>(n_tiles) * 4 * kCB;

  float r[4] = {0.f, 0.f, 0.f, 0.f};
  float h0v[4] = {0.f, 0.f, 0.f, 0.f};   // linearisation point at t = 0, every iteration
  float prevg[4] = {0.f, 0.f, 0.f, 0.f};  // the guess at t0 - 1 (iteration 1)
  if (live) {
#pragma unroll
    for (int g = 0; g < 4; ++g) r[g] = ld(rmix + g * d + c0 + lane);
    if (h0 != nullptr) {
      const TX* p = h0 + static_cast<size_t>(id.b) * row4 + c0 + lane;
#pragma unroll
      for (int k = 0; k < 4; ++k) h0v[k] = ld(p + k * d);
    }
    if (t0 > 0 && n_steps > 0) {
      const TX* p = guess + (first - 1) * row4 + c0 + lane;
#pragma unroll
      for (int k = 0; k < 4; ++k) prevg[k] = ld(p + k * d);
    }
  }
  if (t0 == 0) {
#pragma unroll
    for (int k = 0; k < 4; ++k) prevg[k] = h0v[k];
  }
  // Packed sequences: the heads among this wave's steps, and the initial
  // state of the first one's sequence (later heads of the wave load theirs
  // when they come).
  Heads hd_all{0ull, 0};
  if constexpr (PK) hd_all = find_heads(pk, t0, n_steps);

  uint32_t xs[L][XS::N];
  float hf[L][4];
  {
    const rsrc_t rx = make_rsrc(wx + first * row4 + c0, span * sizeof(TX));
    const rsrc_t rg = make_rsrc(guess + first * row4 + c0, span * sizeof(TX));
    auto load = [&](int s) {
      uint32_t gw[XS::N];
      XS::load(rx, vx, s * row4 * sizeof(TX), d * sizeof(TX), xs[s]);
      XS::load(rg, vx, s * row4 * sizeof(TX), d * sizeof(TX), gw);
      XS::get(gw, hf[s]);
    };
    if (n_steps == L) {
#pragma unroll
      for (int s = 0; s < L; ++s) load(s);
    } else {
#pragma unroll
      for (int s = 0; s < L; ++s) {
        if (s < n_steps) {
          load(s);
        } else {
          // steps past the end run unguarded in packed streams: defined zeros
#pragma unroll
          for (int q = 0; q < XS::N; ++q) xs[s][q] = 0u;
#pragma unroll
          for (int j = 0; j < 4; ++j) hf[s][j] = 0.f;
        }
      }
    }
  }
  const rsrc_t ro = make_rsrc(out + first * row4 + c0, span * sizeof(TX));

  // Iterations 1 .. K-1 keep the new iterate in registers; the last one,
  // compiled separately, writes it (no per-step branch on the iteration).
  auto iterate = [&](const int k, auto last_c) __attribute__((always_inline)) {
    // Packed streams: the head flags re-enter each iteration through an
    // opaque copy (what the steps derive from them is computed where it is
    // used, not hoisted out of the iteration loop into scalar registers for
    // all L steps), and the steps run one unguarded, head-checked loop (a
    // single copy of the unrolled iteration body; steps past the end of the
    // stream's last tile are harmless, as in the warm start).
    Heads hd = hd_all;
    int ns = n_steps;
    if constexpr (PK) {
      uint32_t lo = static_cast<uint32_t>(hd.mask), hi = static_cast<uint32_t>(hd.mask >> 32);
      int q0 = hd.seq0;
      asm volatile("" : "+v"(lo), "+v"(hi), "+v"(q0), "+v"(ns));
      hd.mask = (static_cast<uint64_t>(__builtin_amdgcn_readfirstlane(hi)) << 32) |
                __builtin_amdgcn_readfirstlane(lo);
      hd.seq0 = __builtin_amdgcn_readfirstlane(q0);
      ns = __builtin_amdgcn_readfirstlane(ns);
    }
    auto head_prev = [&](int s, float p[4]) {
      head_state(pk, h0, hd.seq(s), d, c0 + lane, live, p);
    };
    constexpr bool last_iter = decltype(last_c)::value;
    const int tag = tag_base + k + 1;
    // Keep wx packed across iterations (otherwise the unpacking is hoisted out
    // of the loop and holds 4 floats per step).
#pragma unroll
    for (int s = 0; s < L; ++s)
#pragma unroll
      for (int q = 0; q < XS::N; ++q) asm volatile("" : "+v"(xs[s][q]));
    // Linearisation point H^(k-1)_{t0-1}.
    float prev0[4];
    if (PK && hd.at(0)) {
      head_prev(0, prev0);
    } else if (k == 0 || t0 == 0) {
#pragma unroll
      for (int j = 0; j < 4; ++j) prev0[j] = prevg[j];
      if (k > 0) {
#pragma unroll
        for (int j = 0; j < 4; ++j) prev0[j] = h0v[j];
      }
    } else if (wave > 0) {
#pragma unroll
      for (int j = 0; j < 4; ++j) prev0[j] = s_hl[wave - 1][j][lane];
    } else {
      const unsigned long long* hw =
          hlast + (k - 1) * stage_h + (static_cast<size_t>(tile) - B * n_cb) * 4 * kCB + lane;
      int spins = 0;
      bool gave_up = false;
      while (true) {
        bool ok = true;
#pragma unroll
        for (int j = 0; j < 4; ++j) ok = ld_tagged(hw + j * kCB, tag - 1, prev0[j]) && ok;
        if (__ballot(!ok) == 0ull) break;
        if (++spins > 8) {
          if (spins > spin.limit) {  // give up (see Spin)
            spin_give_up(spin);
            gave_up = true;
            break;
          }
          __builtin_amdgcn_s_sleep(8);
        } else {
          __builtin_amdgcn_s_sleep(1);
        }
      }
      if (gave_up) {
#pragma unroll
        for (int j = 0; j < 4; ++j) prev0[j] = __builtin_nanf("");
      }
    }

    // Pass 1: lane segment aggregate (A, b) of the affine maps x -> J x + F.
    Aff a;
    aff_identity(a);
    {
      float prev[4] = {prev0[0], prev0[1], prev0[2], prev0[3]};
      auto step = [&](int s, auto chk) {
        constexpr bool CHECK = decltype(chk)::value;
        const bool head = CHECK && hd.at(s);
        if (head && s > 0) head_prev(s, prev);
        float x[4];
        XS::get(xs[s], x);
        const float zc = cell_z(prev, x, r);
        s_z[wave][s][lane] = zc;
        const CellJ J = cell_jac_z(prev, x, r, eps, zc);
        const float F[4] = {J.pc - hf[s][0], J.pn - hf[s][1], J.pm - hf[s][2],
                            J.ph - hf[s][3]};
        jmv_affine(J, F, a.b);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          float col[4] = {a.A[0][j], a.A[1][j], a.A[2][j], a.A[3][j]};
          jmv(J, col);
#pragma unroll
          for (int i = 0; i < 4; ++i) a.A[i][j] = col[i];
        }
        if (head) {
          // the scan's map at a head is the constant F: no carry crosses it,
          // so the segment's composition restarts there as (0, F)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            a.b[i] = F[i];
#pragma unroll
            for (int j = 0; j < 4; ++j) a.A[i][j] = 0.f;
          }
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) prev[j] = hf[s][j];
      };
      auto run = [&](auto chk) {
        if (PK || ns == L) {
#pragma unroll
          for (int s = 0; s < L; ++s) step(s, chk);
        } else {
#pragma unroll
          for (int s = 0; s < L; ++s)
            if (s < ns) step(s, chk);
        }
      };
      // as in the warm start: head-free waves skip the per-step checks in
      // pass 1 (pass 2 keeps one checked copy, a second spilled)
      if constexpr (PK) {
        if (hd.mask == 0ull)
          run(std::false_type{});
        else
          run(std::true_type{});
      } else {
        run(std::false_type{});
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      s_agg[wave][16 + i][lane] = a.b[i];
#pragma unroll
      for (int j = 0; j < 4; ++j) s_agg[wave][4 * i + j][lane] = a.A[i][j];
    }
    // Hold wx packed through the look-back: pass 2 unpacks it again.
#pragma unroll
    for (int s = 0; s < L; ++s)
#pragma unroll
      for (int q = 0; q < XS::N; ++q) asm volatile("" : "+v"(xs[s][q]));
    __syncthreads();

    unsigned long long* incl_k = incl + k * stage_incl;
    unsigned long long* agg_k = agg + k * stage_agg;
    float carry[4] = {0.f, 0.f, 0.f, 0.f};
    if (wave == 0 && id.chunk > 0) {
      Aff tile_agg;
      aff_identity(tile_agg);
#pragma unroll
      for (int w = 0; w < W; ++w) {
        Aff sw;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          sw.b[i] = s_agg[w][16 + i][lane];
#pragma unroll
          for (int j = 0; j < 4; ++j) sw.A[i][j] = s_agg[w][4 * i + j][lane];
        }
        tile_agg = w == 0 ? sw : aff_compose(tile_agg, sw);
      }
      unsigned long long* ap = agg_k + (static_cast<size_t>(tile) * 20) * kCB + lane;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (DET) s_tagg[16 + i][lane] = tile_agg.b[i];
        st_tagged(ap + (16 + i) * kCB, tile_agg.b[i], tag);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if (DET) s_tagg[4 * i + j][lane] = tile_agg.A[i][j];
          st_tagged(ap + (4 * i + j) * kCB, tile_agg.A[i][j], tag);
        }
      }
    }
    if (id.chunk > 0)
      windowed_lookback<NewtonMonoid, W, KP, DET>(
          id, B, n_cb, tag, incl_k, agg_k, lane, wave, s_lb, carry, spin);
    if (wave == 0) {
      // Per-wave carries; the outgoing carry is the published aggregate
      // applied to the carry in, as a successor's walk would compute it.
#pragma unroll
      for (int w = 0; w < W; ++w) {
#pragma unroll
        for (int j = 0; j < 4; ++j) s_carry[w][j][lane] = carry[j];
        Aff sw;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          sw.b[i] = s_agg[w][16 + i][lane];
#pragma unroll
          for (int j = 0; j < 4; ++j) sw.A[i][j] = s_agg[w][4 * i + j][lane];
        }
        aff_apply(sw, carry);
      }
      if (DET && id.chunk > 0) {
        float a[20];
#pragma unroll
        for (int k = 0; k < 20; ++k) a[k] = s_tagg[k][lane];
#pragma unroll
        for (int j = 0; j < 4; ++j) carry[j] = s_carry[0][j][lane];
        NewtonMonoid::apply(a, carry);
      }
      unsigned long long* ip = incl_k + (static_cast<size_t>(tile) * 4) * kCB + lane;
#pragma unroll
      for (int j = 0; j < 4; ++j) st_tagged(ip + j * kCB, carry[j], tag);
    }
    __syncthreads();

    // Pass 2: delta_t = J_t delta_{t-1} + F_t from the true carry; the new
    // iterate H + omega delta stays in registers (written by the last one).
    float dl[4], hl[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 4; ++j) dl[j] = s_carry[wave][j][lane];
    {
      float prev[4] = {prev0[0], prev0[1], prev0[2], prev0[3]};
      auto replay = [&](int s, auto chk) {
        constexpr bool CHECK = decltype(chk)::value;
        if (CHECK && hd.at(s)) {
          // a head: previous state h0 of its sequence, no incoming delta
          if (s > 0) head_prev(s, prev);
#pragma unroll
          for (int j = 0; j < 4; ++j) dl[j] = 0.f;
        }
        float x[4], hv[4];
        XS::get(xs[s], x);
#pragma unroll
        for (int j = 0; j < 4; ++j) hv[j] = hf[s][j];
        float pv[4], jv[4];
        cell_jvp_z(prev, x, r, eps, s_z[wave][s][lane], dl, pv, jv);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          dl[j] = jv[j] + (pv[j] - hv[j]);
          hl[j] = hv[j] + omega * dl[j];
          prev[j] = hv[j];
        }
        if constexpr (last_iter) {
          const uint32_t so = s * row4 * sizeof(TX);
#pragma unroll
          for (int j = 0; j < 4; ++j) stb<TX>(ro, vx, so + j * d * sizeof(TX), hl[j]);
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j) hf[s][j] = hl[j];
        }
      };
      auto run = [&](auto chk) {
        if (PK || ns == L) {
#pragma unroll
          for (int s = 0; s < L; ++s) replay(s, chk);
        } else {
#pragma unroll
          for (int s = 0; s < L; ++s)
            if (s < ns) replay(s, chk);
        }
      };
      if constexpr (PK)
        run(std::true_type{});
      else
        run(std::false_type{});
    }
    if constexpr (!last_iter) {
#pragma unroll
      for (int j = 0; j < 4; ++j) s_hl[wave][j][lane] = hl[j];
      if (wave == W - 1) {
        unsigned long long* hw = hlast + k * stage_h + static_cast<size_t>(tile) * 4 * kCB + lane;
#pragma unroll
        for (int j = 0; j < 4; ++j) st_tagged(hw + j * kCB, hl[j], tag);
      }
    }
    __syncthreads();
  };
  for (int k = 0; k < K - 1; ++k) iterate(k, std::false_type{});
  iterate(K - 1, std::true_type{});
}


// ---------------------------------------------------------------------------
// Tile shapes the host code and the packed-stream launches share (L steps per
// lane x W waves; the defaults, also the only shapes of deterministic mode and
// of packed streams).
// ---------------------------------------------------------------------------
constexpr Shape kFrozenDefault{64, 4};
constexpr Shape kFrozenF32{32, 4};
constexpr Shape kNewtonGuessDefault{24, 4};
constexpr Shape kNewtonWorkDefault{24, 4};
constexpr Shape kNewtonF32{16, 8};
constexpr Shape kPicardDefault{24, 4};
constexpr Shape kNewtonFusedDefault{20, 4};
constexpr Shape kNewtonFusedF32{16, 4};

// Packed streams: the fused warm start and Newton launches take the
// rectangular tile lengths (their packed bodies are one guarded, head-checked
// loop: no spills); the single-iteration launches run shorter tiles.
constexpr Shape kPicardPacked{24, 4};
constexpr Shape kFrozenPackedF32{32, 4};
constexpr Shape kNewtonFusedPacked{20, 4};
constexpr Shape kNewtonFusedPackedF32{12, 4};
constexpr Shape kNewtonPackedGuess{16, 4};
constexpr Shape kNewtonPackedWork{16, 4};
constexpr Shape kNewtonPackedF32{8, 8};

// scan_backend='eager' iterations (slstm_newton_kernel<EAGER>, one launch per
// iteration): the op-by-op rounding keeps more values live per step than the
// fused arithmetic, so 16-bit storage takes shorter tiles.  bf16 at d=1024,
// B=8, T=16384: 12x4 (~170 VGPRs) runs an iteration in 3.0 ms against 4.6 ms
// for 24x4 (291 VGPRs, one wave per SIMD); packed streams 8x4 (~228 VGPRs)
// 3.9 ms against 4.6 ms for 16x4 (437 VGPRs).
constexpr Shape kNewtonEager{12, 4};
constexpr Shape kNewtonEagerF32{16, 8};
constexpr Shape kNewtonEagerPacked{8, 4};
constexpr Shape kNewtonEagerPackedF32{8, 8};

// Packed-stream launches (B = 1, default shapes), compiled in their own
// translation unit (slstm_packed.hip).
template <typename TN>
void launch_picard_packed(const TN* wx, const TN* r, const TN* h0, TN* out, int T, int d,
                          int P, float eps, const Lookback& lb, unsigned long long* hlast,
                          hipStream_t stream, const Packed& pk);
void launch_frozen_packed(bool has_h, bool full_out, const float* wx, const float* r,
                          const float* h0, const float* src, float* out_full, float* out_h, int T,
                          int d, float eps, const Lookback& lb, int epoch, hipStream_t stream,
                          const Packed& pk);
template <typename TX>
void launch_newton_fused_packed(const TX* wx, const TX* r, const TX* h0, const TX* guess, TX* out,
                                int T, int d, int K, float omega, float eps, const Lookback& lb,
                                unsigned long long* hlast, hipStream_t stream, const Packed& pk);
template <typename TX, typename TIN, typename TOUT>
void launch_newton_packed(const TX* wx, const TX* r, const TX* h0, const TIN* hin, TOUT* hout,
                          int T, int d, float omega, float eps, const Lookback& lb, int epoch,
                          hipStream_t stream, const Packed& pk);

}  // namespace slstm
}  // namespace prnn
