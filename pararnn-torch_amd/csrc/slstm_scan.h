// Shared pieces of the ParaSLSTM mix='diag' scan kernels (forward Newton and
// Picard passes, and the reverse scan of the backward):
//
// * the tile schedule: tile = (batch b, channel block of 64, time chunk),
//   tiles numbered in scan order by an atomic ticket;
// * the windowed decoupled look-back over earlier tiles of the same
//   (b, channel block);
// * the cell value and its 4x4 per-channel Jacobian, and the affine monoid
//   (A, b) of the Newton and adjoint scans;
// * register stashes of a tile's rows, and the host-side geometry and
//   workspace helpers.
#pragma once

#include "prnn_common.h"
#include "pararnn_amd.h"
#include "prnn_host.h"

#include <stdio.h>
#include <stdlib.h>

#include <type_traits>

namespace prnn {
namespace slstm {

constexpr int kCB = 64;  // channels per tile (one per lane)

struct TileId {
  int b, cb, chunk, rem;
};

__device__ __forceinline__ TileId decode_tile(int tile, int B, int n_cb) {
  const int per = B * n_cb;
  TileId t;
  t.chunk = tile / per;
  t.rem = tile - t.chunk * per;
  t.b = t.rem / n_cb;
  t.cb = t.rem - t.b * n_cb;
  return t;
}

__device__ __forceinline__ int take_ticket(int* counter) {
  __shared__ int s_ticket;
  if (threadIdx.x == 0)
    s_ticket = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  return __builtin_amdgcn_readfirstlane(s_ticket);  // wave-uniform
}


// ---------------------------------------------------------------------------
// Packed sequences (cu_seqlens).
//
// With cu != nullptr a kernel sees one stream (B = 1) of T steps holding S
// sequences, sequence q on steps [cu[q], cu[q+1]) (cu[0] = 0, cu[S] = T).  The
// first step of a sequence is a head: its previous state is the sequence's
// initial state -- row tbl[q] (or q without a table) of h0, zeros without h0
// -- and no carry crosses it (the scan's map there is constant: J = 0).  A
// wave learns once, with scalar loads, which of its steps are heads (a
// wave-uniform bit mask) and which sequence its first step belongs to.
// ---------------------------------------------------------------------------
struct Packed {
  const int* cu;   // S + 1 offsets, or nullptr for a rectangular batch
  const int* tbl;  // S rows of h0, or nullptr (row q)
  int n_seq;
};

struct Heads {
  uint64_t mask;  // bit s: step t0 + s is a head
  int seq0;       // sequence of step t0
  __device__ __forceinline__ bool at(int s) const { return (mask >> s) & 1ull; }
  // sequence of step t0 + s
  __device__ __forceinline__ int seq(int s) const {
    const uint64_t upto = s >= 63 ? ~0ull : ((2ull << s) - 1ull);
    return seq0 + __builtin_popcountll(mask & upto) - static_cast<int>(mask & 1ull);
  }
  __device__ __forceinline__ int first() const { return __builtin_ctzll(mask); }
};

// Heads among steps [t0, t0 + n), n <= 64 (wave-uniform arguments).
__device__ __forceinline__ Heads find_heads(const Packed& pk, int t0, int n) {
  Heads h{0ull, 0};
  if (n <= 0) return h;
  // cu[lo] <= t0 < cu[hi]
  int lo = 0, hi = pk.n_seq;
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (pk.cu[mid] <= t0)
      lo = mid;
    else
      hi = mid;
  }
  h.seq0 = lo;
  if (pk.cu[lo] == t0) h.mask |= 1ull;
  for (int q = hi; q < pk.n_seq; ++q) {
    const int t = pk.cu[q];
    if (t >= t0 + n) break;
    h.mask |= 1ull << (t - t0);
  }
  return h;
}

// The 4 slots (c, n, m, h) of sequence q's initial state for this lane's
// channel (zeros without h0 or on dead lanes).
template <typename TX>
__device__ __forceinline__ void head_state(const Packed& pk, const TX* h0, int q, int d, int ch,
                                           bool live, float st[4]) {
#pragma unroll
  for (int k = 0; k < 4; ++k) st[k] = 0.f;
  if (h0 == nullptr || !live) return;
  const int row = pk.tbl != nullptr ? pk.tbl[q] : q;
  const TX* p = h0 + static_cast<size_t>(row) * 4 * d + ch;
#pragma unroll
  for (int k = 0; k < 4; ++k) st[k] = ld(p + k * d);
}

// ---------------------------------------------------------------------------
// Windowed decoupled look-back.
//
// Called by every wave of a tile with chunk > 0 (it contains barriers).  Each
// lane (channel) keeps its own position; in one round every wave w fetches
// predecessor (position - w) for every lane -- W predecessors per memory round
// trip -- and stages its status and payload in LDS; wave 0 then folds them in
// nearest-first: an inclusive carry ends the walk, an aggregate is absorbed
// and the walk continues, a predecessor with nothing published yet stops the
// round (retried next round).  On return wave 0 holds the carry into the tile.
//
// Monoid policy M: NI inclusive values, NA aggregate values, Acc type with
// identity / absorb (acc <- acc o agg of an earlier tile) / finish (carry =
// acc applied to the inclusive value of that tile), and apply (one published
// aggregate applied to a carry vector).
//
// Deterministic mode (DET): which predecessors a walk composes depends on
// timing, and composing aggregates in a different grouping rounds
// differently.  With det set, a walk only ends on an inclusive carry inside
// the window whose nearer predecessors have all published their aggregates,
// and applies those aggregates to it one at a time, oldest first.  Every tile
// publishes its inclusive carry as M::apply(its published aggregate, its
// carry), so by induction every carry equals the serial chain
// carry_i = apply(agg_{i-1}, carry_{i-1}) bit for bit, whichever predecessor a
// walk happened to stop at.  The price is that the walk never reaches past
// the window: a tile waits until one of its W * KP nearest predecessors holds
// its inclusive carry.
// ---------------------------------------------------------------------------
// Bound on the waits of one launch: a wave that has polled `limit` rounds
// without its predecessors' words arriving gives up -- it ORs 1 into *status
// (a word of the call's workspace, read by prnn_slstm_lookback_status), takes
// NaN for what it waited for, and carries on, so every wave still reaches the
// end of the kernel and the output shows the failure.  Publication order
// guarantees progress, so this only fires on a broken invariant (a stale or
// foreign workspace, a tag mismatch) or an artificially small limit.
struct Spin {
  int* status;
  int limit;
};

__device__ __forceinline__ void spin_give_up(const Spin& spin) {
  __hip_atomic_fetch_or(spin.status, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <class M, int NW>
struct LookbackShared {
  float pl[NW][M::NA][kCB];
  int st[NW][kCB];
  int pos[kCB];
  int more;
};

// W waves, each fetching KP predecessors per round (window NW = W * KP).
template <class M, int W, int KP, bool DET>
__device__ __forceinline__ void windowed_lookback(const TileId& id, int B, int n_cb, int epoch,
                                                  const unsigned long long* __restrict__ incl,
                                                  const unsigned long long* __restrict__ agg,
                                                  int lane, int wave,
                                                  LookbackShared<M, W * KP>& sh,
                                                  float carry[M::NI], const Spin& spin) {
  typename M::Acc acc;
  M::identity(acc);
  int pos = id.chunk - 1;  // wave 0: next predecessor chunk to examine
  bool done = false;
  const int per = B * n_cb;
  int idle_rounds = 0;
  int rounds = 0;
  while (true) {
    if (wave == 0) sh.pos[lane] = done ? -1 : pos;
    __syncthreads();
    {
      const int base = sh.pos[lane];
#pragma unroll
      for (int k = 0; k < KP; ++k) {
        const int slot = wave * KP + k;
        const int p = base - slot;
        int st = 0;
        if (base >= 0 && p >= 0) {
          const size_t ptile = static_cast<size_t>(p) * per + id.rem;
          const unsigned long long* ip = incl + ptile * M::NI * kCB + lane;
          const unsigned long long* ap = agg + ptile * M::NA * kCB + lane;
          // Large aggregates (the 4x4 affine monoid) are fetched only when the
          // inclusive carry is not there yet; small ones in the same round.
          constexpr bool kLazyAgg = M::NA > 2 * M::NI;
          float v[M::NI], a[M::NA];
          bool ok_i = true, ok_a = true;
#pragma unroll
          for (int q = 0; q < M::NI; ++q) ok_i = ld_tagged(ip + q * kCB, epoch, v[q]) && ok_i;
          if constexpr (!kLazyAgg) {
#pragma unroll
            for (int q = 0; q < M::NA; ++q) ok_a = ld_tagged(ap + q * kCB, epoch, a[q]) && ok_a;
          }
          if (ok_i) {
            st = 2;
#pragma unroll
            for (int q = 0; q < M::NI; ++q) sh.pl[slot][q][lane] = v[q];
          } else {
            if constexpr (kLazyAgg) {
#pragma unroll
              for (int q = 0; q < M::NA; ++q)
                ok_a = ld_tagged(ap + q * kCB, epoch, a[q]) && ok_a;
            }
            if (ok_a) {
              st = 1;
#pragma unroll
              for (int q = 0; q < M::NA; ++q) sh.pl[slot][q][lane] = a[q];
            }
          }
        }
        sh.st[slot][lane] = st;
      }
    }
    __syncthreads();
    if (wave == 0) {
      bool progressed = false;
      if constexpr (DET) {
        if (!done) {
          // Nearest inclusive carry with no unpublished predecessor before it.
          int s = -1;
          bool gap = false;
#pragma unroll
          for (int w = 0; w < W * KP; ++w) {
            const int st = sh.st[w][lane];
            if (s < 0 && !gap) {
              if (st == 2)
                s = w;
              else if (st == 0)
                gap = true;
            }
          }
          if (s >= 0) {
            float v[M::NI];
#pragma unroll
            for (int k = 0; k < M::NI; ++k) v[k] = sh.pl[s][k][lane];
#pragma unroll
            for (int w = W * KP - 2; w >= 0; --w) {
              if (w < s) {
                float a[M::NA];
#pragma unroll
                for (int k = 0; k < M::NA; ++k) a[k] = sh.pl[w][k][lane];
                M::apply(a, v);
              }
            }
#pragma unroll
            for (int k = 0; k < M::NI; ++k) carry[k] = v[k];
            done = true;
            progressed = true;
          }
        }
      } else if (!done) {
        bool stalled = false;
#pragma unroll
        for (int w = 0; w < W * KP; ++w) {
          if (!done && !stalled) {
            const int st = sh.st[w][lane];
            if (st == 2) {
              float v[M::NI];
#pragma unroll
              for (int k = 0; k < M::NI; ++k) v[k] = sh.pl[w][k][lane];
              M::finish(acc, v, carry);
              done = true;
              progressed = true;
            } else if (st == 1) {
              float a[M::NA];
#pragma unroll
              for (int k = 0; k < M::NA; ++k) a[k] = sh.pl[w][k][lane];
              M::absorb(acc, a);
              --pos;
              progressed = true;
            } else {
              stalled = true;
            }
          }
        }
      }
      if (++rounds > spin.limit && !done) {
        // give up (see Spin): NaN carry, and report it
#pragma unroll
        for (int k = 0; k < M::NI; ++k) carry[k] = __builtin_nanf("");
        done = true;
        spin_give_up(spin);
      }
      const unsigned long long pending = __ballot(!done);
      const unsigned long long moved = __ballot(progressed);
      if (lane == 0) sh.more = pending != 0ull;
      // Nothing new anywhere: back off before polling again.
      idle_rounds = moved ? 0 : idle_rounds + 1;
      if (pending && !moved) {
        if (idle_rounds > 8)
          __builtin_amdgcn_s_sleep(8);
        else
          __builtin_amdgcn_s_sleep(2);
      }
    }
    __syncthreads();
    if (!sh.more) break;
  }
}

// Cell value and the per-channel Jacobian [out, in] over slots (c, n, m, h):
//   c: [f, 0, cm, ch]   n: [0, f, nm, nh]   m: [0, 0, al, mh]
//   h: inv * (c row) + dn * (n row) + [0, 0, 0, g]
// The h row is kept factorised: h' = o c' / (n' + eps), so its derivative is
// inv = o / den times that of c', plus dn = -o c' / den^2 times that of n',
// plus g = (c' / den) do/dh through the output gate.  Applied to a vector
// that costs 3 operations for the h row instead of 4, and the four dense h
// entries are never formed.
struct CellJ {
  float pc, pn, pm, ph;
  float f, cm, ch, nm, nh, al, mh, inv, dn, g;
};

// The cell's z = tanh(z_z) at this step (it depends only on x and h).
__device__ __forceinline__ float cell_z(const float prev[4], const float x[4], const float r[4]) {
  return ftanh5(x[2] + r[2] * prev[3]);
}

// cell_jac with z = cell_z(prev, x, r) given (GIVEN_Z) or evaluated here.
template <bool GIVEN_Z>
__device__ __forceinline__ CellJ cell_jac_impl(const float prev[4], const float x[4],
                                               const float r[4], float eps, float zg) {
  const float c = prev[0], n = prev[1], m = prev[2], h = prev[3];
  const float zi = x[0] + r[0] * h;
  const float zf = x[1] + r[1] * h;
  const float zz = x[2] + r[2] * h;
  const float zo = x[3] + r[3] * h;
  const float left = zf + m;
  const float mn = fmaxf(left, zi);
  // d max(left, z_i) / d left, ties split 0.5 / 0.5 (para_slstm.py:530-534).
  const float al = left > zi ? 1.f : (left == zi ? 0.5f : 0.f);
  const float e = fexp(-fabsf(left - zi));  // the smaller of the two gate exponents
  const bool lf = left >= zi;
  const float f = lf ? 1.f : e;
  const float i = lf ? e : 1.f;
  const float z = GIVEN_Z ? zg : ftanh5(zz);
  const float nn = f * n + i;
  const float cn = f * c + i * z;
  const float o = fsigmoid(zo);
  const float inv_den = frcp(nn + eps);
  CellJ J;
  J.pc = cn;
  J.pn = nn;
  J.pm = mn;
  J.ph = o * (cn * inv_den);
  // With d = r_f - r_i and the gate split a1 = f (1 - al), a2 = i al (al =
  // d m'/d left), the m- and h-derivatives of the c and n rows share their
  // factors: cm = a1 c - a2 z, nm = a1 n - a2, ch = d cm + i (1 - z^2) r_z,
  // nh = d nm, and mh = r_i + al d.
  const float a1 = f * (1.f - al);
  const float a2 = i * al;
  const float dr = r[1] - r[0];
  const float do_dh = o * (1.f - o) * r[3];
  J.f = f;
  J.al = al;
  J.cm = a1 * c - a2 * z;
  J.nm = a1 * n - a2;
  J.ch = dr * J.cm + i * ((1.f - z * z) * r[2]);
  J.nh = dr * J.nm;
  J.mh = r[0] + al * dr;
  J.inv = o * inv_den;
  J.dn = -J.inv * (cn * inv_den);
  J.g = (cn * inv_den) * do_dh;
  return J;
}

__device__ __forceinline__ CellJ cell_jac(const float prev[4], const float x[4], const float r[4],
                                          float eps) {
  return cell_jac_impl<false>(prev, x, r, eps, 0.f);
}
__device__ __forceinline__ CellJ cell_jac_z(const float prev[4], const float x[4],
                                            const float r[4], float eps, float z) {
  return cell_jac_impl<true>(prev, x, r, eps, z);
}

// Cell value p = f(prev, x) and the directional derivative jv = J v along
// v, without forming J (a forward-mode pass through the cell, about half the
// arithmetic of building the 12 entries and multiplying).
// cell_jvp with z = cell_z(prev, x, r) given (GIVEN_Z) or evaluated here.
template <bool GIVEN_Z>
__device__ __forceinline__ void cell_jvp_impl(const float prev[4], const float x[4],
                                              const float r[4], float eps, float zg,
                                              const float v[4], float p[4], float jv[4]) {
  const float c = prev[0], n = prev[1], m = prev[2], h = prev[3];
  const float zi = x[0] + r[0] * h;
  const float zf = x[1] + r[1] * h;
  const float zz = x[2] + r[2] * h;
  const float zo = x[3] + r[3] * h;
  const float left = zf + m;
  const float mn = fmaxf(left, zi);
  const float al = left > zi ? 1.f : (left == zi ? 0.5f : 0.f);
  const float e = fexp(-fabsf(left - zi));
  const bool lf = left >= zi;
  const float f = lf ? 1.f : e;
  const float i = lf ? e : 1.f;
  const float z = GIVEN_Z ? zg : ftanh5(zz);
  const float nn = f * n + i;
  const float cn = f * c + i * z;
  const float o = fsigmoid(zo);
  const float inv_den = frcp(nn + eps);
  const float u = cn * inv_den;
  p[0] = cn;
  p[1] = nn;
  p[2] = mn;
  p[3] = o * u;
  // tangents: z_g' = r_g h', left' = z_f' + m', m_new' = al left' + (1 - al) z_i';
  // with q = left' - z_i' = m' + (r_f - r_i) h', the gate tangents are
  // f' = f (1 - al) q and i' = -i al q.
  const float q = v[2] + (r[1] - r[0]) * v[3];
  const float dmn = r[0] * v[3] + al * q;
  const float a1 = f * (1.f - al);
  const float a2 = i * al;
  const float dnn = f * v[1] + q * (a1 * n - a2);
  const float dcn = f * v[0] + q * (a1 * c - a2 * z) + i * (1.f - z * z) * (r[2] * v[3]);
  const float dso = o * (1.f - o) * (r[3] * v[3]);
  jv[0] = dcn;
  jv[1] = dnn;
  jv[2] = dmn;
  jv[3] = dso * u + o * inv_den * (dcn - u * dnn);
}

__device__ __forceinline__ void cell_jvp(const float prev[4], const float x[4], const float r[4],
                                         float eps, const float v[4], float p[4], float jv[4]) {
  cell_jvp_impl<false>(prev, x, r, eps, 0.f, v, p, jv);
}
__device__ __forceinline__ void cell_jvp_z(const float prev[4], const float x[4],
                                           const float r[4], float eps, float z, const float v[4],
                                           float p[4], float jv[4]) {
  cell_jvp_impl<true>(prev, x, r, eps, z, v, p, jv);
}

// v <- J v
__device__ __forceinline__ void jmv(const CellJ& J, float v[4]) {
  const float c = v[0], n = v[1], m = v[2], h = v[3];
  v[0] = J.f * c + J.cm * m + J.ch * h;
  v[1] = J.f * n + J.nm * m + J.nh * h;
  v[2] = J.al * m + J.mh * h;
  v[3] = J.inv * v[0] + J.dn * v[1] + J.g * h;
}

// v <- J v + F: the affine step of the Newton scan.
__device__ __forceinline__ void jmv_affine(const CellJ& J, const float F[4], float v[4]) {
  const float c = v[0], n = v[1], m = v[2], h = v[3];
  const float tc = J.f * c + J.cm * m + J.ch * h;
  const float tn = J.f * n + J.nm * m + J.nh * h;
  v[0] = tc + F[0];
  v[1] = tn + F[1];
  v[2] = J.al * m + J.mh * h + F[2];
  v[3] = J.inv * tc + J.dn * tn + J.g * h + F[3];
}

// ---- eager-rounding cell (scan_backend='eager' with 16-bit storage) -------
// The reference's eager Newton step evaluates the cell and its Jacobian as a
// chain of tensor ops in the storage dtype S, each rounding its result to S
// (cells/para_slstm.py:241-281 for the cell, :378-446 for the Jacobian,
// :530-534 for the max subgradient), then scans the S-valued J and residual
// in fp32 (solvers/scan.py:229-246).  CellJE restates that op chain: every
// intermediate is rounded where the eager op rounds it, in the same operand
// order, with no contraction into FMAs.  Transcendentals use the accurate
// library functions: the eager ops round a correctly evaluated fp32 result.
// The h row is dense (hc, hn, hm, hh), as the eager Jacobian forms it.
struct CellJE {
  float pc, pn, pm, ph;                      // f(prev, x), S-valued
  float f, cm, ch, nm, nh, al, mh;           // c, n, m rows
  float hc, hn, hm, hh;                      // h row
};

template <typename S>
__device__ __forceinline__ CellJE cell_jac_eager(const float prev[4], const float x[4],
                                                 const float r[4], float eps) {
#pragma clang fp contract(off)
  auto R = [](float v) { return round_to<S>(v); };
  const float c = prev[0], n = prev[1], m = prev[2], h = prev[3];
  // pre = wx + r * h (two ops)
  const float zi = R(x[0] + R(r[0] * h));
  const float zf = R(x[1] + R(r[1] * h));
  const float zz = R(x[2] + R(r[2] * h));
  const float zo = R(x[3] + R(r[3] * h));
  const float left = R(zf + m);
  const float mn = fmaxf(left, zi);
  const float al = left > zi ? 1.f : (left == zi ? 0.5f : 0.f);
  const float ig = R(expf(R(zi - mn)));
  const float fg = R(expf(R(left - mn)));
  const float z = R(tanhf(zz));
  const float nn = R(R(fg * n) + ig);
  const float cn = R(R(fg * c) + R(ig * z));
  const float o = R(1.f / (1.f + expf(-zo)));
  const float den = R(nn + eps);
  const float u = R(cn / den);
  CellJE J;
  J.pc = cn;
  J.pn = nn;
  J.pm = mn;
  J.ph = R(o * u);
  const float be = 1.f - al;
  const float dm_dh = R(R(al * r[1]) + R(be * r[0]));
  const float di_dm = R(-ig * al);
  const float df_dm = R(fg * be);
  const float di_dh = R(ig * R(r[0] - dm_dh));
  const float df_dh = R(fg * R(r[1] - dm_dh));
  const float dz_dh = R(R(1.f - R(z * z)) * r[2]);
  const float do_dh = R(R(o * R(1.f - o)) * r[3]);
  J.f = fg;
  J.al = al;
  J.mh = dm_dh;
  J.cm = R(R(df_dm * c) + R(di_dm * z));
  J.ch = R(R(R(df_dh * c) + R(di_dh * z)) + R(ig * dz_dh));
  J.nm = R(R(df_dm * n) + di_dm);
  J.nh = R(R(df_dh * n) + di_dh);
  const float inv = R(o / den);
  const float dn = R(R(-o * cn) / R(den * den));
  J.hc = R(inv * fg);
  J.hn = R(dn * fg);
  J.hm = R(R(inv * J.cm) + R(dn * J.nm));
  J.hh = R(R(R(inv * J.ch) + R(dn * J.nh)) + R(u * do_dh));
  return J;
}

// v <- J v + F with the dense h row (fp32, as the eager scan composes).
__device__ __forceinline__ void jmv_affine_e(const CellJE& J, const float F[4], float v[4]) {
  const float c = v[0], n = v[1], m = v[2], h = v[3];
  v[0] = J.f * c + J.cm * m + J.ch * h + F[0];
  v[1] = J.f * n + J.nm * m + J.nh * h + F[1];
  v[2] = J.al * m + J.mh * h + F[2];
  v[3] = J.hc * c + J.hn * n + J.hm * m + J.hh * h + F[3];
}

__device__ __forceinline__ void jmv_e(const CellJE& J, float v[4]) {
  const float zero[4] = {0.f, 0.f, 0.f, 0.f};
  jmv_affine_e(J, zero, v);
}

// 4x4 affine element (A, b): x -> A x + b
struct Aff {
  float A[4][4];
  float b[4];
};

__device__ __forceinline__ void aff_identity(Aff& a) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    a.b[i] = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) a.A[i][j] = i == j ? 1.f : 0.f;
  }
}

// y after x: (Ay Ax, Ay bx + by)
__device__ __forceinline__ Aff aff_compose(const Aff& x, const Aff& y) {
  Aff o;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float acc = y.b[i];
#pragma unroll
    for (int k = 0; k < 4; ++k) acc += y.A[i][k] * x.b[k];
    o.b[i] = acc;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float s = 0.f;
#pragma unroll
      for (int k = 0; k < 4; ++k) s += y.A[i][k] * x.A[k][j];
      o.A[i][j] = s;
    }
  }
  return o;
}

// Aggregate words: A row major (16), then b (4).
__device__ __forceinline__ Aff aff_load(const float a[20]) {
  Aff o;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    o.b[i] = a[16 + i];
#pragma unroll
    for (int j = 0; j < 4; ++j) o.A[i][j] = a[4 * i + j];
  }
  return o;
}

__device__ __forceinline__ void aff_apply(const Aff& a, float v[4]) {
  float o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float acc = a.b[i];
#pragma unroll
    for (int k = 0; k < 4; ++k) acc += a.A[i][k] * v[k];
    o[i] = acc;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = o[i];
}


struct NewtonMonoid {
  static constexpr int NI = 4;   // carry delta (c, n, m, h)
  static constexpr int NA = 20;  // aggregate A (16, row major) then b (4)
  using Acc = Aff;
  static __device__ __forceinline__ void identity(Acc& a) { aff_identity(a); }
  static __device__ __forceinline__ void absorb(Acc& acc, const float v[NA]) {
    Aff pa;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      pa.b[i] = v[16 + i];
#pragma unroll
      for (int j = 0; j < 4; ++j) pa.A[i][j] = v[4 * i + j];
    }
    acc = aff_compose(pa, acc);
  }
  static __device__ __forceinline__ void finish(const Acc& acc, const float v[NI], float out[NI]) {
#pragma unroll
    for (int k = 0; k < 4; ++k) out[k] = v[k];
    aff_apply(acc, out);
  }
  static __device__ __forceinline__ void apply(const float a[NA], float v[NI]) {
    aff_apply(aff_load(a), v);
  }
};

// Raw storage words of a tile's steps, held in registers between the two
// passes: 16-bit values packed two to a register, fp32 values one each.
template <typename T>
struct RowStash {
  static constexpr int N = 2;
  // Slot g of the row at byte offset soff (+ g * slot bytes, wave-uniform).
  static __device__ __forceinline__ void load(rsrc_t rs, uint32_t voff, uint32_t soff,
                                              uint32_t slot, uint32_t w[N]) {
    uint32_t v[4];
#pragma unroll
    for (int g = 0; g < 4; ++g)
      v[g] = __builtin_amdgcn_raw_buffer_load_b16(rs, voff, soff + g * slot, 0);
    w[0] = v[0] | (v[1] << 16);
    w[1] = v[2] | (v[3] << 16);
  }
  static __device__ __forceinline__ void get(const uint32_t w[N], float p[4]) {
    p[0] = Narrow<T>::lo(w[0]);
    p[1] = Narrow<T>::hi(w[0]);
    p[2] = Narrow<T>::lo(w[1]);
    p[3] = Narrow<T>::hi(w[1]);
  }
};

template <>
struct RowStash<float> {
  static constexpr int N = 4;
  static __device__ __forceinline__ void load(rsrc_t rs, uint32_t voff, uint32_t soff,
                                              uint32_t slot, uint32_t w[N]) {
#pragma unroll
    for (int g = 0; g < 4; ++g)
      w[g] = __builtin_amdgcn_raw_buffer_load_b32(rs, voff, soff + g * slot, 0);
  }
  static __device__ __forceinline__ void get(const uint32_t w[N], float p[4]) {
#pragma unroll
    for (int g = 0; g < 4; ++g) p[g] = __uint_as_float(w[g]);
  }
};

}  // namespace slstm
}  // namespace prnn

namespace prnn {
namespace slstm {

constexpr int kMaxStages = PRNN_TAG_SPAN;  // ticket counters (and tags) per call

// Tile shape: L steps per lane x W waves.
struct Shape {
  int L, W;
};

struct Geo {
  int n_cb, n_chunks, n_tiles;
};

static Geo geometry(int B, int T, int d, Shape sh) {
  Geo g;
  g.n_cb = (d + kCB - 1) / kCB;
  g.n_chunks = (T + sh.L * sh.W - 1) / (sh.L * sh.W);
  g.n_tiles = B * g.n_cb * g.n_chunks;
  return g;
}

// bf16 and fp16 storage: 16-bit words, fp32 algebra, the same kernels.
static bool narrow(int dtype) { return dtype != PRNN_F32; }
static size_t elem_size(int dtype) { return narrow(dtype) ? 2 : 4; }
template <typename TX>
constexpr int dtype_code() {
  return sizeof(TX) == 4 ? PRNN_F32 : std::is_same<TX, f16>::value ? PRNN_F16 : PRNN_BF16;
}

static int check_dims(int B, int T, int d, int dtype) {
  if (B < 1 || T < 1 || d < 1)
    return fail(PRNN_ERR_VALUE, "B, T, d must be >= 1, got B=%d T=%d d=%d", B, T, d);
  // A wave addresses its steps with 32-bit buffer offsets.
  if (d >= (1 << 20)) return fail(PRNN_ERR_VALUE, "d must be < 2^20, got %d", d);
  if (check_dtype(dtype) != PRNN_OK) return PRNN_ERR_TYPE;
  const long long tiles = static_cast<long long>(B) * ((d + kCB - 1) / kCB) * T;
  if (tiles > (1ll << 30))
    return fail(PRNN_ERR_VALUE, "problem too large: B*T*ceil(d/64) = %lld", tiles);
  return PRNN_OK;
}

// Look-back state shared by the launches of one call, cleared by one kernel
// at the start of the call:
//   counters[kMaxStages] | tagged carries | tagged aggregates
struct Lookback {
  int* counters;  // kMaxStages ticket counters, then the give-up status word
  unsigned long long* incl;
  unsigned long long* agg;
  size_t clear_words;
  // 0: clear every status word before the call; > 0: the caller vouches that
  // every word holds a tag below tag_base + 1 (zero-filled, or written by an
  // earlier call with a smaller base), so only the ticket counters are
  // cleared and this call's tags start at tag_base + 1.
  int tag_base = 0;
  Spin spin() const { return Spin{counters + kMaxStages, spin_limit()}; }
};

static int check_tag_base(int tag_base) {
  if (tag_base < 0 || tag_base > PRNN_TAG_BASE_MAX)
    return fail(PRNN_ERR_VALUE, "tag_base must be in [0, %d], got %d", PRNN_TAG_BASE_MAX,
                tag_base);
  return PRNN_OK;
}

// Zero what the call's look-back needs zeroed (see Lookback::tag_base).
static int clear_status(const Lookback& lb, hipStream_t stream) {
  return clear_words(lb.counters, lb.tag_base > 0 ? kMaxStages + 1 : lb.clear_words, stream);
}

static Lookback carve_lookback(Carver& cv, const Geo& g, int incl_vals, int agg_vals) {
  Lookback lb;
  lb.counters = static_cast<int*>(cv.take(sizeof(int) * (kMaxStages + 1)));
  lb.incl = static_cast<unsigned long long*>(
      cv.take(sizeof(unsigned long long) * incl_vals * kCB * g.n_tiles));
  lb.agg = static_cast<unsigned long long*>(
      cv.take(sizeof(unsigned long long) * agg_vals * kCB * g.n_tiles));
  lb.clear_words = (cv.used - (reinterpret_cast<char*>(lb.counters) - cv.base)) / sizeof(int);
  return lb;
}

}  // namespace slstm
}  // namespace prnn
