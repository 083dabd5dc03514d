// Eq. 2.6 backward of the ParaSLSTM mix='diag' Newton solve for gfx950.
//
// Given the solved trajectory H* and the upstream gradient g = dL/dH, the
// adjoint mu solves the reverse recursion
//     mu_{T-1} = g_{T-1},   mu_t = g_t + J_{t+1}^T mu_{t+1},
// and the parameter / input gradients are the cell VJP of every step with its
// mu.  One kernel does both: a reverse chunked scan with the same tile
// schedule and decoupled look-back as the forward Newton kernel, with time
// chunks taken from the end, and the cell VJP fused into its second pass.
//
// The carry between segments is nu_t = J_t^T mu_t (so mu_{t-1} = g_{t-1} +
// nu_t and nu_T = 0): a segment [t0, t1) maps nu_{t1} -> nu_{t0} through the
// affine steps nu <- J_t^T (nu + g_t), t = t1-1 ... t0, whose aggregate
// (A, b) composes on the same 4x4 affine monoid as the forward solve.  In
// pass 2, nu_t falls out of the VJP itself: with d_* the adjoints of the
// step's intermediates, nu = (d_c' f, d_n' f, d_zf, sum_g r_g d_zg), and
// nu_0 = J_0^T mu_0 is the gradient of h0.
//
// Outputs: g_wx = d L / d wx (B, T, 4d) in the storage dtype, the per-tile
// partial sums of d_zg * h_{t-1} (reduced by a second kernel into
// g_r (4, d) fp32, before the clamp mask), and g_h0 (B, 4, d) fp32.
//
// Reference: solvers/newton/__init__.py:91-190, 765-866 (eq. 2.6),
// solvers/scan.py:166-178 (reverse block-4 scan), kernels/vjp_slstm.py:173-240
// (cell VJP), solvers/newton/dispatch.py:406-410 (h0 adjoint).
#include "slstm_scan.h"

namespace prnn {
namespace slstm {

// v <- J^T v
__device__ __forceinline__ void jtmv(const CellJ& J, float v[4]) {
  // with the factorised h row, J^T v = J_cn^T w + (0, 0, al m, mh m + g h)
  // where w = (c + inv h, n + dn h) feeds the c and n rows
  const float m = v[2], h = v[3];
  const float wc = v[0] + J.inv * h, wn = v[1] + J.dn * h;
  v[0] = J.f * wc;
  v[1] = J.f * wn;
  v[2] = J.cm * wc + J.nm * wn + J.al * m;
  v[3] = J.ch * wc + J.nh * wn + J.mh * m + J.g * h;
}

// VJP of one step f(prev, x) with adjoint mu: the four pre-activation
// adjoints dz = dL/d(z_i, z_f, z_z, z_o) (= dL/dwx) and nu = J^T mu.
__device__ __forceinline__ void cell_vjp(const float prev[4], const float x[4], const float r[4],
                                         float eps, const float mu[4], float dz[4],
                                         float nu[4]) {
  const float c = prev[0], n = prev[1], m = prev[2], h = prev[3];
  const float zi = x[0] + r[0] * h;
  const float zf = x[1] + r[1] * h;
  const float zz = x[2] + r[2] * h;
  const float zo = x[3] + r[3] * h;
  const float left = zf + m;
  // d max(left, z_i) / d left, ties split 0.5 / 0.5 (para_slstm.py:530-534).
  const float al = left > zi ? 1.f : (left == zi ? 0.5f : 0.f);
  const float e = fexp(-fabsf(left - zi));
  const bool lf = left >= zi;
  const float f = lf ? 1.f : e;
  const float i = lf ? e : 1.f;
  const float z = ftanh5(zz);
  const float nn = f * n + i;
  const float cn = f * c + i * z;
  const float o = fsigmoid(zo);
  const float inv_den = frcp(nn + eps);
  const float t1 = mu[3] * inv_den;
  const float d_o = t1 * cn;
  const float d_cn = mu[0] + t1 * o;
  const float d_nn = mu[1] - t1 * o * cn * inv_den;
  const float d_f = d_cn * c + d_nn * n;
  const float d_i = d_cn * z + d_nn;
  const float d_mn = mu[2] - d_i * i - d_f * f;
  dz[0] = d_i * i + d_mn * (1.f - al);
  dz[1] = d_f * f + d_mn * al;
  dz[2] = d_cn * i * (1.f - z * z);
  dz[3] = d_o * o * (1.f - o);
  nu[0] = d_cn * f;
  nu[1] = d_nn * f;
  nu[2] = dz[1];
  nu[3] = r[0] * dz[0] + r[1] * dz[1] + r[2] * dz[2] + r[3] * dz[3];
}

// Per-tile gradient partials: sum_t dz_g h_{t-1} (R) then sum_t dz_g (bias), g = 0..3.
constexpr int kPartials = 8;

template <typename TX, int L, int W, bool DET, bool PK>
__global__ __launch_bounds__(64 * W) void slstm_reverse_kernel(
    const TX* __restrict__ wx, const TX* __restrict__ rmix, const TX* __restrict__ h0,
    const TX* __restrict__ states, const TX* __restrict__ grad, TX* __restrict__ gwx,
    float* __restrict__ gr_part, float* __restrict__ gh0, int B, int T, int d, int n_cb,
    int n_chunks, float eps, int* __restrict__ counter, unsigned long long* __restrict__ agg,
    unsigned long long* __restrict__ incl, int epoch, Spin spin, Packed pk) {
  // predecessors per wave per look-back round (the deterministic walk, which
  // must find an inclusive carry inside its window, looks twice as far)
  constexpr int KP = DET ? 2 : 1;
  using RS = RowStash<TX>;
  constexpr uint32_t SZ = sizeof(TX);
  __shared__ float s_agg[W][20][kCB];
  __shared__ float s_carry[W][4][kCB];
  __shared__ float s_tagg[20][kCB];  // the published tile aggregate (wave 0's lanes)
  __shared__ LookbackShared<NewtonMonoid, W * KP> s_lb;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int tile = take_ticket(counter);
  const TileId id = decode_tile(tile, B, n_cb);  // id.chunk counts from the end of time
  const int tc = n_chunks - 1 - id.chunk;
  const int c0 = id.cb * kCB;
  const bool live = c0 + lane < d;
  const int t0 = tc * (W * L) + wave * L;
  const int n_steps = max(0, min(L, T - t0));
  const size_t row4 = static_cast<size_t>(4) * d;
  const size_t first = static_cast<size_t>(id.b) * T + t0;
  const uint32_t voff = live ? lane * SZ : kOOB;
  const uint32_t slot = d * SZ;
  const uint32_t span = n_steps > 0 ? ((n_steps - 1) * row4 + 3 * d + (d - c0)) * SZ : 0;

  float r[4] = {0.f, 0.f, 0.f, 0.f};
  float prev0[4] = {0.f, 0.f, 0.f, 0.f};  // H*_{t0-1}: states, h0 at t = 0, else zeros
  if (live) {
#pragma unroll
    for (int g = 0; g < 4; ++g) r[g] = ld(rmix + g * d + c0 + lane);
    if (t0 > 0 && n_steps > 0) {
      const TX* p = states + (first - 1) * row4 + c0 + lane;
#pragma unroll
      for (int k = 0; k < 4; ++k) prev0[k] = ld(p + k * d);
    } else if (t0 == 0 && h0 != nullptr) {
      const TX* p = h0 + static_cast<size_t>(id.b) * row4 + c0 + lane;
#pragma unroll
      for (int k = 0; k < 4; ++k) prev0[k] = ld(p + k * d);
    }
  }

  // Registers: H*_{t-1} (step s >= 1; step 0 uses prev0), wx_t and g_t.
  uint32_t hs[L][RS::N], xs[L][RS::N], gs[L][RS::N];
  const rsrc_t rh = make_rsrc(states + first * row4 + c0, span);
  const rsrc_t rx = make_rsrc(wx + first * row4 + c0, span);
  const rsrc_t rg = make_rsrc(grad + first * row4 + c0, span);
  // Packed sequences (see Packed): a head's previous state is its sequence's
  // h0 row; nothing flows from a head to the step before it (nu = 0 there),
  // and the head's nu = J^T mu is that sequence's dL/dh0.
  Heads hd{0ull, 0};
  int ns = n_steps;
  if constexpr (PK) {
    hd = find_heads(pk, t0, n_steps);
    // The head flags and the step count pass through an opaque copy: what the
    // steps derive from them is computed where it is used, not hoisted out of
    // the unrolled loops into scalar registers for all L steps.
    uint32_t lo = static_cast<uint32_t>(hd.mask), hi = static_cast<uint32_t>(hd.mask >> 32);
    int q0 = hd.seq0;
    asm volatile("" : "+v"(lo), "+v"(hi), "+v"(q0), "+v"(ns));
    hd.mask = (static_cast<uint64_t>(__builtin_amdgcn_readfirstlane(hi)) << 32) |
              __builtin_amdgcn_readfirstlane(lo);
    hd.seq0 = __builtin_amdgcn_readfirstlane(q0);
    ns = __builtin_amdgcn_readfirstlane(ns);
  }
  auto prev_of = [&](int s, float p[4]) {
    if (PK && hd.at(s)) {
      head_state(pk, h0, hd.seq(s), d, c0 + lane, live, p);
    } else if (s == 0) {
#pragma unroll
      for (int k = 0; k < 4; ++k) p[k] = prev0[k];
    } else {
      RS::get(hs[s], p);
    }
  };

  // Pass 1: the segment's map nu_{t1} -> nu_{t0}, steps from the last down.
  Aff a;
  aff_identity(a);
  {
    auto step = [&](int s, auto chk) {
      constexpr bool CHECK = decltype(chk)::value;
      const uint32_t so = s * row4 * SZ;
      RS::load(rx, voff, so, slot, xs[s]);
      RS::load(rg, voff, so, slot, gs[s]);
      if (s > 0) RS::load(rh, voff, so - row4 * SZ, slot, hs[s]);
      float prev[4], x[4], g[4];
      prev_of(s, prev);
      RS::get(xs[s], x);
      RS::get(gs[s], g);
      const CellJ J = cell_jac(prev, x, r, eps);
      float v[4] = {a.b[0] + g[0], a.b[1] + g[1], a.b[2] + g[2], a.b[3] + g[3]};
      jtmv(J, v);
#pragma unroll
      for (int k = 0; k < 4; ++k) a.b[k] = v[k];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float col[4] = {a.A[0][j], a.A[1][j], a.A[2][j], a.A[3][j]};
        jtmv(J, col);
#pragma unroll
        for (int k = 0; k < 4; ++k) a.A[k][j] = col[k];
      }
      if (CHECK && hd.at(s)) {
        // a head: nothing reaches the steps before it
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          a.b[i] = 0.f;
#pragma unroll
          for (int j = 0; j < 4; ++j) a.A[i][j] = 0.f;
        }
      }
    };
    // Packed streams: one head-checked copy of the loop (steps past the end
    // of the stream stay guarded: this scan composes from the last step
    // down, so they would come first).
    auto run = [&](auto chk) {
      if (!PK && n_steps == L) {
#pragma unroll
        for (int s = L - 1; s >= 0; --s) step(s, chk);
      } else {
#pragma unroll
        for (int s = L - 1; s >= 0; --s)
          if (s < ns) step(s, chk);
      }
    };
    // a wave whose steps hold no head skips the per-step checks here (pass 2
    // keeps the one checked copy)
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
  __syncthreads();

  auto wave_map = [&](int w, Aff& sw) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      sw.b[i] = s_agg[w][16 + i][lane];
#pragma unroll
      for (int j = 0; j < 4; ++j) sw.A[i][j] = s_agg[w][4 * i + j][lane];
    }
  };
  float carry[4] = {0.f, 0.f, 0.f, 0.f};  // nu entering the tile from later time (0 at T)
  if (wave == 0 && id.chunk > 0) {
    // Scan order inside the tile runs from the last wave to the first.
    Aff tile_agg;
    wave_map(W - 1, tile_agg);
#pragma unroll
    for (int w = W - 2; w >= 0; --w) {
      Aff sw;
      wave_map(w, sw);
      tile_agg = aff_compose(tile_agg, sw);
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
    // Per-wave carries; the outgoing carry is the published aggregate applied
    // to the carry in, as a successor's walk would compute it.
#pragma unroll
    for (int w = W - 1; w >= 0; --w) {
#pragma unroll
      for (int k = 0; k < 4; ++k) s_carry[w][k][lane] = carry[k];
      Aff sw;
      wave_map(w, sw);
      aff_apply(sw, carry);
    }
    if (DET && id.chunk > 0) {
      float a[20];
#pragma unroll
      for (int k = 0; k < 20; ++k) a[k] = s_tagg[k][lane];
#pragma unroll
      for (int k = 0; k < 4; ++k) carry[k] = s_carry[W - 1][k][lane];
      NewtonMonoid::apply(a, carry);
    }
    unsigned long long* ip = incl + (static_cast<size_t>(tile) * 4) * kCB + lane;
#pragma unroll
    for (int k = 0; k < 4; ++k) st_tagged(ip + k * kCB, carry[k], epoch);
  }
  __syncthreads();

  // Pass 2: mu_t = g_t + nu_{t+1}, the cell VJP of step t, nu_t = J_t^T mu_t.
  float nu[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) nu[k] = s_carry[wave][k][lane];
  float gr[4] = {0.f, 0.f, 0.f, 0.f};
  float gb[4] = {0.f, 0.f, 0.f, 0.f};  // sum_t dz_g: the W_x bias gradient
  {
    const rsrc_t ro = make_rsrc(gwx + first * row4 + c0, span);
    auto replay = [&](int s, auto chk) {
      constexpr bool CHECK = decltype(chk)::value;
      float prev[4], x[4], g[4], mu[4], dz[4];
      prev_of(s, prev);
      RS::get(xs[s], x);
      RS::get(gs[s], g);
#pragma unroll
      for (int k = 0; k < 4; ++k) mu[k] = g[k] + nu[k];
      cell_vjp(prev, x, r, eps, mu, dz, nu);
      const uint32_t so = s * row4 * SZ;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        stb<TX>(ro, voff, so + k * slot, dz[k]);
        gr[k] += dz[k] * prev[3];
        gb[k] += dz[k];
      }
      if (CHECK && hd.at(s)) {
        // a head: nu is its sequence's dL/dh0, and nothing flows further back
        if (gh0 != nullptr && live) {
          float* p = gh0 + static_cast<size_t>(hd.seq(s)) * row4 + c0 + lane;
#pragma unroll
          for (int k = 0; k < 4; ++k) p[k * d] = nu[k];
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) nu[k] = 0.f;
      }
    };
    auto run = [&](auto chk) {
      if (!PK && n_steps == L) {
#pragma unroll
        for (int s = L - 1; s >= 0; --s) replay(s, chk);
      } else {
#pragma unroll
        for (int s = L - 1; s >= 0; --s)
          if (s < ns) replay(s, chk);
      }
    };
    if constexpr (PK)
      run(std::true_type{});
    else
      run(std::false_type{});
  }
  if (!PK && gh0 != nullptr && t0 == 0 && live) {
    float* p = gh0 + static_cast<size_t>(id.b) * row4 + c0 + lane;
#pragma unroll
    for (int k = 0; k < 4; ++k) p[k * d] = nu[k];
  }
  // Tile partials of sum_t dz_g * h_{t-1} (R) and sum_t dz_g (bias): waves
  // through LDS (s_agg is free).
  __syncthreads();
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    s_agg[wave][k][lane] = gr[k];
    s_agg[wave][4 + k][lane] = gb[k];
  }
  __syncthreads();
  if (wave == 0) {
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      float acc = 0.f;
#pragma unroll
      for (int w = 0; w < W; ++w) acc += s_agg[w][k][lane];
      gr_part[(static_cast<size_t>(tile) * kPartials + k) * kCB + lane] = acc;
    }
  }
}

// g_r[g][ch] = sum over the tiles of ch's (b, channel block) of the partials.
// One block per (gate, channel block): lane = channel, each of the 16 waves
// sums a fixed share of the tiles (coalesced 256-byte rows), then the
// shares combine in LDS in a fixed order (deterministic).
constexpr int kReduceWaves = 16;
__global__ __launch_bounds__(64 * kReduceWaves) void slstm_gr_reduce_kernel(
    const float* __restrict__ gr_part, float* __restrict__ gr, float* __restrict__ gb, int B,
    int d, int n_cb, int n_chunks) {
  __shared__ float s_part[kReduceWaves][kCB];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int g = blockIdx.x / n_cb, cb = blockIdx.x - g * n_cb;
  const int per_cb = n_chunks * B;  // tiles of this channel block
  const int q0 = static_cast<int>(static_cast<long long>(per_cb) * wave / kReduceWaves);
  const int q1 = static_cast<int>(static_cast<long long>(per_cb) * (wave + 1) / kReduceWaves);
  float acc = 0.f;
  for (int q = q0; q < q1; ++q) {
    // q enumerates (chunk, b) in tile order
    const size_t tile = static_cast<size_t>(q) * n_cb + cb;
    acc += gr_part[(tile * kPartials + g) * kCB + lane];
  }
  s_part[wave][lane] = acc;
  __syncthreads();
  if (wave == 0) {
    float t = 0.f;
#pragma unroll
    for (int w = 0; w < kReduceWaves; ++w) t += s_part[w][lane];
    const int ch = cb * kCB + lane;
    if (ch < d) {
      if (g < 4)
        gr[g * d + ch] = t;
      else
        gb[(g - 4) * d + ch] = t;
    }
  }
}

}  // namespace slstm
}  // namespace prnn

// ===========================================================================
// Host entry points
// ===========================================================================
namespace prnn {
namespace slstm {

// Backward tiles stash H*_{t-1}, wx and g: 6 registers per step in bf16,
// 12 in fp32.  PRNN_SLSTM_BWD_TILES="<L>x<W>" overrides the bf16 shape for
// tuning runs (instantiated shapes only); deterministic mode always runs the
// default shape.
static const Shape kBwdShapes[] = {{24, 4}, {16, 8}, {16, 4}, {32, 4}};
constexpr Shape kBwdDefault{24, 4};
constexpr Shape kBwdF32{8, 8};

static Shape bwd_shape(int dtype) {
  static Shape s = [] {
    Shape r = kBwdDefault;
    if (const char* e = getenv("PRNN_SLSTM_BWD_TILES")) {
      int l, w;
      if (sscanf(e, "%dx%d", &l, &w) == 2)
        for (const Shape& c : kBwdShapes)
          if (c.L == l && c.W == w) r = c;
    }
    return r;
  }();
  if (!narrow(dtype)) return kBwdF32;
  // fp16 storage is compiled in the default shape only
  return deterministic() || dtype == PRNN_F16 ? kBwdDefault : s;
}

struct BwdWs {
  Lookback lb;
  float* gr_part;
};

static BwdWs carve_bwd(void* base, int B, int T, int d, int dtype, size_t* total) {
  // the packed launch takes the default shape: size for both
  Geo g = geometry(B, T, d, bwd_shape(dtype));
  const Geo gd = geometry(B, T, d, narrow(dtype) ? kBwdDefault : kBwdF32);
  if (gd.n_tiles > g.n_tiles) g = gd;
  Carver cv(base);
  BwdWs w;
  w.lb = carve_lookback(cv, g, 4, 20);
  w.gr_part = static_cast<float*>(cv.take(sizeof(float) * kPartials * kCB * g.n_tiles));
  *total = cv.used;
  return w;
}

template <typename TX, int L, int W, bool DET, bool PK = false>
static void launch_reverse(const TX* wx, const TX* r, const TX* h0, const TX* states,
                           const TX* grad, TX* gwx, float* gh0, int B, int T, int d, float eps,
                           const BwdWs& w, hipStream_t stream,
                           const Packed& pk = Packed{nullptr, nullptr, 0}) {
  const Geo g = geometry(B, T, d, Shape{L, W});
  slstm_reverse_kernel<TX, L, W, DET, PK><<<dim3(g.n_tiles), dim3(64 * W), 0, stream>>>(
      wx, r, h0, states, grad, gwx, w.gr_part, gh0, B, T, d, g.n_cb, g.n_chunks, eps,
      w.lb.counters + 1, w.lb.agg, w.lb.incl, w.lb.tag_base + 1, w.lb.spin(), pk);
}

template <typename TX>
static int run_bwd(const TX* wx, const TX* r, const TX* h0, const TX* states, const TX* grad,
                   TX* gwx, float* gr, float* gh0, float* gb, int B, int T, int d, float eps,
                   const BwdWs& w, hipStream_t stream, const Packed& pk) {
  int rc = clear_status(w.lb, stream);
  if (rc != PRNN_OK) return rc;
  timing_begin(stream);
  Shape sh;
  if (pk.cu != nullptr) {
    // packed stream: default shapes
    constexpr Shape dsh = sizeof(TX) == 4 ? kBwdF32 : kBwdDefault;
    sh = dsh;
    if (deterministic())
      launch_reverse<TX, dsh.L, dsh.W, true, true>(wx, r, h0, states, grad, gwx, gh0, B, T, d,
                                                   eps, w, stream, pk);
    else
      launch_reverse<TX, dsh.L, dsh.W, false, true>(wx, r, h0, states, grad, gwx, gh0, B, T, d,
                                                    eps, w, stream, pk);
  } else if constexpr (sizeof(TX) == 4) {
#define PRNN_LAUNCH(LL, WW, DD) \
  launch_reverse<TX, LL, WW, DD>(wx, r, h0, states, grad, gwx, gh0, B, T, d, eps, w, stream)
    sh = kBwdF32;
    if (deterministic())
      PRNN_LAUNCH(kBwdF32.L, kBwdF32.W, true);
    else
      PRNN_LAUNCH(kBwdF32.L, kBwdF32.W, false);
  } else {
    sh = bwd_shape(dtype_code<TX>());
#define PRNN_SHAPE(LL, WW) \
  else if (sh.L == LL && sh.W == WW) PRNN_LAUNCH(LL, WW, false);
    if (deterministic()) PRNN_LAUNCH(kBwdDefault.L, kBwdDefault.W, true);
    else if constexpr (std::is_same<TX, f16>::value) PRNN_LAUNCH(kBwdDefault.L, kBwdDefault.W, false);
    PRNN_SHAPE(16, 8)
    PRNN_SHAPE(16, 4)
    PRNN_SHAPE(24, 4)
    PRNN_SHAPE(32, 4)
#undef PRNN_SHAPE
  }
#undef PRNN_LAUNCH
  timing_end(stream);
  PRNN_HIP(hipGetLastError());
  const Geo g = geometry(B, T, d, sh);
  // g_r, and g_b when asked for (blocks 4 n_cb .. 8 n_cb)
  slstm_gr_reduce_kernel<<<dim3((gb != nullptr ? 8 : 4) * g.n_cb), dim3(64 * kReduceWaves), 0,
                           stream>>>(w.gr_part, gr, gb, B, d, g.n_cb, g.n_chunks);
  PRNN_HIP(hipGetLastError());
  return PRNN_OK;
}

}  // namespace slstm
}  // namespace prnn

using namespace prnn;

extern "C" PRNN_API size_t prnn_slstm_backward_workspace_size(int B, int T, int d, int dtype) {
  if (slstm::check_dims(B, T, d, dtype) != PRNN_OK) return 0;
  size_t total = 0;
  slstm::carve_bwd(nullptr, B, T, d, dtype, &total);
  return total;
}

namespace {

int backward_call(const void* wx, const void* r, const void* h0, const void* states,
                  const void* grad, void* gwx, float* gr, float* gh0, float* gb, int B, int T,
                  int d, float eps, int dtype, void* workspace, size_t workspace_bytes,
                  int tag_base, void* stream, const slstm::Packed& pk) {
  int rc = slstm::check_dims(B, T, d, dtype);
  if (rc != PRNN_OK) return rc;
  rc = slstm::check_tag_base(tag_base);
  if (rc != PRNN_OK) return rc;
  if (pk.cu != nullptr && B != 1)
    return fail(PRNN_ERR_VALUE, "a packed stream has B = 1, got B = %d", B);
  if (pk.cu != nullptr && (pk.n_seq < 1 || pk.n_seq > T))
    return fail(PRNN_ERR_VALUE, "n_seq must be in [1, T], got %d (T = %d)", pk.n_seq, T);
  if (!wx || !r || !states || !grad || !gwx || !gr || !workspace)
    return fail(PRNN_ERR_VALUE, "wx, r, states, grad, g_wx, g_r and workspace must be non-null");
  size_t need = 0;
  slstm::BwdWs w = slstm::carve_bwd(workspace, B, T, d, dtype, &need);
  if (workspace_bytes < need)
    return fail(PRNN_ERR_VALUE, "workspace too small: %zu < %zu bytes", workspace_bytes, need);
  w.lb.tag_base = tag_base;
  hipStream_t s = static_cast<hipStream_t>(stream);
  return with_storage(dtype, [&](auto tag) {
    using TX = decltype(tag);
    return slstm::run_bwd(static_cast<const TX*>(wx), static_cast<const TX*>(r),
                          static_cast<const TX*>(h0), static_cast<const TX*>(states),
                          static_cast<const TX*>(grad), static_cast<TX*>(gwx), gr, gh0, gb, B, T,
                          d, eps, w, s, pk);
  });
}

}  // namespace

extern "C" PRNN_API int prnn_slstm_backward_ex(const void* wx, const void* r, const void* h0,
                                               const void* states, const void* grad, void* gwx,
                                               float* gr, float* gh0, float* gb, int B, int T,
                                               int d,
                                               float eps, int dtype, void* workspace,
                                               size_t workspace_bytes, int tag_base,
                                               void* stream) {
  return backward_call(wx, r, h0, states, grad, gwx, gr, gh0, gb, B, T, d, eps, dtype, workspace,
                       workspace_bytes, tag_base, stream, slstm::Packed{nullptr, nullptr, 0});
}

extern "C" PRNN_API int prnn_slstm_backward_packed(const void* wx, const void* r,
                                                   const void* h0, const void* states,
                                                   const void* grad, void* gwx, float* gr,
                                                   float* gh0, float* gb, int T, int d,
                                                   float eps, int dtype, const int* cu_seqlens,
                                                   int n_seq, void* workspace,
                                                   size_t workspace_bytes, int tag_base,
                                                   void* stream) {
  if (!cu_seqlens) return fail(PRNN_ERR_VALUE, "cu_seqlens must be non-null");
  return backward_call(wx, r, h0, states, grad, gwx, gr, gh0, gb, 1, T, d, eps, dtype, workspace,
                       workspace_bytes, tag_base, stream,
                       slstm::Packed{cu_seqlens, nullptr, n_seq});
}

extern "C" PRNN_API int prnn_slstm_backward(const void* wx, const void* r, const void* h0,
                                            const void* states, const void* grad, void* gwx,
                                            float* gr, float* gh0, int B, int T, int d, float eps,
                                            int dtype, void* workspace, size_t workspace_bytes,
                                            void* stream) {
  return prnn_slstm_backward_ex(wx, r, h0, states, grad, gwx, gr, gh0, nullptr, B, T, d, eps, dtype,
                                workspace, workspace_bytes, 0, stream);
}
